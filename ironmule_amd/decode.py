"""One decode step of a Qwen3-style decoder whose projections are 4-bit qmv on MI355X.

Mirrors the reference's decode composition (ironmule/dense_plan.py:351-383,
`DensePlan.forward`; ironmule/dense_cpu.py:188-220, `CpuDensePlan.forward`) over B
continuous-batched requests, each with its own KV slot and position:

    h = embed(tokens)                          imq_embed (fp32 residual stream)
    per layer:
        x = rms_norm(h)                        imq_add_rmsnorm (adds the previous delta)
        q, k, v = x @ W.T                      imq_qmv_grouped (one launch, three weights)
        q, k = rope(norm(q)), rope(norm(k))    imq_qk_norm_rope (+ the KV write)
        o = attention(q, KV[slot][:pos+1])     imq_attention_decode
        h += o @ Wo.T                          imq_qmv, added by the next imq_add_rmsnorm
        x = rms_norm(h)
        g, u = x @ Wg.T, x @ Wu.T              imq_qmv_grouped
        h += (silu(g) * u) @ Wd.T              imq_silu_mul, imq_qmv
    logits = rms_norm(h) @ E.T                 imq_add_rmsnorm, imq_qmv (fp32, tied head)

All buffers are allocated once per (model, batch size) in `DecodeState`; a step only
launches kernels, so it can be captured in a HIP graph and replayed.  Every launch goes
through the C ABI; there is no host fallback.

`PersistentDecode` runs the same step at batch 1 as one persistent-kernel program
(include/ironmule_step.h): the embedding launch, then one launch for all layers and the
head, with bit-identical results.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch

from . import _native


@dataclass(frozen=True)
class DecoderConfig:
    """Shapes of a Qwen3-style decoder (defaults: Qwen3-4B)."""
    hidden: int = 2560
    layers: int = 36
    heads: int = 32
    kv_heads: int = 8
    head_dim: int = 128
    intermediate: int = 9728
    vocab: int = 151936
    eps: float = 1e-6
    theta: float = 1_000_000.0

    @property
    def projections(self) -> dict[str, tuple[int, int]]:
        """(out_features, in_features) of each 4-bit projection of a layer."""
        d, h = self.hidden, self.head_dim
        return {"q": (self.heads * h, d), "k": (self.kv_heads * h, d), "v": (self.kv_heads * h, d),
                "o": (d, self.heads * h), "gate": (self.intermediate, d),
                "up": (self.intermediate, d), "down": (d, self.intermediate)}

    def weight_bytes(self) -> int:
        """Packed weights + bf16 scales and biases of every projection and the head."""
        def qbytes(n, k):
            return n * k // 2 + n * (k // 64) * 4
        layer = sum(qbytes(n, k) for n, k in self.projections.values())
        return self.layers * layer + qbytes(self.vocab, self.hidden)


Quant = tuple  # (w int32 (N, K/8), scales bf16 (N, K/64), biases bf16 (N, K/64))


@dataclass
class DecoderWeights:
    """4-bit projections per layer, bf16 norm weights, the tied 4-bit embedding/head."""
    config: DecoderConfig
    layers: list = field(default_factory=list)  # dict name -> Quant, plus norm weights
    embed: Quant = None
    norm: torch.Tensor = None


def random_weights(config: DecoderConfig, device, seed: int = 0) -> DecoderWeights:
    """Seeded synthetic weights: uniform 4-bit words, scales U(0.005, 0.02), biases
    U(-0.1, 0.1), norm weights U(0.9, 1.1) (bf16)."""
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)

    def quant(n, k):
        w = torch.randint(0, 2**32, (n, k // 8), dtype=torch.int64, device=device,
                          generator=gen).to(torch.int32)
        s = torch.empty((n, k // 64), device=device).uniform_(0.005, 0.02, generator=gen)
        b = torch.empty((n, k // 64), device=device).uniform_(-0.1, 0.1, generator=gen)
        return w, s.to(torch.bfloat16), b.to(torch.bfloat16)

    def norm(n):
        return torch.empty(n, device=device).uniform_(0.9, 1.1, generator=gen).to(torch.bfloat16)

    weights = DecoderWeights(config)
    for _ in range(config.layers):
        layer = {name: quant(n, k) for name, (n, k) in config.projections.items()}
        layer.update(input_norm=norm(config.hidden), post_norm=norm(config.hidden),
                     q_norm=norm(config.head_dim), k_norm=norm(config.head_dim))
        weights.layers.append(layer)
    weights.embed = quant(config.vocab, config.hidden)
    weights.norm = norm(config.hidden)
    return weights


class DecodeState:
    """KV pools and every activation buffer of a decode step for `batch` rows.

    The pools are (slots, kv_heads, capacity, 128) bf16 per layer, the reference's pool
    layout (ironmule/dense_plan.py:294-299).  `max_len` bounds the lengths a step may
    attend over (it sizes the attention workspace and grid)."""

    def __init__(self, config: DecoderConfig, batch: int, slots: int, capacity: int,
                 max_len: int, device) -> None:
        if not 1 <= batch <= _native.MAX_ROWS:
            raise ValueError(f"batch must be 1..{_native.MAX_ROWS}")
        c = config
        self.config, self.batch, self.slots, self.capacity = c, batch, slots, capacity
        self.max_len = min(max_len, capacity)
        bf = dict(dtype=torch.bfloat16, device=device)
        self.k_pool = [torch.zeros((slots, c.kv_heads, capacity, c.head_dim), **bf)
                       for _ in range(c.layers)]
        self.v_pool = [torch.zeros((slots, c.kv_heads, capacity, c.head_dim), **bf)
                       for _ in range(c.layers)]
        self.h = torch.zeros((batch, c.hidden), dtype=torch.float32, device=device)
        self.x = torch.empty((batch, c.hidden), **bf)
        self.q = torch.empty((batch, c.heads * c.head_dim), **bf)
        self.k = torch.empty((batch, c.kv_heads * c.head_dim), **bf)
        self.v = torch.empty((batch, c.kv_heads * c.head_dim), **bf)
        self.q_rot = torch.empty((batch, c.heads * c.head_dim), **bf)
        self.attn = torch.empty((batch, c.heads * c.head_dim), **bf)
        self.delta = torch.empty((batch, c.hidden), **bf)
        self.gate = torch.empty((batch, c.intermediate), **bf)
        self.up = torch.empty((batch, c.intermediate), **bf)
        self.act = torch.empty((batch, c.intermediate), **bf)
        self.logits = torch.empty((batch, c.vocab), dtype=torch.float32, device=device)
        self.workspace = torch.empty(_native.attention_workspace(batch, c.heads, self.max_len),
                                     dtype=torch.float32, device=device)
        self.attn_counters = torch.zeros(batch * c.kv_heads, dtype=torch.int32, device=device)
        self.tokens = torch.zeros(batch, dtype=torch.int32, device=device)
        self.slot_ids = torch.arange(batch, dtype=torch.int32, device=device) % slots
        self.positions = torch.zeros(batch, dtype=torch.int32, device=device)
        self.lengths = torch.ones(batch, dtype=torch.int32, device=device)

    def set_requests(self, tokens, slots, positions) -> None:
        """Copy this step's tokens, slots and positions into the device buffers."""
        self.tokens.copy_(torch.as_tensor(tokens, dtype=torch.int32))
        self.slot_ids.copy_(torch.as_tensor(slots, dtype=torch.int32))
        pos = torch.as_tensor(positions, dtype=torch.int32)
        if int(pos.max()) >= self.max_len or int(pos.min()) < 0:
            raise ValueError(f"positions must lie in [0, {self.max_len})")
        self.positions.copy_(pos)
        self.lengths.copy_(pos + 1)


def decode_step(weights: DecoderWeights, state: DecodeState, stream=None) -> torch.Tensor:
    """Launches one decode step for the requests in `state` (tokens, slots, positions set
    by `set_requests`); returns state.logits (B, vocab) fp32, written on `stream`."""
    c, s = weights.config, state
    n = _native
    n.embed(*weights.embed, s.tokens, s.h, stream=stream)
    delta = None
    for i, layer in enumerate(weights.layers):
        n.add_rmsnorm(s.h, layer["input_norm"], s.x, c.eps, delta=delta, stream=stream)
        n.qmv_grouped([layer["q"], layer["k"], layer["v"]], [s.x, s.x, s.x],
                      outs=[s.q, s.k, s.v], stream=stream)
        if s.batch == 1:  # one launch (the decode programs' attention stage, same bits)
            n.attention_fused(s.q, s.k, s.v, layer["q_norm"], layer["k_norm"], s.positions,
                              s.slot_ids, s.k_pool[i], s.v_pool[i], s.attn, s.max_len, c.theta,
                              c.eps, s.workspace, s.attn_counters, stream=stream)
        else:  # three launches: measured faster than the fused form at batch 32
            n.qk_norm_rope(s.q, s.k, s.v, layer["q_norm"], layer["k_norm"], s.positions,
                           s.slot_ids, s.q_rot, s.k_pool[i], s.v_pool[i], c.theta, c.eps,
                           stream=stream)
            n.attention_decode(s.q_rot, s.k_pool[i], s.v_pool[i], s.lengths, s.slot_ids, s.attn,
                               s.max_len, c.head_dim ** -0.5, s.workspace, stream=stream)
        n.qmv(*layer["o"], s.attn, out=s.delta, stream=stream)
        n.add_rmsnorm(s.h, layer["post_norm"], s.x, c.eps, delta=s.delta, stream=stream)
        n.qmv_grouped([layer["gate"], layer["up"]], [s.x, s.x], outs=[s.gate, s.up], stream=stream)
        n.silu_mul(s.gate, s.up, s.act, stream=stream)
        n.qmv(*layer["down"], s.act, out=s.delta, stream=stream)
        delta = s.delta
    n.add_rmsnorm(s.h, weights.norm, s.x, c.eps, delta=delta, stream=stream)
    n.qmv(*weights.embed, s.x, out=s.logits, stream=stream)
    return s.logits


class PersistentDecode:
    """The batch-1 decode step as a program of fused stages (imq_decode_program_create):
    `step()` launches the embedding and the program and returns state.logits.  With
    `staged` each stage is its own launch (5 per layer: q/k/v with the RMSNorm, attention
    with q/k norm + rotary + KV write + the split merge, o with the residual add, gate/up
    with the RMSNorm and SiLU * up, down with the residual add); otherwise one persistent
    launch runs them all.  Same inputs, same bits as `decode_step`."""

    def __init__(self, weights: DecoderWeights, state: DecodeState, staged: bool = False) -> None:
        if state.batch != 1:
            raise ValueError("the persistent decode step runs batch 1")
        self.weights, self.state, self.staged = weights, state, staged
        self.program = _native.decode_program(
            weights.config, weights.layers, weights.norm, weights.embed, state.k_pool,
            state.v_pool, state.positions, state.slot_ids, state.h, state.logits, state.max_len)

    def step(self, stream=None) -> torch.Tensor:
        w, s = self.weights, self.state
        _native.embed(*w.embed, s.tokens, s.h, stream=stream)
        self.program.launch(stream, staged=self.staged)
        return s.logits

    def failed(self) -> bool:
        return self.program.failed()
