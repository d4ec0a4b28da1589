"""One decode step of a Qwen3-style decoder whose projections are 4-bit qmv on MI355X.

Mirrors the reference's decode composition (ironmule/dense_plan.py:337-363,
`DensePlan.forward`; ironmule/dense_cpu.py:188-220, `CpuDensePlan.forward`) over B
continuous-batched requests, each with its own KV slot and position:

    h = embed(tokens)                          imq_embed (fp32 residual stream)
    per layer:
        x = rms_norm(h)                        imq_add_rmsnorm (adds the previous delta)
        q, k, v = x @ W.T                      imq_qmv_grouped (one launch, three weights)
        q, k = rope(norm(q)), rope(norm(k))    imq_attention_fused: one launch for the q/k
        o = attention(q, KV[slot][:pos+1])     norm + rotary, the KV write and the attention
                                               (the pools of imq_qk_norm_rope followed by
                                               imq_attention_decode)
        h += o @ Wo.T                          imq_qmv, added by the next imq_add_rmsnorm
        x = rms_norm(h)
        g, u = x @ Wg.T, x @ Wu.T              imq_qmv_grouped + imq_silu_mul; imq_qmv
        h += (silu(g) * u) @ Wd.T
    logits = rms_norm(h) @ E.T                 imq_add_rmsnorm, imq_qmv (fp32, tied head)

for 1 and 2 requests; from FUSED_NORM_ROWS (3) requests the same step runs with the RMSNorms
folded into the projections (`_decode_step_fused_norms`: five projection or attention
launches per layer, and an epilogue launch after each of o and down where they split K).

All buffers are allocated once per (model, batch size) in `DecodeState`; a step only
launches kernels, so it can be captured in a HIP graph and replayed.  Every launch goes
through the C ABI; there is no host fallback.

`PersistentDecode` runs the step at batch 1 as a program of fused stages
(include/ironmule_step.h): the embedding launch, then one launch for all layers and the
head (or one launch per stage), with every RMSNorm but the first layer's input norm folded
into the projections around it.

`prefill` runs a whole prompt through the same model at once, the library path a prompt
takes (ironmule/cuda_native.py:171-179): every projection of more than 32 rows is
imq_dequant to fp16 and one GEMM, attention is causal over the prompt in fp32, the KV
pools of the request's slot are written for positions 0..T-1, and the head is computed
for the last position only (ironmule/cuda_native.py:271-303, `head_skip_prefill`).
"""

from __future__ import annotations

import contextlib
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
    layout (ironmule/dense_plan.py:297-301).  `max_len` bounds the lengths a step may
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
        self.attn = torch.empty((batch, c.heads * c.head_dim), **bf)
        self.delta = torch.empty((batch, c.hidden), **bf)
        self.gate = torch.empty((batch, c.intermediate), **bf)
        self.up = torch.empty((batch, c.intermediate), **bf)
        self.act = torch.empty((batch, c.intermediate), **bf)
        self.logits = torch.empty((batch, c.vocab), dtype=torch.float32, device=device)
        # the residual stream's per-row sums of squares for the RMSNorms folded into the
        # projections (batches of FUSED_NORM_ROWS or more)
        self.stats_in = _native.NormStats(batch, c.hidden, device)
        self.stats_post = _native.NormStats(batch, c.hidden, device)
        self.qkv_planes = _native.QkvPlanes(batch, c.heads, c.kv_heads, device)
        # the o and down projections' K-range planes (both hidden wide), added into h by
        # their own epilogue launch
        self.res_planes = _native.ResidualPlanes(batch, c.hidden, device)
        # the activations the batched step's launches hand to one another, in the 32-row
        # tile layout (the MFMA kernels read them as contiguous 1 KB pieces): x' for q/k/v
        # and gate/up, the attention output for o, SiLU * up for down
        rows = _native.MAX_ROWS
        self.x_t = torch.zeros(rows * c.hidden, **bf)
        self.attn_t = torch.zeros(rows * c.heads * c.head_dim, **bf)
        self.act_t = torch.zeros(rows * c.intermediate, **bf)
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


# From this batch the RMSNorms run inside the projections: on the synthetic Qwen3-4B step
# 2.21 against 2.32 ms at 3 requests and 2.27 against 2.53 at 4, but 2.41 against 1.85 at 2
# (where the few-row VALU kernels take the projections).
FUSED_NORM_ROWS = 3


def decode_step(weights: DecoderWeights, state: DecodeState, stream=None) -> torch.Tensor:
    """Launches one decode step for the requests in `state` (tokens, slots, positions set
    by `set_requests`); returns state.logits (B, vocab) fp32, written on `stream`."""
    if state.batch >= FUSED_NORM_ROWS:
        return _decode_step_fused_norms(weights, state, stream)
    c, s = weights.config, state
    n = _native
    n.embed(*weights.embed, s.tokens, s.h, stream=stream)
    delta = None
    for i, layer in enumerate(weights.layers):
        n.add_rmsnorm(s.h, layer["input_norm"], s.x, c.eps, delta=delta, stream=stream)
        n.qmv_grouped([layer["q"], layer["k"], layer["v"]], [s.x, s.x, s.x],
                      outs=[s.q, s.k, s.v], stream=stream)
        # one launch (the decode programs' attention stage; the KV pools of qk_norm_rope
        # followed by attention_decode, the output to the attention's oracle bar)
        n.attention_fused(s.q, s.k, s.v, layer["q_norm"], layer["k_norm"], s.positions,
                          s.slot_ids, s.k_pool[i], s.v_pool[i], s.attn, s.max_len, c.theta,
                          c.eps, s.workspace, s.attn_counters, stream=stream)
        n.qmv(*layer["o"], s.attn, out=s.delta, stream=stream)
        n.add_rmsnorm(s.h, layer["post_norm"], s.x, c.eps, delta=s.delta, stream=stream)
        if s.batch >= 5:  # gate, up and SiLU * up in one launch (the same bits)
            n.gate_up_silu(layer["gate"], layer["up"], s.x, s.act, stream=stream)
        else:
            n.qmv_grouped([layer["gate"], layer["up"]], [s.x, s.x], outs=[s.gate, s.up],
                          stream=stream)
            n.silu_mul(s.gate, s.up, s.act, stream=stream)
        n.qmv(*layer["down"], s.act, out=s.delta, stream=stream)
        delta = s.delta
    n.add_rmsnorm(s.h, weights.norm, s.x, c.eps, delta=delta, stream=stream)
    n.qmv(*weights.embed, s.x, out=s.logits, stream=stream)
    return s.logits


# Hidden sizes whose gate/up launch takes the row-band kernel (K / 256 wavefronts of 4, 8,
# 10 or 12): the batched step then hands its activations on in the 32-row tile layout.
TILED_GATE_UP_K = (1024, 2048, 2560, 3072)

# The widest K the row-band projection (a workgroup per 32 weight rows over the whole K)
# takes in the decode step: its x stream, the whole of x per workgroup, runs at about 70
# GB/s per CU, which beats the K-range planes and their epilogue launch at o's K = 4096
# (9.2 against 12.1 us at batch 32) but not at down's 9728 (18.0 against 14.7).
RESIDUAL_BANDS_MAX_K = 4096


def _residual_projection(weight, x, state: DecodeState, next_norm, x_out, stats_out, stream,
                         tiled: bool = False) -> None:
    """h += bf16(x @ W.T), x_out = bf16(h * next_norm) and the per-row partial sums of
    squares of the new h: over bands of 32 rows and the whole K up to RESIDUAL_BANDS_MAX_K,
    else as K-range planes and an epilogue launch when the projection splits, else in one
    launch.  With `tiled` x and x_out are 32-row tile layout buffers."""
    n, s = _native, state
    k = int(weight[0].shape[1]) * 8
    if k % 256 == 0 and k <= RESIDUAL_BANDS_MAX_K:
        n.qmv_residual_bands(weight, x, s.batch, s.h, next_norm=next_norm, x_out=x_out, stats_out=stats_out,
                             tiled=tiled, tiled_out=tiled, stream=stream)
        return
    if tiled:  # K-range planes read the tiled x, the epilogue writes x' tiled
        n.qmv_residual_planes(weight, x, s.res_planes, stream=stream, tiled=True)
        n.residual_planes(s.res_planes, s.h, next_norm=next_norm, x_out=x_out, stats_out=stats_out,
                          stream=stream, tiled_out=True)
        return
    if 2 <= n.residual_split_planes(weight, x) <= s.res_planes.max_planes:
        n.qmv_residual_planes(weight, x, s.res_planes, stream=stream)
        n.residual_planes(s.res_planes, s.h, next_norm=next_norm, x_out=x_out, stats_out=stats_out,
                          stream=stream)
    else:
        n.qmv_norm([weight], x, residual=s.h, next_norm=next_norm, x_out=x_out, stats_out=stats_out,
                   stream=stream)


def _decode_step_fused_norms(weights: DecoderWeights, state: DecodeState, stream=None) -> torch.Tensor:
    """decode_step with every RMSNorm but the last folded into the launches around it, six
    launches per layer:

        x' = bf16(h * w_in), stats                 imq_rmsnorm_prescale (first layer only)
        per layer:
            q, k, v = inv * (x' @ W.T)             imq_qmv_norm_planes (norm_in: the stats;
                                                   bands of 32 rows over the whole K, one
                                                   fp32 plane per projection; the first
                                                   layer's from x' as rows: K-range planes)
            attention                              imq_attention_fused_planes (adds the
                                                   planes as it reads q, k and v)
            h += o @ Wo.T; x' = bf16(h * w_post)   imq_qmv_residual_bands (bands of 32 rows
                                                   over the whole K with the residual add, x'
                                                   and per-band sums of squares)
            act = silu(inv * g) * (inv * u)        imq_qmv_gate_up_silu_norm (bands of rows
                                                   of both weights, one workgroup per CU)
            h += act @ Wd.T; x' = bf16(h * w_in')  imq_qmv_norm_planes + imq_residual_planes
                                                   (K-range planes, then the residual
                                                   epilogue: h, x' and the per-tile sums of
                                                   squares; the last layer updates h only)
        logits = rms_norm(h) @ E.T                 imq_add_rmsnorm, imq_qmv

    inv is each row's 1 / rms(h), so inv * (x' W^T) is rms_norm(h) W^T up to the place of one
    bf16 rounding (x' is rounded before the scaling instead of after it).  Where the hidden
    size takes the row-band gate/up kernel (TILED_GATE_UP_K), the launches hand x', the
    attention output and act to one another in the 32-row tile layout (IMQ_LD_TILED), which
    the batched kernels read as contiguous 1 KB pieces; otherwise as rows."""
    c, s = weights.config, state
    n = _native
    n.embed(*weights.embed, s.tokens, s.h, stream=stream)
    n.rmsnorm_prescale(s.h, weights.layers[0]["input_norm"], s.x, s.stats_in, stream=stream)
    t = c.hidden in TILED_GATE_UP_K  # the activations between launches in the tile layout
    xn, attn, act = (s.x_t, s.attn_t, s.act_t) if t else (s.x, s.attn, s.act)
    for i, layer in enumerate(weights.layers):
        # the first layer's x' comes from the prescale as rows
        n.qmv_norm_planes([layer["q"], layer["k"], layer["v"]], s.x if i == 0 else xn, s.qkv_planes,
                          norm_in=s.stats_in, eps=c.eps, stream=stream, tiled=t and i > 0)
        n.attention_fused_planes(s.qkv_planes, layer["q_norm"], layer["k_norm"], s.positions,
                                 s.slot_ids, s.k_pool[i], s.v_pool[i], attn, s.max_len,
                                 c.theta, c.eps, s.workspace, s.attn_counters, stream=stream, tiled=t)
        _residual_projection(layer["o"], attn, s, layer["post_norm"], xn, s.stats_post, stream, tiled=t)
        n.gate_up_silu_norm(layer["gate"], layer["up"], xn, act, s.stats_post, c.eps,
                            stream=stream, rows=s.batch, tiled_x=t, tiled_out=t)
        last = i + 1 == len(weights.layers)
        _residual_projection(layer["down"], act, s, None if last else weights.layers[i + 1]["input_norm"],
                             None if last else xn, None if last else s.stats_in, stream, tiled=t)
    n.add_rmsnorm(s.h, weights.norm, s.x, c.eps, stream=stream)
    n.qmv(*weights.embed, s.x, out=s.logits, stream=stream)
    return s.logits


class PersistentDecode:
    """The batch-1 decode step as a program of fused stages (imq_decode_program_create):
    `step()` launches the embedding and the program and returns state.logits.  With
    `staged` each stage is its own launch (5 per layer: q/k/v with the RMSNorm, attention
    with q/k norm + rotary + KV write + the split merge, o with the residual add, gate/up
    with the RMSNorm and SiLU * up, down with the residual add); otherwise one persistent
    launch runs them all.  The two forms give the same bits; every RMSNorm but the first
    layer's input norm is folded into the projections around it (the o and down stages
    write x' = bf16(h * w_next) and per-tile sums of squares, the next stage scales its
    outputs by 1/rms), so against `decode_step` at batch 1 (RMSNorm launches) the logits
    agree to the folding's rounding level."""

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


# ------------------------------------------------------------------ prefill

def _rms_norm(h: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """fp32 rows scaled to unit root-mean-square, times a bf16 weight, rounded to bf16."""
    inv = torch.rsqrt(h.pow(2).mean(dim=-1, keepdim=True) + eps)
    return (h * inv * weight.float()).to(torch.bfloat16)


def _rotary(x: torch.Tensor, positions: torch.Tensor, theta: float) -> torch.Tensor:
    """Non-interleaved rotary embedding of (T, H, D) fp32 rows: the pair (i, i + D/2) turns
    by position * theta^(-2i/D), as the decode kernels apply it."""
    half = x.shape[-1] // 2
    freq = theta ** (-torch.arange(half, dtype=torch.float64, device=x.device) * 2.0 / x.shape[-1])
    angle = positions.to(torch.float64)[:, None] * freq[None, :]
    cos, sin = angle.cos().float()[:, None, :], angle.sin().float()[:, None, :]
    lo, hi = x[..., :half], x[..., half:]
    return torch.cat([lo * cos - hi * sin, lo * sin + hi * cos], dim=-1)


def _project(x: torch.Tensor, quant: Quant, stream=None) -> torch.Tensor:
    """bf16 rows times a 4-bit weight: the qmv kernel up to 32 rows, else imq_dequant to
    fp16 and one GEMM (fp16 products, fp32 accumulation), rounded to bf16."""
    w, s, b = quant
    if x.shape[0] <= _native.MAX_ROWS:
        return _native.qmv(w, s, b, x, stream=stream)
    dense = _native.dequant(w, s, b, torch.float16, stream=stream)
    return torch.matmul(x.to(torch.float16), dense.T).to(torch.bfloat16)


def prefill(weights: DecoderWeights, state: DecodeState, tokens, slot: int,
            stream=None) -> torch.Tensor:
    """Runs the prompt `tokens` (positions 0..T-1) of one request through the model,
    writes its keys and values into KV slot `slot` of `state`'s pools, and returns the
    fp32 logits (vocab,) of the last position.  A decode step for this request then
    continues at position T."""
    c = weights.config
    count = len(tokens)
    if not 1 <= count <= state.max_len:
        raise ValueError(f"a prompt holds 1 to {state.max_len} tokens, got {count}")
    if not 0 <= slot < state.slots:
        raise ValueError(f"slot must lie in [0, {state.slots})")
    device = state.h.device
    with torch.cuda.stream(stream) if stream is not None else contextlib.nullcontext():
        ids = torch.as_tensor(list(tokens), dtype=torch.int32).to(device)
        h = torch.empty((count, c.hidden), dtype=torch.float32, device=device)
        _native.embed(*weights.embed, ids, h, stream=stream)
        positions = torch.arange(count, device=device)
        causal = torch.ones((count, count), dtype=torch.bool, device=device).tril()
        group = c.heads // c.kv_heads
        for i, layer in enumerate(weights.layers):
            x = _rms_norm(h, layer["input_norm"], c.eps)
            q = _project(x, layer["q"], stream).float().view(count, c.heads, c.head_dim)
            k = _project(x, layer["k"], stream).float().view(count, c.kv_heads, c.head_dim)
            v = _project(x, layer["v"], stream).view(count, c.kv_heads, c.head_dim)
            q = _rotary(_rms_norm(q, layer["q_norm"], c.eps).float(), positions, c.theta)
            k = _rotary(_rms_norm(k, layer["k_norm"], c.eps).float(), positions, c.theta)
            state.k_pool[i][slot, :, :count] = k.to(torch.bfloat16).transpose(0, 1)
            state.v_pool[i][slot, :, :count] = v.transpose(0, 1)
            # causal attention in fp32 over the bf16 q, keys and values
            qh = q.to(torch.bfloat16).float().transpose(0, 1).contiguous()       # (H, T, D)
            kh = state.k_pool[i][slot, :, :count].float().repeat_interleave(group, dim=0)
            vh = state.v_pool[i][slot, :, :count].float().repeat_interleave(group, dim=0)
            scores = torch.matmul(qh, kh.transpose(1, 2).contiguous()) * c.head_dim ** -0.5
            scores = scores.masked_fill(~causal, float("-inf"))
            attn = torch.matmul(torch.softmax(scores, dim=-1), vh)                 # (H, T, D)
            attn = attn.transpose(0, 1).reshape(count, c.heads * c.head_dim).to(torch.bfloat16)
            h = h + _project(attn, layer["o"], stream).float()
            x = _rms_norm(h, layer["post_norm"], c.eps)
            gate = _project(x, layer["gate"], stream).float()
            up = _project(x, layer["up"], stream).float()
            act = (torch.nn.functional.silu(gate) * up).to(torch.bfloat16)
            h = h + _project(act, layer["down"], stream).float()
        last = _rms_norm(h[-1:], weights.norm, c.eps)
        return _native.qmv(*weights.embed, last, out_dtype=torch.float32, stream=stream)[0]


# ------------------------------------------------------------------ module form

class KVCache:
    """One request's keys and values for one layer: (kv_heads, capacity, head_dim) bf16, the
    first `offset` positions filled."""

    def __init__(self, kv_heads: int, capacity: int, head_dim: int, device) -> None:
        self.keys = torch.zeros((kv_heads, capacity, head_dim), dtype=torch.bfloat16, device=device)
        self.values = torch.zeros_like(self.keys)
        self.offset = 0

    @property
    def capacity(self) -> int:
        return int(self.keys.shape[1])

    def update_and_fetch(self, k: torch.Tensor, v: torch.Tensor):
        """Appends one position's (kv_heads, head_dim) key and value; returns the filled
        keys and values (kv_heads, offset, head_dim)."""
        if self.offset >= self.capacity:
            raise ValueError(f"the cache holds {self.capacity} positions")
        self.keys[:, self.offset] = k
        self.values[:, self.offset] = v
        self.offset += 1
        return self.keys[:, :self.offset], self.values[:, :self.offset]


class DecoderLayer(torch.nn.Module):
    """One layer's 4-bit projections (QuantizedLinear over the layer's tensors) and norms."""

    def __init__(self, layer: dict) -> None:
        super().__init__()
        from .quantized import QuantizedLinear
        for name in ("q", "k", "v", "o", "gate", "up", "down"):
            setattr(self, f"{name}_proj", QuantizedLinear(*layer[name]))
        for name in ("input_norm", "post_norm", "q_norm", "k_norm"):
            self.register_buffer(name, layer[name])


class Decoder(torch.nn.Module):
    """The decoder of `DecoderWeights` as modules: each projection a QuantizedLinear (its
    forward is the library path: imq_qmv for a decode row), the tied 4-bit embedding and
    head.  `step` decodes one token of one request over that request's KVCaches; the
    composition is `ironmule_amd.paired.paired_forward`'s, which steps several requests."""

    def __init__(self, weights: DecoderWeights) -> None:
        super().__init__()
        from .quantized import QuantizedEmbedding
        self.config = weights.config
        self.layers = torch.nn.ModuleList([DecoderLayer(layer) for layer in weights.layers])
        self.embed_tokens = QuantizedEmbedding(*weights.embed)
        self.register_buffer("norm", weights.norm)

    def make_caches(self, capacity: int) -> list[KVCache]:
        c = self.config
        device = self.norm.device
        return [KVCache(c.kv_heads, capacity, c.head_dim, device) for _ in range(c.layers)]

    def embed(self, token: int) -> torch.Tensor:
        """The token's embedding row, fp32 (1, hidden)."""
        ids = torch.tensor([int(token)], dtype=torch.int32, device=self.norm.device)
        h = torch.empty((1, self.config.hidden), dtype=torch.float32, device=self.norm.device)
        e = self.embed_tokens
        return _native.embed(e.weight, e.scales, e.biases, ids, h)

    def attend(self, layer: DecoderLayer, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
               cache: KVCache) -> torch.Tensor:
        """q/k norm, rotary at the cache's next position, the KV append and attention over
        the cache, for one request's (1, ...) bf16 q, k, v; returns bf16 (1, heads * head_dim)."""
        c = self.config
        pos = torch.tensor([cache.offset], device=q.device)
        qh = _rotary(_rms_norm(q.float().view(1, c.heads, c.head_dim), layer.q_norm, c.eps).float(),
                     pos, c.theta).to(torch.bfloat16)
        kh = _rotary(_rms_norm(k.float().view(1, c.kv_heads, c.head_dim), layer.k_norm, c.eps).float(),
                     pos, c.theta).to(torch.bfloat16)
        keys, values = cache.update_and_fetch(kh[0], v.view(c.kv_heads, c.head_dim))
        group = c.heads // c.kv_heads
        kf = keys.float().repeat_interleave(group, dim=0)                  # (H, L, D)
        vf = values.float().repeat_interleave(group, dim=0)
        scores = torch.matmul(kf, qh[0].float().unsqueeze(-1)).squeeze(-1) * c.head_dim ** -0.5
        out = torch.matmul(torch.softmax(scores, dim=-1).unsqueeze(1), vf).squeeze(1)  # (H, D)
        return out.reshape(1, c.heads * c.head_dim).to(torch.bfloat16)

    def head(self, h: torch.Tensor) -> torch.Tensor:
        """Final norm and the tied head: fp32 logits (vocab,)."""
        e = self.embed_tokens
        x = _rms_norm(h, self.norm, self.config.eps)
        return _native.qmv(e.weight, e.scales, e.biases, x, out_dtype=torch.float32)[0]

    def step(self, token: int, caches: list[KVCache]) -> torch.Tensor:
        from .paired import paired_forward
        return paired_forward(self, [token], [caches], share=False)[0]
