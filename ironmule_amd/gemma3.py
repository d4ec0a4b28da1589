"""A Gemma 3 text decoder on the 4-bit projections: the architecture the reference's paired
decode step composes (ironmule/paired_research.py:177-215, over mlx-lm's gemma3_text).

`Gemma3Decoder` is the module form `paired.paired_forward` steps for this architecture:
every projection a `QuantizedLinear` (its forward is the library path: imq_qmv for a decode
row), the tied 4-bit embedding and head, and the operations around them as the reference's
model defines them:

* the embedding row rounded to bf16 and multiplied by bf16(sqrt(hidden));
* RMSNorm with the weight 1 + w (rounded to bf16, as the reference adds 1 to its bf16
  weight), computed in fp32 and rounded to bf16 -- before attention, after attention (on
  its output, before the residual add), before and after the MLP, on q and k per head, and
  before the head;
* rotary embedding with base `theta_local` on sliding-window layers and `theta_global` on
  the global ones (layer i is global when i % pattern == pattern - 1); a sliding layer
  attends to the last `window` positions only; the attention scale is
  query_scalar ** -0.5;
* the MLP's gelu_tanh(gate) * up, each product rounded to bf16;
* the residual stream in bf16, each add rounded (the reference's clip_residual is a plain
  add for bf16).

The defaults are Gemma 3 12B's text shapes (hidden 3840: the q/k/v and gate/up
projections are the K=3840 ones the shared sweep serves; o has K = 16 x 256 = 4096 and
down K = 15360, the aligned shapes).
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch

from . import _native
from .decode import KVCache, Quant, _rotary


@dataclass(frozen=True)
class Gemma3Config:
    hidden: int = 3840
    layers: int = 48
    heads: int = 16
    kv_heads: int = 8
    head_dim: int = 256
    intermediate: int = 15360
    vocab: int = 262144
    eps: float = 1e-6
    theta_global: float = 1_000_000.0
    theta_local: float = 10_000.0
    window: int = 1024
    pattern: int = 6
    query_scalar: float = 256.0

    @property
    def projections(self) -> dict[str, tuple[int, int]]:
        """(out_features, in_features) of each 4-bit projection of a layer."""
        d, h = self.hidden, self.head_dim
        return {"q": (self.heads * h, d), "k": (self.kv_heads * h, d), "v": (self.kv_heads * h, d),
                "o": (d, self.heads * h), "gate": (self.intermediate, d),
                "up": (self.intermediate, d), "down": (d, self.intermediate)}

    def is_global(self, layer: int) -> bool:
        return layer % self.pattern == self.pattern - 1


NORMS = ("input_norm", "post_attn_norm", "pre_ff_norm", "post_ff_norm")


@dataclass
class Gemma3Weights:
    """4-bit projections and bf16 norm weights (the w of 1 + w) per layer, the tied 4-bit
    embedding and the final norm weight."""
    config: Gemma3Config
    layers: list = field(default_factory=list)
    embed: Quant = None
    norm: torch.Tensor = None


def random_gemma3_weights(config: Gemma3Config, device, seed: int = 0) -> Gemma3Weights:
    """Seeded synthetic weights: uniform 4-bit words, scales U(0.005, 0.02), biases
    U(-0.1, 0.1), norm weights w ~ U(-0.1, 0.1) (bf16)."""
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)

    def quant(n, k):
        w = torch.randint(0, 2**32, (n, k // 8), dtype=torch.int64, device=device,
                          generator=gen).to(torch.int32)
        s = torch.empty((n, k // 64), device=device).uniform_(0.005, 0.02, generator=gen)
        b = torch.empty((n, k // 64), device=device).uniform_(-0.1, 0.1, generator=gen)
        return w, s.to(torch.bfloat16), b.to(torch.bfloat16)

    def norm(n):
        return torch.empty(n, device=device).uniform_(-0.1, 0.1, generator=gen).to(torch.bfloat16)

    weights = Gemma3Weights(config)
    for _ in range(config.layers):
        layer = {name: quant(n, k) for name, (n, k) in config.projections.items()}
        layer.update({name: norm(config.hidden) for name in NORMS})
        layer.update(q_norm=norm(config.head_dim), k_norm=norm(config.head_dim))
        weights.layers.append(layer)
    weights.embed = quant(config.vocab, config.hidden)
    weights.norm = norm(config.hidden)
    return weights


class Gemma3Layer(torch.nn.Module):
    """One layer's 4-bit projections (QuantizedLinear over the layer's tensors) and norms."""

    def __init__(self, layer: dict) -> None:
        super().__init__()
        from .quantized import QuantizedLinear
        for name in ("q", "k", "v", "o", "gate", "up", "down"):
            setattr(self, f"{name}_proj", QuantizedLinear(*layer[name]))
        for name in (*NORMS, "q_norm", "k_norm"):
            self.register_buffer(name, layer[name])


def gelu_tanh(x: torch.Tensor) -> torch.Tensor:
    """The tanh approximation of GELU, in the precision of x."""
    return 0.5 * x * (1.0 + torch.tanh(math.sqrt(2.0 / math.pi) * (x + 0.044715 * x * x * x)))


class Gemma3Decoder(torch.nn.Module):
    """The decoder of `Gemma3Weights` as modules.  `step` decodes one token of one request
    over that request's KVCaches; the composition is `paired.paired_forward`'s."""

    architecture = "gemma3"

    def __init__(self, weights: Gemma3Weights) -> None:
        super().__init__()
        from .quantized import QuantizedEmbedding
        self.config = weights.config
        self.layers = torch.nn.ModuleList([Gemma3Layer(layer) for layer in weights.layers])
        self.embed_tokens = QuantizedEmbedding(*weights.embed)
        self.register_buffer("final_norm", weights.norm)
        c = self.config
        self._embed_scale = torch.tensor(math.sqrt(c.hidden), dtype=torch.bfloat16)

    def make_caches(self, capacity: int) -> list[KVCache]:
        c = self.config
        device = self.final_norm.device
        return [KVCache(c.kv_heads, capacity, c.head_dim, device) for _ in range(c.layers)]

    def norm(self, x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
        """RMSNorm over the last axis with the weight 1 + w (in bf16), fp32 arithmetic,
        bf16 result."""
        xf = x.float()
        inv = torch.rsqrt(xf.pow(2).mean(dim=-1, keepdim=True) + self.config.eps)
        return (xf * inv * (1.0 + weight).float()).to(torch.bfloat16)

    def embed(self, token: int) -> torch.Tensor:
        """The token's embedding row times bf16(sqrt(hidden)), bf16 (1, hidden)."""
        device = self.final_norm.device
        ids = torch.tensor([int(token)], dtype=torch.int32, device=device)
        h = torch.empty((1, self.config.hidden), dtype=torch.float32, device=device)
        e = self.embed_tokens
        row = _native.embed(e.weight, e.scales, e.biases, ids, h).to(torch.bfloat16)
        return (row.float() * self._embed_scale.float()).to(torch.bfloat16)

    def attend(self, index: int, layer: Gemma3Layer, q: torch.Tensor, k: torch.Tensor,
               v: torch.Tensor, cache: KVCache) -> torch.Tensor:
        """q/k norm, rotary at the cache's next position (the layer's base), the KV append and
        attention over the cache (its last `window` positions on a sliding layer), for one
        request's (1, ...) bf16 q, k, v; returns bf16 (1, heads * head_dim)."""
        c = self.config
        is_global = c.is_global(index)
        theta = c.theta_global if is_global else c.theta_local
        pos = cache.offset
        at = torch.tensor([pos], device=q.device)
        qh = _rotary(self.norm(q.view(1, c.heads, c.head_dim), layer.q_norm).float(), at, theta)
        kh = _rotary(self.norm(k.view(1, c.kv_heads, c.head_dim), layer.k_norm).float(), at, theta)
        keys, values = cache.update_and_fetch(kh.to(torch.bfloat16)[0], v.view(c.kv_heads, c.head_dim))
        lo = 0 if is_global else max(0, pos - c.window + 1)
        group = c.heads // c.kv_heads
        kf = keys[:, lo:].float().repeat_interleave(group, dim=0)      # (H, L, D)
        vf = values[:, lo:].float().repeat_interleave(group, dim=0)
        qf = qh.to(torch.bfloat16)[0].float()
        scores = torch.matmul(kf, qf.unsqueeze(-1)).squeeze(-1) * c.query_scalar ** -0.5
        out = torch.matmul(torch.softmax(scores, dim=-1).unsqueeze(1), vf).squeeze(1)  # (H, D)
        return out.reshape(1, c.heads * c.head_dim).to(torch.bfloat16)

    def head(self, h: torch.Tensor) -> torch.Tensor:
        """Final norm and the tied head: fp32 logits (vocab,)."""
        e = self.embed_tokens
        x = self.norm(h, self.final_norm)
        return _native.qmv(e.weight, e.scales, e.biases, x, out_dtype=torch.float32)[0]

    def step(self, token: int, caches: list[KVCache]) -> torch.Tensor:
        from .paired import paired_forward
        return paired_forward(self, [token], [caches], share=False)[0]
