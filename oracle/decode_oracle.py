"""CPU oracle for the decode step around the 4-bit projections — TEST INFRASTRUCTURE ONLY.

Only `tests/`, `__graft_entry__.smoke()` and the CPU-baseline leg of `bench.py` may use
this module, and only as the checker.  It restates, in numpy float64, the reference's
decode step for a Qwen3-style decoder (ironmule/dense_cpu.py:188-220, `CpuDensePlan.
forward`; ironmule/dense_plan.py:337-371, `DensePlan.forward` and `_rope`):

    h = embed(tokens)                                         (fp32 residual stream)
    per layer:
        x = rms_norm(h, input_layernorm)                      -> bf16 (qmv input)
        q, k, v = x @ Wq.T, x @ Wk.T, x @ Wv.T                 -> bf16
        q, k = q_norm(q), k_norm(k)                           -> bf16 (module outputs)
        q, k = rope(q, pos), rope(k, pos)                     -> bf16
        KV[slot][:, pos] = k, v
        o = softmax(scale * q . K[:pos+1]) V[:pos+1]          -> bf16 (GQA)
        h = h + o @ Wo.T                                      (o_proj output bf16)
        x = rms_norm(h, post_attention_layernorm)             -> bf16
        h = h + (silu(x @ Wg.T) * (x @ Wu.T)) @ Wd.T          (bf16 at each output)
    logits = rms_norm(h, norm) @ Whead.T                      (fp32)

`gemma3_decode_step` restates the composition of the reference's paired step for its admitted
architecture, Gemma 3 (ironmule/paired_research.py:177-215, over mlx-lm 0.31.3's
`models/gemma3_text`, a dependency not in the reference tree): the embedding times
bf16(sqrt(hidden)); per layer x = rms_norm(h) with weight 1 + w, q/k/v, q/k norm (1 + w),
rotary with base 10^4 on sliding-window layers and 10^6 on global ones (every `pattern`-th
layer is global), attention with scale query_pre_attn_scalar^-0.5 over the whole context
(global) or the last `window` positions (sliding), h += rms_norm(o_proj(attn)) (1 + w; a
plain add in bf16, the reference's clip_residual for bf16), the MLP gelu_tanh(gate) * up
between a pre and a post RMSNorm, h += its output; a final RMSNorm (1 + w) and the tied head.
It is pinned against transformers' Gemma3ForCausalLM (tests/test_decode_oracle_hf.py).
Parity unpinned there: MLX's bf16 op-by-op rounding inside gelu_approx and rms_norm (this
restatement rounds once per operation's output, as the GPU module form does).

The "-> bf16" marks are where this build's GPU step rounds to bf16 (the projections'
inputs and outputs are bf16, as in the reference's GPU plans); `round_bf16=False` drops
them, giving the all-fp32 composition of the CPU plan.  Each helper names the reference
lines it restates; tests/test_decode_oracle.py pins every helper against an independent
implementation (torch's rms_norm / scaled_dot_product_attention / silu on the CPU) or a
closed form (rotations compose and preserve length, position 0 is the identity, one key
returns its value), and tests/test_decode_oracle_hf.py pins the composition itself: with
round_bf16=False, step-by-step decoding matches transformers' Qwen3ForCausalLM (same
weights, one causal forward) at the fp32 rounding level, while compositions with the rotary
or the q/k-norm skipped, or the MLP fed from the residual stream, do not.

`fold_norms` restates the rounding points of this build's GPU steps that fold an RMSNorm
into the projections it feeds: x' = bf16(h * w) is the projections' input and each output
row is scaled by 1 / rms(h) before its own rounding, so rms_norm(h) W^T is computed as
inv * ((h * w) W^T) with the bf16 rounding of the input placed before the scaling instead
of after it.  `fold_first` and `fold_final` say whether the first layer's input norm and the
final norm are folded too (the batched step folds every layer's norms but not the final
one; the batch-1 program folds every norm but the first layer's input norm).  Without
rounding the two placements are the same composition (tests/test_decode_oracle.py pins
that fold_norms=True with round_bf16=False equals the unfolded step).
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from . import oracle as qmv_oracle

HEAD_DIM = 128


def bf16_round(x: np.ndarray) -> np.ndarray:
    """Round to bf16 (nearest even) and back to float64."""
    f = np.asarray(x, dtype=np.float32)
    return qmv_oracle.bf16_to_f32(qmv_oracle.f32_to_bf16(f)).astype(np.float64)


def rms_norm(x: np.ndarray, weight: np.ndarray, eps: float) -> np.ndarray:
    """x * rsqrt(mean(x^2) + eps) * weight over the last axis (mx.fast.rms_norm,
    ironmule/dense_plan.py:348-352, 359, 362)."""
    x = np.asarray(x, dtype=np.float64)
    inv = 1.0 / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)
    return x * inv * np.asarray(weight, dtype=np.float64)


def rope(x: np.ndarray, positions: np.ndarray, theta: float) -> np.ndarray:
    """Non-interleaved rotary embedding over the last axis (D = 128): pair (i, i + D/2)
    turns by pos * theta^(-2i / D) (mx.fast.rope(..., traditional=False, base=theta,
    scale=1.0, offset=pos), ironmule/dense_plan.py:365-371).  x is (B, H, D), positions (B,)."""
    x = np.asarray(x, dtype=np.float64)
    half = x.shape[-1] // 2
    inv_freq = theta ** (-np.arange(half, dtype=np.float64) * 2.0 / x.shape[-1])
    ang = np.asarray(positions, dtype=np.float64)[:, None, None] * inv_freq[None, None, :]
    c, s = np.cos(ang), np.sin(ang)
    x1, x2 = x[..., :half], x[..., half:]
    return np.concatenate([x1 * c - x2 * s, x1 * s + x2 * c], axis=-1)


def attention(q: np.ndarray, keys: np.ndarray, values: np.ndarray, scale: float) -> np.ndarray:
    """Grouped-query attention of one request: q (Hq, D) against keys/values (Hkv, L, D);
    query head h reads KV head h // (Hq / Hkv) (ironmule/dense_cpu.py:180-185, `_attend`)."""
    hq, d = q.shape
    hkv = keys.shape[0]
    grouped = np.asarray(q, np.float64).reshape(hkv, hq // hkv, d)
    scores = grouped @ np.asarray(keys, np.float64).transpose(0, 2, 1) * scale  # (Hkv, G, L)
    scores -= scores.max(axis=-1, keepdims=True)
    p = np.exp(scores)
    p /= p.sum(axis=-1, keepdims=True)
    return (p @ np.asarray(values, np.float64)).reshape(hq, d)


def silu_mul(gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    """silu(gate) * up, silu(g) = g / (1 + exp(-g)) (swiglu, ironmule/dense_plan.py:360)."""
    g = np.asarray(gate, np.float64)
    return g / (1.0 + np.exp(-g)) * np.asarray(up, np.float64)


@dataclass
class Layer:
    """One decoder layer's dequantised weights (float64) and norm weights."""
    wq: np.ndarray
    wk: np.ndarray
    wv: np.ndarray
    wo: np.ndarray
    wg: np.ndarray
    wu: np.ndarray
    wd: np.ndarray
    input_norm: np.ndarray
    post_norm: np.ndarray
    q_norm: np.ndarray
    k_norm: np.ndarray


@dataclass
class Model:
    layers: list
    embed: np.ndarray   # (vocab, dim) dequantised, also the tied head
    norm: np.ndarray
    heads: int
    kv_heads: int
    eps: float
    theta: float


def decode_step(model: Model, keys: list, values: list, tokens, slots, positions,
                round_bf16: bool = True, fold_norms: bool = False, fold_first: bool = True,
                fold_final: bool = False):
    """One decode step of B requests; keys/values[layer] are (slots, Hkv, C, D) float64
    pools, updated in place at (slot, :, pos).  Returns float64 logits (B, vocab).
    fold_norms (with fold_first, fold_final): the folded-norm rounding points (module
    docstring)."""
    r = bf16_round if round_bf16 else (lambda a: np.asarray(a, np.float64))

    def normed(h, weight, folded):
        """The projections' input and the scale of their outputs for rms_norm(h, weight)."""
        if not (fold_norms and folded):
            return r(rms_norm(h, weight, model.eps)), 1.0
        hh = np.asarray(h, np.float64)
        inv = 1.0 / np.sqrt(np.mean(hh * hh, axis=-1, keepdims=True) + model.eps)
        return r(hh * np.asarray(weight, np.float64)), inv

    d = HEAD_DIM
    tokens = np.asarray(tokens)
    slots = np.asarray(slots)
    positions = np.asarray(positions)
    b = tokens.shape[0]
    h = model.embed[tokens].astype(np.float64)
    scale = d ** -0.5
    for i, lay in enumerate(model.layers):
        x, s = normed(h, lay.input_norm, i > 0 or fold_first)
        q = r(s * (x @ lay.wq.T)).reshape(b, model.heads, d)
        k = r(s * (x @ lay.wk.T)).reshape(b, model.kv_heads, d)
        v = r(s * (x @ lay.wv.T)).reshape(b, model.kv_heads, d)
        q = r(rope(r(rms_norm(q, lay.q_norm, model.eps)), positions, model.theta))
        k = r(rope(r(rms_norm(k, lay.k_norm, model.eps)), positions, model.theta))
        for row in range(b):
            keys[i][slots[row], :, positions[row]] = k[row]
            values[i][slots[row], :, positions[row]] = v[row]
        o = np.stack([r(attention(q[row], keys[i][slots[row], :, :positions[row] + 1],
                                  values[i][slots[row], :, :positions[row] + 1], scale))
                      for row in range(b)]).reshape(b, model.heads * d)
        h = h + r(o @ lay.wo.T)
        x, s = normed(h, lay.post_norm, True)
        act = r(silu_mul(r(s * (x @ lay.wg.T)), r(s * (x @ lay.wu.T))))
        h = h + r(act @ lay.wd.T)
    x, s = normed(h, model.norm, fold_final)
    return s * (x @ model.embed.T)


# ------------------------------------------------------------------ Gemma 3

def gemma_norm(x: np.ndarray, weight: np.ndarray, eps: float, r=lambda a: np.asarray(a, np.float64)) -> np.ndarray:
    """Gemma's RMSNorm: the weight is 1 + w (rounded by `r`, bf16 in the reference's
    arithmetic), the rest as rms_norm."""
    return rms_norm(x, r(1.0 + np.asarray(weight, np.float64)), eps)


def gelu_tanh(x: np.ndarray) -> np.ndarray:
    """The tanh approximation of GELU (mlx's gelu_approx, transformers' gelu_pytorch_tanh)."""
    x = np.asarray(x, np.float64)
    return 0.5 * x * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (x + 0.044715 * x ** 3)))


@dataclass
class Gemma3Layer:
    """One Gemma 3 layer's dequantised weights (float64) and its six norm weights (w of
    the 1 + w form)."""
    wq: np.ndarray
    wk: np.ndarray
    wv: np.ndarray
    wo: np.ndarray
    wg: np.ndarray
    wu: np.ndarray
    wd: np.ndarray
    input_norm: np.ndarray
    post_attn_norm: np.ndarray
    pre_ff_norm: np.ndarray
    post_ff_norm: np.ndarray
    q_norm: np.ndarray
    k_norm: np.ndarray


@dataclass
class Gemma3Model:
    layers: object       # an iterable of Gemma3Layer
    embed: np.ndarray    # (vocab, hidden) dequantised, also the tied head
    norm: np.ndarray
    heads: int
    kv_heads: int
    head_dim: int
    eps: float
    theta_global: float
    theta_local: float
    window: int          # a sliding layer attends to positions pos - window + 1 .. pos
    pattern: int         # layer i is global when i % pattern == pattern - 1
    query_scalar: float  # attention scale query_scalar ** -0.5


def gemma3_decode_step(model: Gemma3Model, keys: list, values: list, tokens, slots, positions,
                       round_bf16: bool = True):
    """One decode step of B requests through a Gemma 3 decoder; keys/values[layer] are
    (slots, Hkv, C, D) float64 pools, updated in place at (slot, :, pos).  With round_bf16
    every module output is rounded to bf16 (the residual stream included, as in the
    reference's bf16 model); without, the all-float64 composition.  Returns float64 logits
    (B, vocab)."""
    r = bf16_round if round_bf16 else (lambda a: np.asarray(a, np.float64))
    d = model.head_dim
    tokens = np.asarray(tokens)
    slots = np.asarray(slots)
    positions = np.asarray(positions)
    b = tokens.shape[0]
    hidden = model.embed.shape[1]
    h = r(r(model.embed[tokens]) * r(np.sqrt(float(hidden))))
    scale = model.query_scalar ** -0.5
    eps = model.eps
    for i, lay in enumerate(model.layers):
        is_global = i % model.pattern == model.pattern - 1
        theta = model.theta_global if is_global else model.theta_local
        x = r(gemma_norm(h, lay.input_norm, eps, r))
        q = r(x @ lay.wq.T).reshape(b, model.heads, d)
        k = r(x @ lay.wk.T).reshape(b, model.kv_heads, d)
        v = r(x @ lay.wv.T).reshape(b, model.kv_heads, d)
        q = r(rope(r(gemma_norm(q, lay.q_norm, eps, r)), positions, theta))
        k = r(rope(r(gemma_norm(k, lay.k_norm, eps, r)), positions, theta))
        outs = []
        for row in range(b):
            pos = int(positions[row])
            keys[i][slots[row], :, pos] = k[row]
            values[i][slots[row], :, pos] = v[row]
            lo = 0 if is_global else max(0, pos - model.window + 1)
            outs.append(r(attention(q[row], keys[i][slots[row], :, lo:pos + 1],
                                    values[i][slots[row], :, lo:pos + 1], scale)))
        o = np.stack(outs).reshape(b, model.heads * d)
        h = r(h + r(gemma_norm(r(o @ lay.wo.T), lay.post_attn_norm, eps, r)))
        x = r(gemma_norm(h, lay.pre_ff_norm, eps, r))
        act = r(r(gelu_tanh(r(x @ lay.wg.T))) * r(x @ lay.wu.T))
        h = r(h + r(gemma_norm(r(act @ lay.wd.T), lay.post_ff_norm, eps, r)))
    x = r(gemma_norm(h, model.norm, eps, r))
    return x @ model.embed.T

