"""The Gemma 3 module form's own arithmetic on the CPU (ironmule_amd/gemma3.py): its
attention (q/k RMSNorm with 1 + w, rotary with the layer kind's base, the
query_pre_attn_scalar scale, the sliding window) against the decode oracle's helpers, and
its configuration.  The projections, embedding and head run on the GPU
(tests/test_paired_gpu.py); `attend` is plain torch and runs here on CPU tensors."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from ironmule_amd.gemma3 import Gemma3Config, Gemma3Decoder, gelu_tanh, random_gemma3_weights
from oracle import decode_oracle as do

CFG = Gemma3Config(hidden=256, layers=2, heads=4, kv_heads=2, head_dim=128, intermediate=512,
                   vocab=64, window=3, pattern=2, query_scalar=96.0)


@pytest.fixture(scope="module")
def model():
    return Gemma3Decoder(random_gemma3_weights(CFG, "cpu", seed=4))


def _bf16(a):
    return torch.from_numpy(np.asarray(a, np.float32)).to(torch.bfloat16)


def _vals(t):
    return t.float().numpy().astype(np.float64)


def _oracle_attend(layer, qs, ks, vs, index, window):
    """The oracle's q/k norm (1 + w, bf16 weight), rotary and attention over the positions a
    layer of this kind sees; one row per position."""
    r = do.bf16_round
    is_global = CFG.is_global(index)
    theta = CFG.theta_global if is_global else CFG.theta_local
    qn, kn = _vals(layer.q_norm), _vals(layer.k_norm)
    keys, values, outs = [], [], []
    for pos, (q, k, v) in enumerate(zip(qs, ks, vs)):
        qh = r(do.rope(r(do.gemma_norm(q.reshape(1, CFG.heads, CFG.head_dim), qn, CFG.eps, r)), [pos], theta))[0]
        kh = r(do.rope(r(do.gemma_norm(k.reshape(1, CFG.kv_heads, CFG.head_dim), kn, CFG.eps, r)), [pos], theta))[0]
        keys.append(kh)
        values.append(v.reshape(CFG.kv_heads, CFG.head_dim))
        lo = 0 if is_global else max(0, pos - window + 1)
        K = np.stack(keys[lo:], axis=1)
        V = np.stack(values[lo:], axis=1)
        outs.append(r(do.attention(qh, K, V, CFG.query_scalar ** -0.5)).reshape(-1))
    return np.stack(outs)


@pytest.mark.parametrize("index", [0, 1])
def test_attend_matches_the_oracle(model, index):
    """Layer 0 is a sliding-window layer (window 3), layer 1 global; seven positions."""
    rng = np.random.default_rng(index)
    n = 7
    qs = [_vals(_bf16(rng.standard_normal(CFG.heads * CFG.head_dim))) for _ in range(n)]
    ks = [_vals(_bf16(rng.standard_normal(CFG.kv_heads * CFG.head_dim))) for _ in range(n)]
    vs = [_vals(_bf16(rng.standard_normal(CFG.kv_heads * CFG.head_dim))) for _ in range(n)]
    layer = model.layers[index]
    cache = model.make_caches(n)[index]
    got = np.stack([_vals(model.attend(index, layer, _bf16(q)[None], _bf16(k)[None], _bf16(v)[None], cache))[0]
                    for q, k, v in zip(qs, ks, vs)])
    ref = _oracle_attend(layer, qs, ks, vs, index, CFG.window)
    ulp = np.maximum(np.abs(ref), 2.0 ** -126) * 2.0 ** -7
    assert (np.abs(got - ref) <= 2 * ulp).all(), np.abs(got - ref).max()
    if not CFG.is_global(index):  # the window matters: unwindowed attention differs
        wide = _oracle_attend(layer, qs, ks, vs, index, 10 ** 6)
        assert np.abs(got[-1] - wide[-1]).max() > 0.05


def test_config_and_helpers():
    c = Gemma3Config()
    assert (c.hidden, c.heads * c.head_dim, c.intermediate) == (3840, 4096, 15360)
    assert [c.is_global(i) for i in range(12)] == [i % 6 == 5 for i in range(12)]
    assert c.projections["o"] == (3840, 4096) and c.projections["down"] == (3840, 15360)
    x = torch.linspace(-6, 6, 101, dtype=torch.float64)
    assert torch.allclose(gelu_tanh(x), torch.nn.functional.gelu(x, approximate="tanh"), atol=1e-12)


def test_norm_uses_one_plus_w(model):
    x = _bf16(np.linspace(-2, 2, CFG.hidden))[None]
    w = model.layers[0].input_norm
    got = _vals(model.norm(x, w))
    ref = do.gemma_norm(_vals(x), _vals(w), CFG.eps, do.bf16_round)
    assert np.abs(got - do.bf16_round(ref)).max() <= 2.0 ** -7 * np.abs(ref).max()
