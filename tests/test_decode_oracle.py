"""Pins the decode-step oracle (oracle/decode_oracle.py) on the CPU.

Each helper is checked against an independent implementation (torch's own CPU
rms_norm, scaled_dot_product_attention and silu, in float64) or a closed form the
mathematics fixes, chosen so a plausible mistake (the interleaved rotary layout, a
missing scale, the wrong query-head to KV-head map, a mean over the wrong axis) fails.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import decode_oracle as do

RNG = np.random.default_rng(20261201)


def test_rms_norm_matches_torch():
    x = RNG.standard_normal((5, 2560))
    w = RNG.uniform(0.5, 1.5, 2560)
    got = do.rms_norm(x, w, 1e-6)
    want = torch.nn.functional.rms_norm(torch.from_numpy(x), (2560,), torch.from_numpy(w), 1e-6)
    np.testing.assert_allclose(got, want.numpy(), rtol=1e-12, atol=0)


def test_rms_norm_of_a_constant_row_is_the_weight():
    w = RNG.uniform(0.5, 1.5, 128)
    np.testing.assert_allclose(do.rms_norm(np.full((1, 128), -3.0), w, 0.0)[0], -w, rtol=1e-14)


def _rope_complex(x, positions, theta):
    """The same rotation written as complex multiplication of (x_i + j x_{i+64})."""
    half = x.shape[-1] // 2
    z = x[..., :half] + 1j * x[..., half:]
    freq = theta ** (-np.arange(half) / half)
    z = z * np.exp(1j * np.asarray(positions)[:, None, None] * freq)
    return np.concatenate([z.real, z.imag], axis=-1)


def test_rope_position_zero_is_identity():
    x = RNG.standard_normal((3, 4, 128))
    np.testing.assert_array_equal(do.rope(x, np.zeros(3), 1e6), x)


def test_rope_matches_complex_rotation_and_preserves_pair_lengths():
    x = RNG.standard_normal((4, 8, 128))
    pos = np.array([1, 17, 512, 4095])
    got = do.rope(x, pos, 1e6)
    np.testing.assert_allclose(got, _rope_complex(x, pos, 1e6), rtol=1e-12, atol=1e-12)
    before = x[..., :64] ** 2 + x[..., 64:] ** 2
    after = got[..., :64] ** 2 + got[..., 64:] ** 2
    np.testing.assert_allclose(after, before, rtol=1e-12)


def test_rope_rotations_compose():
    x = RNG.standard_normal((2, 2, 128))
    a, b = np.array([5, 300]), np.array([7, 211])
    np.testing.assert_allclose(do.rope(do.rope(x, a, 1e4), b, 1e4), do.rope(x, a + b, 1e4),
                               rtol=1e-10, atol=1e-12)


def test_rope_is_not_the_interleaved_layout():
    x = np.zeros((1, 1, 128))
    x[0, 0, 0] = 1.0  # dimension 0 pairs with 64, not with 1
    out = do.rope(x, np.array([1]), 1e6)
    assert abs(out[0, 0, 64] - np.sin(1.0)) < 1e-12 and out[0, 0, 1] == 0.0


def _sdpa(q, k, v, scale):
    hq, hkv = q.shape[0], k.shape[0]
    kk = torch.from_numpy(k).repeat_interleave(hq // hkv, dim=0)
    vv = torch.from_numpy(v).repeat_interleave(hq // hkv, dim=0)
    out = torch.nn.functional.scaled_dot_product_attention(
        torch.from_numpy(q)[:, None, :], kk, vv, scale=scale)
    return out[:, 0, :].numpy()


@pytest.mark.parametrize("hq,hkv,length", [(32, 8, 513), (8, 8, 1), (16, 2, 64), (8, 1, 65)])
def test_attention_matches_torch_sdpa(hq, hkv, length):
    q = RNG.standard_normal((hq, 128))
    k = RNG.standard_normal((hkv, length, 128))
    v = RNG.standard_normal((hkv, length, 128))
    np.testing.assert_allclose(do.attention(q, k, v, 128 ** -0.5), _sdpa(q, k, v, 128 ** -0.5),
                               rtol=1e-10, atol=1e-12)


def test_attention_special_cases():
    k = RNG.standard_normal((2, 1, 128))
    v = RNG.standard_normal((2, 1, 128))
    q = RNG.standard_normal((8, 128))
    out = do.attention(q, k, v, 0.1)  # one key: its value, for every head of the group
    np.testing.assert_allclose(out, np.repeat(v[:, 0, :], 4, axis=0), rtol=1e-14)
    k = RNG.standard_normal((2, 9, 128))
    v = RNG.standard_normal((2, 9, 128))
    out = do.attention(np.zeros((4, 128)), k, v, 0.1)  # q = 0: the mean of the values
    np.testing.assert_allclose(out, np.repeat(v.mean(axis=1), 2, axis=0), rtol=1e-12)


def test_silu_mul_matches_torch():
    g = RNG.standard_normal(1000) * 6
    u = RNG.standard_normal(1000)
    want = torch.nn.functional.silu(torch.from_numpy(g)) * torch.from_numpy(u)
    np.testing.assert_allclose(do.silu_mul(g, u), want.numpy(), rtol=1e-13, atol=1e-300)


def _tiny_model(layers=2, dim=256, heads=4, kv_heads=2, inter=512, vocab=300):
    def w(n, k):
        return RNG.uniform(-0.05, 0.05, (n, k))
    lay = [do.Layer(wq=w(heads * 128, dim), wk=w(kv_heads * 128, dim), wv=w(kv_heads * 128, dim),
                    wo=w(dim, heads * 128), wg=w(inter, dim), wu=w(inter, dim), wd=w(dim, inter),
                    input_norm=RNG.uniform(0.9, 1.1, dim), post_norm=RNG.uniform(0.9, 1.1, dim),
                    q_norm=RNG.uniform(0.9, 1.1, 128), k_norm=RNG.uniform(0.9, 1.1, 128))
           for _ in range(layers)]
    return do.Model(layers=lay, embed=RNG.uniform(-0.1, 0.1, (vocab, dim)),
                    norm=RNG.uniform(0.9, 1.1, dim), heads=heads, kv_heads=kv_heads, eps=1e-6,
                    theta=1e6)


def _pools(model, slots=4, capacity=16):
    shape = (slots, model.kv_heads, capacity, 128)
    return ([RNG.standard_normal(shape) * 0.5 for _ in model.layers],
            [RNG.standard_normal(shape) * 0.5 for _ in model.layers])


@pytest.mark.parametrize("round_bf16", [True, False])
def test_decode_step_rows_are_independent(round_bf16):
    """A batched step equals the single-row steps (each row reads only its own slot)."""
    model = _tiny_model()
    keys, values = _pools(model)
    k1, v1 = [a.copy() for a in keys], [a.copy() for a in values]
    tokens, slots, positions = [3, 250, 17], [2, 0, 3], [5, 0, 15]
    batched = do.decode_step(model, keys, values, tokens, slots, positions, round_bf16)
    for r in range(3):
        single = do.decode_step(model, k1, v1, [tokens[r]], [slots[r]], [positions[r]], round_bf16)
        np.testing.assert_allclose(batched[r], single[0], rtol=1e-12, atol=1e-12)
    for i in range(len(model.layers)):  # and both wrote the same keys and values
        np.testing.assert_allclose(keys[i], k1[i], rtol=1e-12, atol=1e-14)
        np.testing.assert_allclose(values[i], v1[i], rtol=1e-12, atol=1e-14)


def test_decode_step_rounding_points_are_small_perturbations():
    """The bf16 rounding points move the logits by about bf16 precision, not more."""
    model = _tiny_model()
    keys, values = _pools(model)
    k2, v2 = [a.copy() for a in keys], [a.copy() for a in values]
    a = do.decode_step(model, keys, values, [7], [1], [9], True)
    b = do.decode_step(model, k2, v2, [7], [1], [9], False)
    rel = np.abs(a - b).max() / np.abs(b).max()
    assert 1e-5 < rel < 5e-2, rel


@pytest.mark.parametrize("fold_first,fold_final", [(True, False), (False, True), (True, True)])
def test_folded_norms_are_the_same_composition_without_rounding(fold_first, fold_final):
    """Without rounding, inv * ((h * w) W^T) is rms_norm(h) W^T: the folded-norm step equals
    the unfolded one to float64 precision, whichever norms are folded."""
    model = _tiny_model()
    keys, values = _pools(model)
    k2, v2 = [a.copy() for a in keys], [a.copy() for a in values]
    a = do.decode_step(model, keys, values, [7, 120], [1, 2], [9, 3], False)
    b = do.decode_step(model, k2, v2, [7, 120], [1, 2], [9, 3], False, fold_norms=True,
                       fold_first=fold_first, fold_final=fold_final)
    np.testing.assert_allclose(b, a, rtol=1e-11, atol=1e-13 * np.abs(a).max())
    for i in range(len(model.layers)):
        np.testing.assert_allclose(k2[i], keys[i], rtol=1e-11, atol=1e-13)


def test_folded_norms_move_only_rounding_points():
    """With rounding the folded step differs from the unfolded one by bf16-level amounts
    (the inputs are rounded before the 1/rms scaling instead of after it); the previous test
    shows that without rounding they are one composition, so a fold that dropped the scale
    or applied it twice would fail there."""
    model = _tiny_model()
    keys, values = _pools(model)
    k2, v2 = [a.copy() for a in keys], [a.copy() for a in values]
    a = do.decode_step(model, keys, values, [7], [1], [9], True)
    b = do.decode_step(model, k2, v2, [7], [1], [9], True, fold_norms=True)
    rel = np.abs(a - b).max() / np.abs(a).max()
    assert 0 < rel < 5e-2, rel
