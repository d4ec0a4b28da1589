"""Pins the CPU oracle before anything is checked against it.

Every oracle function is checked against something that does not share its code:
exact rational fixtures (tests/golden/qmv_golden.json, written by make_golden.py with
`fractions.Fraction`), closed forms, torch's own bf16 rounding, and special cases that
reduce the product to a textbook sum.  Planted mistakes (high-nibble-first unpack, a
dropped bias, a transposed group index) are shown to fail those checks, so the checks
can tell a wrong oracle from a right one.
"""

from __future__ import annotations

import json
import os

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
GOLDEN = json.load(open(os.path.join(HERE, "golden", "qmv_golden.json")))


def _arrays(p):
    w = np.array([[int(h, 16) for h in row] for row in p["w"]], dtype=np.uint32)
    s = np.array(p["scales"], dtype=np.uint16)
    b = np.array(p["biases"], dtype=np.uint16)
    x = np.array(p["x"], dtype=np.uint16)
    return w, s, b, x


PROBLEMS = [pytest.param(p, id=p["name"]) for p in GOLDEN["problems"]]


# --------------------------------------------------------------- known answers

def test_unpack_known_answers(oracle):
    for case in GOLDEN["known_answers"]["unpack"]:
        w = np.array([int(case["word"], 16)], dtype=np.uint32)
        assert oracle.unpack(w).tolist() == case["q"]
        q = np.empty(8, dtype=np.uint8)
        oracle.lib().imo_unpack(oracle._p(w), oracle._p(q), 1)
        assert q.tolist() == case["q"]
        assert oracle.pack(np.array(case["q"], dtype=np.uint8)).tolist() == w.tolist()


def test_bf16_rounding_known_answers(oracle):
    for case in GOLDEN["known_answers"]["bf16_round"]:
        f = np.array([int(case["f32"], 16)], dtype=np.uint32).view(np.float32)
        want = int(case["bf16"], 16)
        assert int(oracle.f32_to_bf16(f)[0]) == want, case
        assert int(oracle.lib().imo_f32_to_bf16(float(f[0]))) == want or np.isnan(f[0]), case


def test_bf16_rounding_matches_torch():
    import torch

    from oracle import oracle as o
    rng = np.random.default_rng(7)
    u = rng.integers(0, 2**32, size=200_000, dtype=np.uint64).astype(np.uint32)
    u[:1000] = (u[:1000] & 0xFFFF0000) | 0x8000  # exact ties
    f = u.view(np.float32)
    finite = np.isfinite(f)
    ours = o.f32_to_bf16(f[finite])
    theirs = torch.from_numpy(f[finite].copy()).to(torch.bfloat16).view(torch.int16).numpy()
    assert np.array_equal(ours, theirs.view(np.uint16))
    c = np.empty(int(finite.sum()), dtype=np.uint16)
    ff = np.ascontiguousarray(f[finite])
    o.lib().imo_f32_to_bf16_array(o._p(ff), o._p(c), ff.size)
    assert np.array_equal(c, ours)


def test_bf16_widening_is_exact(oracle):
    h = np.arange(0, 2**16, dtype=np.uint16)
    f = oracle.bf16_to_f32(h)
    back = oracle.f32_to_bf16(f)
    nan = np.isnan(f)
    assert np.array_equal(back[~nan], h[~nan])
    c = np.empty(h.size, dtype=np.float32)
    oracle.lib().imo_bf16_to_f32_array(oracle._p(h), oracle._p(c), h.size)
    assert np.array_equal(c.view(np.uint32), f.view(np.uint32))


def test_bf16_ulp(oracle):
    assert oracle.bf16_ulp(np.array([1.0]))[0] == 2.0 ** -7
    assert oracle.bf16_ulp(np.array([1.5]))[0] == 2.0 ** -7
    assert oracle.bf16_ulp(np.array([-6.0]))[0] == 2.0 ** -5
    assert oracle.bf16_ulp(np.array([0.75]))[0] == 2.0 ** -8


# ------------------------------------------------------------ golden problems

@pytest.mark.parametrize("p", PROBLEMS)
def test_dequant_is_bit_exact_to_the_exact_value(oracle, p):
    w, s, b, _ = _arrays(p)
    want = np.array(p["dequant_f32"], dtype=np.float32)
    assert np.array_equal(oracle.dequant_f32(w, s, b).view(np.uint32), want.view(np.uint32))
    assert np.array_equal(oracle.dequant_np(w, s, b).view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("p", PROBLEMS)
def test_f64_product_matches_exact(oracle, p):
    w, s, b, x = _arrays(p)
    y, mag = oracle.qmv_f64(w, s, b, x)
    exact = np.array(p["y_f64"])
    assert np.all(np.abs(y - exact) <= 1e-12 * mag + 1e-300)


@pytest.mark.parametrize("p", PROBLEMS)
@pytest.mark.parametrize("which", ["dequant_f32", "rowkernel", "mlx8"])
def test_fp32_restatements_within_the_parity_bound(oracle, p, which):
    w, s, b, x = _arrays(p)
    exact = np.array(p["y_f64"])
    _, mag = oracle.qmv_f64(w, s, b, x)
    if which == "dequant_f32":
        y = oracle.f32_to_bf16(oracle.qmv_dequant_f32(w, s, b, x))
    elif which == "rowkernel":
        y = oracle.qmv_rowkernel(w, s, b, x)
    else:
        y = oracle.qmv_mlx(w, s, b, x, values_per_thread=8)
    v = oracle.check_bf16(y, exact, mag)
    assert v.ok, v.detail
    # where the exact value is well away from a rounding boundary, bf16 agrees exactly
    want = np.array(p["y_bf16"], dtype=np.uint16)
    assert np.mean(y == want) > 0.9


def test_fast_order_restatement_needs_k_multiple_of_512(oracle):
    pr = oracle.synthetic(16, 1024, 2, seed=5)
    y64, mag = oracle.qmv_f64(pr.w, pr.s, pr.b, pr.x)
    y = oracle.qmv_mlx(pr.w, pr.s, pr.b, pr.x, values_per_thread=16)
    assert oracle.check_bf16(y, y64, mag).ok


# ------------------------------------------------------- planted mistakes fail

def _mutant_dequant(w, s, b, mode, oracle):
    q = oracle.unpack(w).astype(np.float64)
    if mode == "high_nibble_first":
        q = q.reshape(q.shape[0], -1, 8)[:, :, ::-1].reshape(q.shape[0], -1)
    sf = np.repeat(oracle.bf16_to_f32(s).astype(np.float64), 64, axis=-1)
    bf = np.repeat(oracle.bf16_to_f32(b).astype(np.float64), 64, axis=-1)
    if mode == "no_bias":
        bf = bf * 0
    if mode == "group_index_transposed":
        g = s.shape[1]
        idx = (np.arange(q.shape[1]) % g) if g > 1 else np.zeros(q.shape[1], dtype=int)
        sf = oracle.bf16_to_f32(s).astype(np.float64)[:, idx]
        bf = oracle.bf16_to_f32(b).astype(np.float64)[:, idx]
    if mode == "bias_sign":
        bf = -bf
    return (sf * q + bf).astype(np.float32)


@pytest.mark.parametrize("mode", ["high_nibble_first", "no_bias", "group_index_transposed",
                                  "bias_sign"])
def test_planted_mistakes_are_caught_by_the_fixtures(oracle, mode):
    caught = 0
    for p in GOLDEN["problems"]:
        w, s, b, x = _arrays(p)
        got = _mutant_dequant(w, s, b, mode, oracle)
        want = np.array(p["dequant_f32"], dtype=np.float32)
        caught += int(not np.array_equal(got.view(np.uint32), want.view(np.uint32)))
    assert caught >= 3, f"{mode} slipped through {len(GOLDEN['problems']) - caught} fixtures"


# ----------------------------------------------------------- special cases

def test_zero_nibbles_reduce_to_bias_times_group_sums(oracle):
    pr = oracle.synthetic(32, 640, 2, seed=11)
    w = np.zeros_like(pr.w)
    y, _ = oracle.qmv_f64(w, pr.s, pr.b, pr.x)
    xs = oracle.bf16_to_f32(pr.x).astype(np.float64).reshape(2, -1, 64).sum(-1)  # (M, G)
    want = xs @ oracle.bf16_to_f32(pr.b).astype(np.float64).T
    assert np.allclose(y, want, rtol=1e-12, atol=1e-12)


def test_zero_scales_reduce_to_bias_times_group_sums(oracle):
    pr = oracle.synthetic(16, 256, 1, seed=12)
    s = np.zeros_like(pr.s)
    y, _ = oracle.qmv_f64(pr.w, s, pr.b, pr.x)
    xs = oracle.bf16_to_f32(pr.x).astype(np.float64).reshape(1, -1, 64).sum(-1)
    want = xs @ oracle.bf16_to_f32(pr.b).astype(np.float64).T
    assert np.allclose(y, want, rtol=1e-12, atol=1e-12)


def test_one_hot_input_selects_a_dequantised_column(oracle):
    pr = oracle.synthetic(24, 512, 1, seed=13)
    d = oracle.dequant_f32(pr.w, pr.s, pr.b)
    for col in (0, 63, 64, 511):
        x = np.zeros((1, 512), dtype=np.uint16)
        x[0, col] = 0x3F80
        y32 = oracle.qmv_dequant_f32(pr.w, pr.s, pr.b, x)
        assert np.array_equal(y32[0], d[:, col])
        yr = oracle.qmv_rowkernel(pr.w, pr.s, pr.b, x, out_f32=True)
        assert np.array_equal(yr[0], d[:, col])


def test_single_group_product_is_scale_times_dot_plus_bias_times_sum(oracle):
    pr = oracle.synthetic(8, 64, 1, seed=14)
    q = oracle.unpack(pr.w).astype(np.float64)
    xv = oracle.bf16_to_f32(pr.x[0]).astype(np.float64)
    want = oracle.bf16_to_f32(pr.s[:, 0]) * (q @ xv) + oracle.bf16_to_f32(pr.b[:, 0]) * xv.sum()
    y, _ = oracle.qmv_f64(pr.w, pr.s, pr.b, pr.x)
    assert np.allclose(y[0], want, rtol=1e-12)


def test_f64_product_matches_numpy_matmul_of_dequantised_weights(oracle):
    pr = oracle.synthetic(64, 1280, 3, seed=15)
    d = oracle.dequant_np(pr.w, pr.s, pr.b).astype(np.float64)
    want = oracle.bf16_to_f32(pr.x).astype(np.float64) @ d.T
    y, _ = oracle.qmv_f64(pr.w, pr.s, pr.b, pr.x)
    assert np.allclose(y, want, rtol=1e-11, atol=1e-9)


def test_linearity_in_x(oracle):
    pr = oracle.synthetic(32, 512, 2, seed=16)
    x2 = oracle.f32_to_bf16(oracle.bf16_to_f32(pr.x[0]) * 2.0)[None]
    y1, _ = oracle.qmv_f64(pr.w, pr.s, pr.b, pr.x[:1])
    y2, _ = oracle.qmv_f64(pr.w, pr.s, pr.b, x2)
    assert np.allclose(2 * y1, y2, rtol=1e-12)


def test_rowkernel_is_batch_invariant(oracle):
    pr = oracle.synthetic(40, 2560, 3, seed=17)
    many = oracle.qmv_rowkernel(pr.w, pr.s, pr.b, pr.x)
    for m in range(3):
        one = oracle.qmv_rowkernel(pr.w, pr.s, pr.b, pr.x[m:m + 1])
        assert np.array_equal(one[0], many[m])


@pytest.mark.parametrize("n,k,m", [(96, 2560, 1), (64, 3840, 2), (32, 4096, 1), (16, 9728, 1)])
def test_restatements_agree_at_path_shapes(oracle, n, k, m):
    pr = oracle.synthetic(n, k, m, seed=18 + k)
    y64, mag = oracle.qmv_f64(pr.w, pr.s, pr.b, pr.x)
    for y in (oracle.qmv_rowkernel(pr.w, pr.s, pr.b, pr.x),
              oracle.qmv_mlx(pr.w, pr.s, pr.b, pr.x),
              oracle.f32_to_bf16(oracle.qmv_dequant_f32(pr.w, pr.s, pr.b, pr.x))):
        v = oracle.check_bf16(y, y64, mag)
        assert v.ok, v.detail
    v = oracle.check_f32(oracle.qmv_rowkernel(pr.w, pr.s, pr.b, pr.x, out_f32=True), y64, mag)
    assert v.ok, v.detail


def test_check_bf16_rejects_a_two_ulp_error(oracle):
    ref = np.array([[1.0, 3.0, -0.75]])
    mag = np.abs(ref)
    good = oracle.f32_to_bf16(ref.astype(np.float32))
    assert oracle.check_bf16(good, ref, mag).ok
    bad = good.copy()
    bad[0, 1] += 2
    assert not oracle.check_bf16(bad, ref, mag).ok


def test_check_f32_rejects_a_planted_error(oracle):
    """check_f32 passes the fp32 dequantise-then-matmul reference and rejects it with one
    output moved by 1e-4 of max|ref| (far inside the 1e-3 max-relative bound, so the
    per-output summation allowance is what catches it) and with one output scaled by 1.01."""
    pr = oracle.synthetic(64, 2560, 2, seed=oracle.SEED_BASE + 42)
    ref, mag = oracle.qmv_f64(pr.w, pr.s, pr.b, pr.x)
    y = oracle.qmv_dequant_f32(pr.w, pr.s, pr.b, pr.x)
    assert oracle.check_f32(y, ref, mag).ok
    i = int(np.argmax(np.abs(ref[0])))
    nudged = y.copy()
    nudged[0, i] += np.float32(1e-4 * np.max(np.abs(ref)))
    v = oracle.check_f32(nudged, ref, mag)
    assert not v.ok and v.violations == 1, v.detail
    scaled = y.copy()
    scaled[1, 7] *= np.float32(1.01)
    assert not oracle.check_f32(scaled, ref, mag).ok


def test_literal_bar_counts_and_the_cancellation_exemption(oracle):
    """check_bf16_literal: the fp32 reference rounded to bf16 has no violations; the exactly
    rounded product misses the literal bar only at deep cancellations (the floor reported
    beside every GPU count); a planted two-ulp error at an ordinary output fails; the same
    error at an output below the cancellation threshold is counted but exempt."""
    pr = oracle.synthetic(3072, 3840, 4, seed=oracle.SEED_BASE + 43)
    ref, mag = oracle.qmv_f64(pr.w, pr.s, pr.b, pr.x)
    ref32 = oracle.qmv_dequant_f32(pr.w, pr.s, pr.b, pr.x)
    own = oracle.check_bf16_literal(oracle.f32_to_bf16(ref32), ref32, ref, mag)
    assert own.ok and own.violations == 0
    exact = oracle.f32_to_bf16(ref.astype(np.float32))
    v = oracle.check_bf16_literal(exact, ref32, ref, mag)
    assert v.ok and v.violations == v.exact_violations, v.detail
    big = np.unravel_index(int(np.argmax(np.abs(ref))), ref.shape)
    bad = oracle.f32_to_bf16(ref32).copy()
    bad[big] += 2
    v = oracle.check_bf16_literal(bad, ref32, ref, mag)
    assert not v.ok and v.outside == 1, v.detail
    tiny = np.unravel_index(int(np.argmin(np.abs(ref) / mag)), ref.shape)
    assert abs(ref[tiny]) < oracle.LITERAL_CANCELLATION * mag[tiny]
    bad = oracle.f32_to_bf16(ref32).copy()
    bad[tiny] += 2
    v = oracle.check_bf16_literal(bad, ref32, ref, mag)
    assert v.ok and v.violations == 1, v.detail


def test_synthetic_distribution(oracle):
    pr = oracle.synthetic(256, 2560, 2, seed=oracle.SEED_BASE + 1)
    q = oracle.unpack(pr.w)
    counts = np.bincount(q.ravel(), minlength=16)
    assert counts.min() > 0.9 * q.size / 16
    s = oracle.bf16_to_f32(pr.s)
    b = oracle.bf16_to_f32(pr.b)
    assert 0.0049 < s.min() and s.max() < 0.0201
    assert -0.1001 < b.min() and b.max() < 0.1001
    x = oracle.bf16_to_f32(pr.x)
    assert abs(float(x.mean())) < 0.05 and 0.95 < float(x.std()) < 1.05


def test_gather_oracle_is_the_per_pair_product(oracle):
    """The gather restatement: pair p equals the qmv of expert idx[p] on row p // rows_per_x
    (the down form rows_per_x = 1 and the gate/up broadcast), and an index outside the
    stack gives a zero row.  Planted mistake: reading row p instead of p // rows_per_x
    changes the broadcast result."""
    rng = np.random.default_rng(5)
    e, n, k = 5, 12, 128
    probs = [oracle.synthetic(n, k, 1, seed=oracle.SEED_BASE + 300 + i) for i in range(e)]
    w = np.stack([p.w for p in probs])
    s = np.stack([p.s for p in probs])
    b = np.stack([p.b for p in probs])
    x = oracle.f32_to_bf16(rng.standard_normal((3, k)).astype(np.float32))
    idx = np.array([4, 0, 2, 2, 7, 1], dtype=np.int64)
    for xs in (1, 2):
        rows = x if xs == 2 else np.concatenate([x, x])
        ref, mag = oracle.gather_qmv_f64(w, s, b, rows, idx, rows_per_x=xs)
        for p, ex in enumerate(idx):
            if ex >= e:
                assert not ref[p].any() and not mag[p].any()
                continue
            want, _ = oracle.qmv_f64(w[ex], s[ex], b[ex], rows[p // xs].reshape(1, -1))
            assert np.array_equal(ref[p], want[0])
    # the broadcast reads row p // 2: pairs 0 and 1 share row 0, so a per-pair read differs
    ref2, _ = oracle.gather_qmv_f64(w, s, b, x, idx[:2], rows_per_x=2)
    wrong, _ = oracle.qmv_f64(w[idx[1]], s[idx[1]], b[idx[1]], x[1].reshape(1, -1))
    assert not np.array_equal(ref2[1], wrong[0])
