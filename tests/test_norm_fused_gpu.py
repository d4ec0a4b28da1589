"""GPU parity of the RMSNorm folded into the projections (imq_rmsnorm_prescale,
imq_qmv_norm, imq_qmv_gate_up_silu_norm), through the C ABI.

rms_norm(h) W^T = inv * ((h * w) W^T) row by row, inv = 1 / sqrt(sum h^2 / dim + eps): the
producer writes x' = bf16(h * w) and partial sums of squares, the consumer scales its rows.

* prescale: x' = bf16(h * w) and h += delta bit-exact against torch, the row's sum of
  squares within fp32 rounding of the float64 sum.
* input norm with partials whose sum makes inv exactly 1/2: every output is half the plain
  projection's, bit for bit (the scaling by a power of two commutes with the rounding), at
  the decode shapes (q/k/v, o and down at 5 and 32 rows) and for the gate/up launch against
  silu_mul of the halved grouped outputs.
* input norm with random partials: within the oracle's bf16 bar of inv * (x' W^T), inv from
  the float64 sum (plus 2^-18 relative for the fp32 sum of up to 128 partials).
* residual epilogue: h_new = h + bf16(y) bit-exact with y the plain projection's output, x' =
  bf16(h_new * w) bit-exact, the per-tile sums of squares within fp32 rounding; h only
  without a weight; a small forced plan (K = 512, 8 rows, whole-K tiles) against the oracle.
* refusals: a residual epilogue over two weights, partial counts outside 1..128, ld not a
  multiple of 4.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from tests.conftest import gpu_available
from tests.gpu_util import announce, bf16_bits, to_device

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not gpu_available(), reason="needs a ROCm GPU")]


@pytest.fixture(scope="module")
def native():
    from ironmule_amd import _native
    code, arch, _ = _native.device_check()
    assert code == 0, f"device {arch} is not supported"
    return _native


def _stats(native, rows, dim, tiles, values):
    """NormStats over `rows` rows with `tiles` partials per row set to `values` (rows, tiles)."""
    st = native.NormStats(rows, dim, "cuda")
    if tiles > st.ld:
        st.ld = -(-tiles // 4) * 4
        st.ssq = torch.zeros((rows, st.ld), dtype=torch.float32, device="cuda")
    st.ssq.zero_()
    st.ssq[:, :tiles] = torch.as_tensor(np.asarray(values, np.float32), device="cuda")
    st.tiles = tiles
    return st


def _weights(oracle, shapes, m, seed):
    probs = [oracle.synthetic(n, k, m, seed=seed + i) for i, (n, k) in enumerate(shapes)]
    x = probs[0].x
    probs = [oracle.Problem(p.w, p.s, p.b, x, 0) for p in probs]
    dev = [to_device(p) for p in probs]
    return probs, [d[:3] for d in dev], dev[0][3]


def test_prescale(native):
    g = torch.Generator(device="cuda")
    g.manual_seed(11)
    for b, dim, with_delta in ((1, 2560, False), (32, 2560, True), (5, 320, True)):
        announce("rmsnorm prescale", b, dim, with_delta)
        h = torch.randn((b, dim), device="cuda", generator=g) * 3
        w = (torch.rand(dim, device="cuda", generator=g) + 0.5).to(torch.bfloat16)
        delta = torch.randn((b, dim), device="cuda", generator=g).to(torch.bfloat16) if with_delta else None
        h0 = h.clone()
        out = torch.empty((b, dim), dtype=torch.bfloat16, device="cuda")
        st = native.NormStats(b, dim, "cuda")
        native.rmsnorm_prescale(h, w, out, st, delta=delta)
        torch.cuda.synchronize()
        hn = h0 + delta.float() if with_delta else h0
        assert torch.equal(h, hn)
        assert torch.equal(out, (hn * w.float()).to(torch.bfloat16))
        ss = (hn.double() ** 2).sum(dim=1)
        assert st.tiles == 1
        assert torch.allclose(st.ssq[:, 0].double(), ss, rtol=2e-6, atol=0)


# Partials summing to exactly 4 * dim: inv = 1 / sqrt(4) = 1/2 with eps = 0.
def _half_stats(native, m, dim, tiles):
    return _stats(native, m, dim, tiles, np.full((m, tiles), 4.0 * dim / tiles))


@pytest.mark.parametrize("shapes,m", [
    ([(4096, 2560), (1024, 2560), (1024, 2560)], 32),
    ([(4096, 2560), (1024, 2560), (1024, 2560)], 5),
    ([(2560, 4096)], 32), ([(2560, 9728)], 32), ([(2560, 9728)], 7),
])
def test_input_norm_halves_the_plain_projection(native, oracle, shapes, m):
    _, weights, x = _weights(oracle, shapes, m, oracle.SEED_BASE + 2000 + m)
    announce("input norm = plain / 2", shapes, m)
    plain = native.qmv_grouped(weights, [x] * len(weights))
    st = _half_stats(native, m, 2560, 40)
    got = native.qmv_norm(weights, x, norm_in=st, eps=0.0)
    again = native.qmv_norm(weights, x, norm_in=st, eps=0.0)
    torch.cuda.synchronize()
    for p, y, y2 in zip(plain, got, again):
        assert torch.equal(y, (p.float() * 0.5).to(torch.bfloat16))
        assert torch.equal(y, y2)


@pytest.mark.parametrize("shapes,m,tiles", [
    ([(4096, 2560), (1024, 2560), (1024, 2560)], 32, 40),
    ([(2560, 4096)], 6, 1), ([(1000, 512)], 8, 64), ([(2560, 9728)], 32, 13),
    ([(640, 2560)], 1, 40),
])
def test_input_norm_matches_oracle(native, oracle, shapes, m, tiles):
    probs, weights, x = _weights(oracle, shapes, m, oracle.SEED_BASE + 2100 + m)
    rng = np.random.default_rng(2100 + m + tiles)
    dim, eps = 2560, 1e-6
    vals = rng.uniform(0.5, 3.0, size=(m, tiles)).astype(np.float32) * dim / tiles
    st = _stats(native, m, dim, tiles, vals)
    announce("input norm vs oracle", shapes, m, tiles)
    got = native.qmv_norm(weights, x, norm_in=st, eps=eps)
    torch.cuda.synchronize()
    inv = 1.0 / np.sqrt(vals.astype(np.float64).sum(axis=1) / dim + eps)
    for pr, y in zip(probs, got):
        ref, mag = oracle.qmv_f64(pr.w, pr.s, pr.b, pr.x)
        ref = ref * inv[:, None]
        v = oracle.check_bf16(bf16_bits(y), ref, mag * inv[:, None] + 4.0 * np.abs(ref))
        assert v.ok, v.detail


@pytest.mark.parametrize("n,k,m", [(9728, 2560, 32), (9728, 2560, 5), (1000, 512, 9), (16416, 1024, 8),
                                   (9728, 2560, 3), (1000, 512, 1), (1004, 2048, 32), (2000, 3072, 17),
                                   (9728, 2560, 1)])
def test_gate_up_norm_halves(native, oracle, n, k, m):
    """With the input norm folded in the launch takes any M from 1 (the decode step folds
    its norms from 3 requests); without it, from 5.  K of 4, 8, 10 or 12 times 256 takes the
    row-band kernel (one workgroup per CU, no workspace; 16416 rows: two rounds, 1004: a
    last band of 4 rows), K = 512 the staged kernel with the last round's K-parts."""
    pg = oracle.synthetic(n, k, m, seed=oracle.SEED_BASE + 2200 + m)
    pu = oracle.synthetic(n, k, m, seed=oracle.SEED_BASE + 2201 + m)
    pu = oracle.Problem(pu.w, pu.s, pu.b, pg.x, 0)
    dg, du = to_device(pg), to_device(pu)
    gate, up, x = dg[:3], du[:3], dg[3]
    announce("gate/up norm = silu(g/2) * u/2", n, k, m)
    st = _half_stats(native, m, 2560, 40)
    out = native.gate_up_silu_norm(gate, up, x, torch.empty((m, n), dtype=torch.bfloat16, device="cuda"),
                                   st, 0.0)
    whole = native.gate_up_silu_norm(gate, up, x, torch.empty((m, n), dtype=torch.bfloat16, device="cuda"),
                                     st, 0.0, split_tail=False)
    again = native.gate_up_silu_norm(gate, up, x, torch.empty((m, n), dtype=torch.bfloat16, device="cuda"),
                                     st, 0.0)
    if m >= 5:
        plain = native.gate_up_silu(gate, up, x, torch.empty((m, n), dtype=torch.bfloat16, device="cuda"))
    else:
        with pytest.raises(native.NativeError):
            native.gate_up_silu(gate, up, x, torch.empty((m, n), dtype=torch.bfloat16, device="cuda"))
        plain = native.gate_up_silu_norm(gate, up, x, torch.empty((m, n), dtype=torch.bfloat16, device="cuda"),
                                         _stats(native, m, 2560, 40, np.full((m, 40), 64.0, np.float32)),
                                         0.0)  # inv = 1: no scaling
    torch.cuda.synchronize()
    assert torch.equal(out, again)  # the sums add in a fixed order
    if k // 256 in (4, 8, 10, 12):  # the row-band kernel either way
        assert torch.equal(out, whole)
    else:  # the tiles of whole rounds over the CUs are whole tiles either way: the same bits
        cus = native.device_check()[2]
        tiles = -(-n // 32)
        cut = 32 * (tiles - tiles % cus) if tiles > cus else n
        assert torch.equal(out[:, :cut], whole[:, :cut])
    # against the oracle (every column, the K-parts of the last round's tiles included):
    # each projection within one bf16 ulp (plus the summation allowance) of its exact value,
    # then SiLU (slope <= 1.1) and one more rounding
    g64, mg = oracle.qmv_f64(pg.w, pg.s, pg.b, pg.x)
    u64, mu = oracle.qmv_f64(pu.w, pu.s, pu.b, pu.x)
    g64, u64, mg, mu = g64 / 2, u64 / 2, mg / 2, mu / 2
    eg = oracle.bf16_ulp(g64) + 2.0 ** -20 * mg
    eu = oracle.bf16_ulp(u64) + 2.0 ** -20 * mu
    sg = g64 / (1.0 + np.exp(-g64))
    ref = sg * u64
    bound = oracle.bf16_ulp(ref) + 1.1 * eg * (np.abs(u64) + eu) + np.abs(sg) * eu
    for t in (out, whole):
        got = oracle.bf16_to_f32(bf16_bits(t)).astype(np.float64)
        assert (np.abs(got - ref) <= bound).all(), float(np.max(np.abs(got - ref) / bound))
    assert not torch.equal(out, plain)  # the scaling took effect


@pytest.mark.parametrize("n,k,m", [(2560, 4096, 32), (2560, 9728, 32), (2560, 4096, 5)])
def test_residual_epilogue(native, oracle, n, k, m):
    probs, weights, x = _weights(oracle, [(n, k)], m, oracle.SEED_BASE + 2300 + m)
    g = torch.Generator(device="cuda")
    g.manual_seed(2300 + m)
    h = torch.randn((m, n), device="cuda", generator=g) * 4
    w = (torch.rand(n, device="cuda", generator=g) + 0.5).to(torch.bfloat16)
    announce("residual epilogue", n, k, m)
    (y,) = native.qmv_grouped(weights, [x])
    h1 = h.clone()
    xo = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
    st = native.NormStats(m, n, "cuda")
    out = native.qmv_norm(weights, x, residual=h1, next_norm=w, x_out=xo, stats_out=st)
    h2 = h.clone()
    native.qmv_norm(weights, x, residual=h2)  # h only
    torch.cuda.synchronize()
    assert out == []
    hn = h + y.float()
    assert torch.equal(h1, hn)
    assert torch.equal(h2, hn)
    assert torch.equal(xo, (hn * w.float()).to(torch.bfloat16))
    tiles = n // 64
    assert st.tiles == tiles
    ss = (hn.double() ** 2).reshape(m, tiles, 64).sum(dim=2)
    assert torch.allclose(st.ssq[:, :tiles].double(), ss, rtol=2e-6, atol=0)


@pytest.mark.parametrize("n,k,m", [(2560, 4096, 32), (2560, 9728, 32), (2560, 4096, 5),
                                   (2560, 9728, 3), (1000, 4096, 8), (2560, 4096, 1)])
def test_residual_planes_same_bits(native, oracle, n, k, m):
    """The projection as K-range planes (imq_qmv_norm_planes) and the residual epilogue as a
    launch of its own (imq_residual_planes) give the bits of imq_qmv_norm's residual epilogue:
    h, x' and the per-tile sums of squares, with and without the next norm (a ragged last
    tile at N = 1000)."""
    probs, weights, x = _weights(oracle, [(n, k)], m, oracle.SEED_BASE + 2350 + m)
    g = torch.Generator(device="cuda")
    g.manual_seed(2350 + m)
    h = torch.randn((m, n), device="cuda", generator=g) * 4
    w = (torch.rand(n, device="cuda", generator=g) + 0.5).to(torch.bfloat16)
    count = native.residual_split_planes(weights[0], x)
    announce("residual planes", n, k, m, count)
    assert 1 <= count <= native.RESIDUAL_MAX_PLANES
    fused_h, fused_x = h.clone(), torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
    fused_st = native.NormStats(m, n, "cuda")
    native.qmv_norm(weights, x, residual=fused_h, next_norm=w, x_out=fused_x, stats_out=fused_st)
    planes = native.ResidualPlanes(m, n, "cuda")
    assert native.qmv_residual_planes(weights[0], x, planes) == count
    two_h, two_x = h.clone(), torch.full((m, n), 7, dtype=torch.bfloat16, device="cuda")
    two_st = native.NormStats(m, n, "cuda")
    native.residual_planes(planes, two_h, next_norm=w, x_out=two_x, stats_out=two_st)
    only_h = h.clone()
    native.residual_planes(planes, only_h)  # h only
    torch.cuda.synchronize()
    assert torch.equal(two_h, fused_h)
    assert torch.equal(only_h, fused_h)
    assert torch.equal(two_x, fused_x)
    tiles = -(-n // 64)
    assert two_st.tiles == fused_st.tiles == tiles
    assert torch.equal(two_st.ssq[:, :tiles], fused_st.ssq[:, :tiles])
    # and the planes hold the projection: their sum in plane order, rounded, is within the
    # oracle's bar
    tot = torch.zeros((m, n), device="cuda")
    for sp in range(count):
        tot = tot + planes.view()[sp]
    v, lit = oracle.check_bf16_both(bf16_bits(tot.to(torch.bfloat16)), probs[0].w, probs[0].s, probs[0].b,
                                    probs[0].x)
    assert v.ok and lit.ok, (v.detail, lit.detail)


def test_residual_epilogue_forced_plan_matches_oracle(native, oracle):
    n, k, m = 256, 512, 8  # the usual plan would not take the direct-to-LDS kernel here
    probs, weights, x = _weights(oracle, [(n, k)], m, oracle.SEED_BASE + 2400)
    h = torch.zeros((m, n), device="cuda")
    w = torch.ones(n, dtype=torch.bfloat16, device="cuda")
    xo = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
    st = native.NormStats(m, n, "cuda")
    announce("residual epilogue forced plan", n, k, m)
    native.qmv_norm(weights, x, residual=h, next_norm=w, x_out=xo, stats_out=st)
    torch.cuda.synchronize()
    # h was zero: h_new = bf16(y) exactly, and x' = bf16(h_new * 1) = y
    v, lit = oracle.check_bf16_both(bf16_bits(xo), probs[0].w, probs[0].s, probs[0].b, probs[0].x)
    assert v.ok and lit.ok, (v.detail, lit.detail)
    assert torch.equal(h, xo.float())


def test_refusals(native, oracle):
    from ironmule_amd._native import NativeError, NormIn, Problem, lib
    import ctypes
    _, weights, x = _weights(oracle, [(512, 512), (512, 512)], 8, oracle.SEED_BASE + 2500)
    announce("fused norm refusals")
    h = torch.zeros((8, 512), device="cuda")
    with pytest.raises(ValueError):
        native.qmv_norm(weights, x, residual=h)
    for tiles, ld in ((0, 4), (129, 132), (5, 6)):
        st = native.NormStats(8, 512, "cuda")
        nin = NormIn(st.ssq.data_ptr(), tiles, ld, 512, 1e-6)
        probs = (Problem * 1)()
        y = torch.empty((8, 512), dtype=torch.bfloat16, device="cuda")
        w, s, b = weights[0]
        probs[0] = Problem(w.data_ptr(), s.data_ptr(), b.data_ptr(), x.data_ptr(), 512, y.data_ptr(), 512, 512, 512)
        code = lib().imq_qmv_norm(probs, 1, 8, 64, 4, ctypes.byref(nin), None, None, 0, None)
        assert code in (1, 2), (tiles, ld, code)
    pr = oracle.synthetic(64, 320, 8, seed=oracle.SEED_BASE + 2501)  # K % 256 != 0
    w3, s3, b3, x3 = to_device(pr)
    with pytest.raises(NativeError):
        native.qmv_norm([(w3, s3, b3)], x3, norm_in=native.NormStats(8, 512, "cuda"))


@pytest.mark.parametrize("m", [32, 5, 1])
def test_qkv_planes(native, oracle, m):
    """imq_qmv_norm_planes: the planes added in order equal the in-launch reduction (inv = 1/2
    exactly: half the plain projection, bit for bit, where that takes the same kernel; the
    oracle's bar at one row); then imq_attention_fused_planes gives
    the bits imq_attention_fused gives on those q/k/v rows, outputs and KV pools alike."""
    shapes = [(4096, 2560), (1024, 2560), (1024, 2560)]
    probs, weights, x = _weights(oracle, shapes, m, oracle.SEED_BASE + 2600 + m)
    announce("q/k/v planes", m)
    st = _half_stats(native, m, 2560, 40)
    planes = native.QkvPlanes(m, 32, 8, "cuda")
    count = native.qmv_norm_planes(weights, x, planes, norm_in=st, eps=0.0)
    plain = native.qmv_grouped(weights, [x] * 3)
    torch.cuda.synchronize()
    assert 1 <= count <= 4
    rows = []
    for i in range(3):
        pl = planes.view(i)
        tot = torch.zeros_like(pl[0])
        for s in range(count):
            tot = tot + pl[s]
        got = tot.to(torch.bfloat16)
        if m >= 5:  # the plain launch takes the same kernel and plan from 5 rows
            assert torch.equal(got, (plain[i].float() * 0.5).to(torch.bfloat16)), i
        else:  # one row takes the one-row VALU tile: the oracle's bar instead
            ref, mag = oracle.qmv_f64(probs[i].w, probs[i].s, probs[i].b, probs[i].x)
            v = oracle.check_bf16(bf16_bits(got), ref * 0.5, mag * 0.5)
            assert v.ok, (i, v.detail)
        rows.append(got)
    # the attention launch on the planes against the launch on the bf16 rows
    g = torch.Generator(device="cuda")
    g.manual_seed(2600 + m)
    slots_n, cap = max(m, 2), 96
    pools = [torch.randn((slots_n, 8, cap, 128), device="cuda", generator=g).to(torch.bfloat16) for _ in range(2)]
    qn = (torch.rand(128, device="cuda", generator=g) + 0.5).to(torch.bfloat16)
    kn = (torch.rand(128, device="cuda", generator=g) + 0.5).to(torch.bfloat16)
    positions = torch.tensor([(7 * i + 3) % cap for i in range(m)], dtype=torch.int32, device="cuda")
    slots = torch.arange(m, dtype=torch.int32, device="cuda") % slots_n
    ws = torch.empty(native.attention_workspace(m, 32, cap), dtype=torch.float32, device="cuda")
    outs, kps, vps = [], [], []
    for use_planes in (False, True):
        kp, vp = pools[0].clone(), pools[1].clone()
        out = torch.empty((m, 32 * 128), dtype=torch.bfloat16, device="cuda")
        cnt = torch.zeros(m * 8, dtype=torch.int32, device="cuda")
        if use_planes:
            native.attention_fused_planes(planes, qn, kn, positions, slots, kp, vp, out, cap, 1e6, 1e-6, ws, cnt)
        else:
            native.attention_fused(rows[0], rows[1], rows[2], qn, kn, positions, slots, kp, vp, out, cap,
                                   1e6, 1e-6, ws, cnt)
        torch.cuda.synchronize()
        outs.append(out)
        kps.append(kp)
        vps.append(vp)
    assert torch.equal(outs[0], outs[1])
    assert torch.equal(kps[0], kps[1]) and torch.equal(vps[0], vps[1])
