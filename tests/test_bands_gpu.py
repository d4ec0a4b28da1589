"""GPU parity of imq_qmv_residual_bands, one projection over bands of 32 weight rows and the
whole K with the residual epilogue (the batched decode step's o and down projections),
through the C ABI.

For each shape: y = x W^T is never written, so it is read back from a call on h = 0 (h_new
is then bf16(y) exactly), and bf16(y) must be within one bf16 ulp (plus the fp32 summation
allowance) of the oracle's exact product; on a random h, h_new = h + bf16(y) in fp32.
x' = bf16(h_new * w) bit for bit against torch, each band's per-row sum of squares within
fp32 rounding of the float64 sum over its 32 columns.  x in the 32-row tile layout gives the
same bits as x in rows; repeated calls give the same bits.  Shapes: the decode step's o and
down (K = 4096: one 4-group chunk per wavefront; K = 9728: three for the first six), a ragged
N, one row, and K = 256 (one chunk: fifteen wavefronts without work)."""

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


@pytest.mark.parametrize("n,k,m", [(2560, 4096, 32), (2560, 9728, 32), (2560, 9728, 5), (1000, 2048, 9),
                                   (2560, 4096, 1), (96, 256, 3)])
def test_residual_bands_match_the_oracle(native, oracle, n, k, m):
    p = oracle.synthetic(n, k, m, seed=oracle.SEED_BASE + 3000 + m)
    w, s, b, x = to_device(p)
    g = torch.Generator(device="cuda")
    g.manual_seed(3000 + n + m)
    h = torch.randn((m, n), device="cuda", generator=g) * 0.25
    wn = (torch.rand(n, device="cuda", generator=g) + 0.5).to(torch.bfloat16)
    announce("residual bands", n, k, m)
    outs = []
    for tiled in (False, True, False):
        h1 = h.clone()
        xo = torch.full((m, n), 7.0, dtype=torch.bfloat16, device="cuda")
        st = native.NormStats(m, n, "cuda")
        st.ssq.fill_(-1.0)
        xin = native.tile_rows(x) if tiled else x
        native.qmv_residual_bands((w, s, b), xin, m, h1, next_norm=wn, x_out=xo, stats_out=st, tiled=tiled)
        outs.append((h1, xo, st))
    torch.cuda.synchronize()
    (h1, xo, st), (h2, xo2, st2), (h3, xo3, st3) = outs
    bands = -(-n // 32)
    assert st.tiles == bands
    for hh, xx, ss in ((h2, xo2, st2), (h3, xo3, st3)):  # tiled x and a second call: same bits
        assert torch.equal(hh, h1) and torch.equal(xx, xo)
        assert torch.equal(ss.ssq[:, :bands], st.ssq[:, :bands])
    # bf16(y) itself from a call on h = 0, against the oracle; h_new = h + bf16(y) in fp32
    y = torch.zeros((m, n), device="cuda")
    native.qmv_residual_bands((w, s, b), x, m, y)
    torch.cuda.synchronize()
    ybits = oracle.f32_to_bf16(y.cpu().numpy())
    assert torch.equal(y, y.to(torch.bfloat16).float()), "the update is one bf16 value"
    ref, mag = oracle.qmv_f64(p.w, p.s, p.b, p.x)
    v = oracle.check_bf16(ybits, ref, mag)
    assert v.ok, v.detail
    assert torch.equal(h1, h + y)
    # x' = bf16(h_new * w), the bands' sums of squares
    assert torch.equal(xo, (h1 * wn.float()).to(torch.bfloat16))
    hn = h1.double().cpu().numpy()
    pad = np.zeros((m, bands * 32))
    pad[:, :n] = hn
    want = (pad.reshape(m, bands, 32) ** 2).sum(axis=2)
    got = st.ssq[:, :bands].double().cpu().numpy()
    assert np.allclose(got, want, rtol=2e-6, atol=0), float(np.max(np.abs(got - want) / np.maximum(want, 1e-30)))


def test_residual_bands_h_only(native, oracle):
    n, k, m = 2560, 4096, 8
    p = oracle.synthetic(n, k, m, seed=oracle.SEED_BASE + 3100)
    w, s, b, x = to_device(p)
    h = torch.zeros((m, n), device="cuda")
    announce("residual bands, h only", n, k, m)
    native.qmv_residual_bands((w, s, b), native.tile_rows(x), m, h, tiled=True)
    y = h.clone()
    torch.cuda.synchronize()
    ref, mag = oracle.qmv_f64(p.w, p.s, p.b, p.x)
    v = oracle.check_bf16(oracle.f32_to_bf16(y.cpu().numpy()), ref, mag)
    assert v.ok, v.detail
