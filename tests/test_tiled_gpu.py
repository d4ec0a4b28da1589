"""GPU parity of the 32-row tile layout (IMQ_LD_TILED) in the batched decode launches: each
producer's tiled output is tile_rows of its output as rows, and each consumer gives the same
bits from a tiled x as from x in rows, through the C ABI.

* q/k/v planes (imq_qmv_norm_planes) and the o/down K-range planes (imq_qmv_norm_planes, one
  weight) from a tiled x; the residual epilogue (imq_residual_planes) and the row-band
  projection (imq_qmv_residual_bands) writing x' tiled;
* the gate/up launch (imq_qmv_gate_up_silu_norm) reading x and writing SiLU * up tiled;
* the planes attention (imq_attention_fused_planes) writing its output tiled.
At 32, 8 and 3 rows (rows past M are neither read nor written: the buffers start as 7.0)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from tests.conftest import gpu_available
from tests.gpu_util import announce, to_device

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not gpu_available(), reason="needs a ROCm GPU")]


@pytest.fixture(scope="module")
def native():
    from ironmule_amd import _native
    code, arch, _ = _native.device_check()
    assert code == 0, f"device {arch} is not supported"
    return _native


def _stats(native, m, dim, seed):
    st = native.NormStats(m, dim, "cuda")
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    st.ssq[:, :40] = torch.rand((m, 40), device="cuda", generator=g) * 100 + 10
    st.tiles = 40
    return st


def _untile(native, t, m, k):
    return native.untile_rows(t, m, k)


@pytest.mark.parametrize("m", [32, 8, 3])
def test_tiled_producers_and_consumers(native, oracle, m):
    seed = oracle.SEED_BASE + 3300 + m
    announce("tile layout", m)
    # q/k/v planes
    probs = [oracle.synthetic(n, 2560, m, seed=seed + i) for i, n in enumerate((4096, 1024, 1024))]
    x = to_device(probs[0])[3]
    weights = [to_device(oracle.Problem(p.w, p.s, p.b, probs[0].x, 0))[:3] for p in probs]
    xt = native.tile_rows(x)
    st = _stats(native, m, 2560, seed)
    a, b = native.QkvPlanes(m, 32, 8, "cuda"), native.QkvPlanes(m, 32, 8, "cuda")
    ca = native.qmv_norm_planes(weights, x, a, norm_in=st)
    cb = native.qmv_norm_planes(weights, xt, b, norm_in=st, tiled=True)
    torch.cuda.synchronize()
    assert ca == cb
    for i in range(3):
        assert torch.equal(a.view(i), b.view(i)), i
    # attention on the planes, output as rows and tiled
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    cap = 96
    pools = [torch.randn((m, 8, cap, 128), device="cuda", generator=g).to(torch.bfloat16) for _ in range(2)]
    qn = (torch.rand(128, device="cuda", generator=g) + 0.5).to(torch.bfloat16)
    kn = (torch.rand(128, device="cuda", generator=g) + 0.5).to(torch.bfloat16)
    positions = torch.tensor([(5 * i + 2) % cap for i in range(m)], dtype=torch.int32, device="cuda")
    slots = torch.arange(m, dtype=torch.int32, device="cuda")
    ws = torch.empty(native.attention_workspace(m, 32, cap), dtype=torch.float32, device="cuda")
    outs = []
    for tiled in (False, True):
        kp, vp = pools[0].clone(), pools[1].clone()
        out = torch.full((32 * 4096,) if tiled else (m, 4096), 7.0, dtype=torch.bfloat16, device="cuda")
        cnt = torch.zeros(m * 8, dtype=torch.int32, device="cuda")
        native.attention_fused_planes(a, qn, kn, positions, slots, kp, vp, out, cap, 1e6, 1e-6, ws, cnt,
                                      tiled=tiled)
        outs.append(out)
    torch.cuda.synchronize()
    assert torch.equal(_untile(native, outs[1], m, 4096), outs[0])
    assert bool((outs[1].view(4096 // 64, 4, 2, 32, 8)[:, :, :, m:, :] == 7.0).all())  # rows past M untouched
    # o as K-range planes from a tiled x, and its epilogue writing x' tiled
    po = oracle.synthetic(2560, 4096, m, seed=seed + 10)
    wo = to_device(po)[:3]
    xo = outs[0]
    h0 = torch.randn((m, 2560), device="cuda", generator=g)
    wn = (torch.rand(2560, device="cuda", generator=g) + 0.5).to(torch.bfloat16)
    res = []
    for tiled in (False, True):
        pl = native.ResidualPlanes(m, 2560, "cuda")
        native.qmv_residual_planes(wo, outs[1] if tiled else xo, pl, tiled=tiled)
        h = h0.clone()
        xp = torch.full((32 * 2560,) if tiled else (m, 2560), 7.0, dtype=torch.bfloat16, device="cuda")
        sto = native.NormStats(m, 2560, "cuda")
        native.residual_planes(pl, h, next_norm=wn, x_out=xp, stats_out=sto, tiled_out=tiled)
        res.append((pl.view().clone(), h, xp, sto.ssq.clone()))
    torch.cuda.synchronize()
    assert torch.equal(res[0][0], res[1][0]) and torch.equal(res[0][1], res[1][1])
    assert torch.equal(_untile(native, res[1][2], m, 2560), res[0][2]) and torch.equal(res[0][3], res[1][3])
    # the row-band projection: tiled x in, x' tiled out
    bands = []
    for tiled in (False, True):
        h = h0.clone()
        xp = torch.full((32 * 2560,) if tiled else (m, 2560), 7.0, dtype=torch.bfloat16, device="cuda")
        stb = native.NormStats(m, 2560, "cuda")
        native.qmv_residual_bands(wo, outs[1] if tiled else xo, m, h, next_norm=wn, x_out=xp, stats_out=stb,
                                  tiled=tiled, tiled_out=tiled)
        bands.append((h, xp, stb.ssq.clone()))
    torch.cuda.synchronize()
    assert torch.equal(bands[0][0], bands[1][0]) and torch.equal(bands[0][2], bands[1][2])
    assert torch.equal(_untile(native, bands[1][1], m, 2560), bands[0][1])
    # gate/up: x and act tiled
    pg = oracle.synthetic(9728, 2560, m, seed=seed + 20)
    pu = oracle.synthetic(9728, 2560, m, seed=seed + 21)
    gate, up = to_device(pg)[:3], to_device(pu)[:3]
    xg = bands[0][1]
    stp = _stats(native, m, 2560, seed + 22)
    act = torch.full((m, 9728), 7.0, dtype=torch.bfloat16, device="cuda")
    act_t = torch.full((32 * 9728,), 7.0, dtype=torch.bfloat16, device="cuda")
    native.gate_up_silu_norm(gate, up, xg, act, stp, 1e-6)
    native.gate_up_silu_norm(gate, up, bands[1][1], act_t, stp, 1e-6, rows=m, tiled_x=True, tiled_out=True)
    torch.cuda.synchronize()
    assert torch.equal(_untile(native, act_t, m, 9728), act)
    # down as K-range planes from the tiled act
    pd = oracle.synthetic(2560, 9728, m, seed=seed + 30)
    wd = to_device(pd)[:3]
    pa, pb = native.ResidualPlanes(m, 2560, "cuda"), native.ResidualPlanes(m, 2560, "cuda")
    native.qmv_residual_planes(wd, act, pa)
    native.qmv_residual_planes(wd, act_t, pb, tiled=True)
    torch.cuda.synchronize()
    assert pa.planes == pb.planes and torch.equal(pa.view(), pb.view())
