"""GPU parity of the 32-row tile layout (IMQ_LD_TILED) in the batched decode launches: each
producer's tiled output is tile_rows of its output as rows, and each consumer gives the same
bits from a tiled x as from x in rows, through the C ABI.

* q/k/v (imq_qmv_norm_planes) from a tiled x take the row-band kernel, one plane per
  projection: against the oracle's bar of inv * (x' W^T) like the K-range planes from rows,
  and the same bits on a second call; down's K-range planes (K = 9728, past the row-band
  range) from a tiled x give the bits of rows; the residual epilogue (imq_residual_planes)
  and the row-band projection (imq_qmv_residual_bands) writing x' tiled;
* the gate/up launch (imq_qmv_gate_up_silu_norm) reading x and writing SiLU * up tiled;
* the planes attention (imq_attention_fused_planes) writing its output tiled.
At 32, 8 and 3 rows (rows past M are neither read nor written: the buffers start as 7.0)."""

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
    again = native.QkvPlanes(m, 32, 8, "cuda")
    native.qmv_norm_planes(weights, xt, again, norm_in=st, tiled=True)
    torch.cuda.synchronize()
    # rows: K-range planes of the direct-to-LDS kernel; tiled: one plane per projection from
    # the row-band kernel.  Each against the oracle's bar of inv * (x' W^T).
    assert ca >= 1 and cb == 1
    ssq = st.ssq[:, :40].double().cpu().numpy().sum(axis=1)
    inv = 1.0 / np.sqrt(ssq / 2560 + 1e-6)
    for i in range(3):
        ref, mag = oracle.qmv_f64(probs[i].w, probs[i].s, probs[i].b, probs[0].x)
        for pl, cnt in ((a, ca), (b, cb)):
            v = pl.view(i)
            tot = v[0].clone()
            for s_ in range(1, cnt):
                tot = tot + v[s_]
            got = tot.to(torch.bfloat16)
            chk = oracle.check_bf16(bf16_bits(got), ref * inv[:, None], mag * inv[:, None] + 4.0 * np.abs(ref * inv[:, None]) * 2.0 ** -18)
            assert chk.ok, (i, cnt, chk.detail)
        assert torch.equal(b.view(i), again.view(i)), i
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
        native.qmv_residual_planes(wo, xo, pl)  # K-range planes from rows (tiled: one row-band plane)
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
