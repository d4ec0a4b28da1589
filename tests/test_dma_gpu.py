"""GPU parity of the direct-to-LDS MFMA kernel (qmv_dma_kernel), through the C ABI.

The launch plan takes it for M >= 5 (M >= 3 with whole-K tiles) when the launch has at most
one tile of 64 weight rows per CU (256 on MI355X) and every K is a multiple of 256: whole-K tiles when there are more
tiles than half the CUs, else the groups of each tile split into K-ranges (four-group
multiples of at most 28 groups, at least 8) toward at least 0.6 workgroups per CU, the last
range of a tile adding the others' fp32 partials in range order.  The shapes below cover its
variants: K = 3840 x 15360 (8 groups per wavefront, eight wavefronts, the last one with four
groups), K = 512 with a ragged last tile (four groups per wavefront, two wavefronts), K = 256
(the second wavefront has no groups), K = 4096 x 8192 (three ranges, the last shorter),
K = 2304 (a part-full and an idle wavefront), two weights sharing one x and two weights with
their own x (two ranges each), the q/k/v projections of a 2560-wide layer in one launch
(two ranges), a 4096-deep weight in four ranges, a 9728-deep one in six (the last with 12
groups), a 3328-deep one in three and K = 2560 x 2560 in four (the last with four groups),
and x rows strided inside a wider buffer.  Bars are the oracle's (check_bf16 and the literal
bar / check_f32) on sampled rows, which include the ragged last tile; repeated calls give
the same bits (the split counters return to zero).
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


def _rows(n, step):
    return np.unique(np.concatenate([np.arange(0, n, step), np.arange(max(0, n - 70), n)]))


def _check(oracle, pr, y, rows, out_f32=False):
    if out_f32:
        ref, mag = oracle.qmv_f64(pr.w[rows], pr.s[rows], pr.b[rows], pr.x)
        v = oracle.check_f32(y.float().cpu().numpy()[:, rows], ref, mag)
    else:
        v, lit = oracle.check_bf16_both(bf16_bits(y)[:, rows], pr.w[rows], pr.s[rows], pr.b[rows], pr.x)
        assert lit.ok, lit.detail
    assert v.ok, v.detail


@pytest.mark.parametrize("n,k,m,out_f32", [
    (15360, 3840, 3, False), (15360, 3840, 4, True),
    (15360, 3840, 5, False), (15360, 3840, 8, False), (15360, 3840, 31, False),
    (15360, 3840, 32, False), (15360, 3840, 32, True),
    (8200, 512, 5, False), (8200, 512, 32, True),
    (8192, 256, 16, False),
    (8192, 4096, 32, True),
    (8256, 2304, 7, False),
])
def test_single_weight_matches_oracle(native, oracle, n, k, m, out_f32):
    pr = oracle.synthetic(n, k, m, seed=oracle.SEED_BASE + 800 + m + k // 64)
    w, s, b, x = to_device(pr)
    announce("dma single", n, k, m, out_f32)
    dtype = torch.float32 if out_f32 else torch.bfloat16
    y = native.qmv(w, s, b, x, out_dtype=dtype)
    y2 = native.qmv(w, s, b, x, out_dtype=dtype)
    torch.cuda.synchronize()
    _check(oracle, pr, y, _rows(n, 97), out_f32)
    assert torch.equal(y, y2)


def test_two_weights_share_one_x(native, oracle):
    """Two 6144 x 2560 weights (96 tiles each), one x of 32 rows, one launch."""
    m, n, k = 32, 6144, 2560
    pg = oracle.synthetic(n, k, m, seed=oracle.SEED_BASE + 850)
    pu = oracle.synthetic(n, k, m, seed=oracle.SEED_BASE + 851)
    pu = oracle.Problem(pu.w, pu.s, pu.b, pg.x, 0)
    wg, sg, bg, x = to_device(pg)
    wu, su, bu, _ = to_device(pu)
    announce("dma gate/up", m)
    g, u = native.qmv_grouped([(wg, sg, bg), (wu, su, bu)], [x, x])
    torch.cuda.synchronize()
    rows = _rows(n, 89)
    _check(oracle, pg, g, rows)
    _check(oracle, pu, u, rows)


def test_two_weights_with_their_own_x(native, oracle):
    """Two 4096 x 2048 weights (64 tiles each, two K-ranges), each with its own 9 activation
    rows."""
    m = 9
    prs = [oracle.synthetic(4096, 2048, m, seed=oracle.SEED_BASE + 860 + i) for i in range(2)]
    dev = [to_device(pr) for pr in prs]
    announce("dma two x", m)
    outs = native.qmv_grouped([(w, s, b) for (w, s, b, _) in dev], [x for (*_, x) in dev])
    torch.cuda.synchronize()
    for pr, y in zip(prs, outs):
        _check(oracle, pr, y, _rows(4096, 37))


@pytest.mark.parametrize("m", [32, 7])
def test_split_qkv_projections_in_one_launch(native, oracle, m):
    """q (4096 rows), k and v (1024 each) of a 2560-wide layer: 96 tiles in two K-ranges of
    20 groups, one x."""
    shapes = [(4096, 2560), (1024, 2560), (1024, 2560)]
    prs = [oracle.synthetic(n, k, m, seed=oracle.SEED_BASE + 870 + i) for i, (n, k) in enumerate(shapes)]
    prs = [prs[0]] + [oracle.Problem(p.w, p.s, p.b, prs[0].x, 0) for p in prs[1:]]
    dev = [to_device(pr) for pr in prs]
    x = dev[0][3]
    announce("dma split q/k/v", m)
    weights = [(w, s, b) for (w, s, b, _) in dev]
    outs = native.qmv_grouped(weights, [x, x, x])
    again = native.qmv_grouped(weights, [x, x, x])
    torch.cuda.synchronize()
    for (n, _), pr, y, y2 in zip(shapes, prs, outs, again):
        _check(oracle, pr, y, _rows(n, 41))
        assert torch.equal(y, y2)


@pytest.mark.parametrize("n,k,m,out_f32", [
    (2600, 4096, 32, True), (2600, 4096, 5, False),
    (2560, 9728, 32, False), (2560, 9728, 32, True),
    (3000, 3328, 19, False), (2560, 2560, 32, False),
])
def test_split_ranges_match_oracle(native, oracle, n, k, m, out_f32):
    pr = oracle.synthetic(n, k, m, seed=oracle.SEED_BASE + 880 + m + k // 64)
    w, s, b, x = to_device(pr)
    announce("dma split", n, k, m, out_f32)
    dtype = torch.float32 if out_f32 else torch.bfloat16
    y = native.qmv(w, s, b, x, out_dtype=dtype)
    y2 = native.qmv(w, s, b, x, out_dtype=dtype)
    torch.cuda.synchronize()
    _check(oracle, pr, y, _rows(n, 53), out_f32)
    assert torch.equal(y, y2)


def test_strided_rows_through_the_abi(native, oracle):
    """imq_qmv with ldx > K (x rows inside a wider buffer) and ldy > N, 128 whole-K tiles."""
    n, k, m = 8192, 256, 9
    pr = oracle.synthetic(n, k, m, seed=oracle.SEED_BASE + 890)
    w, s, b, x = to_device(pr)
    wide = torch.zeros((m, k + 64), dtype=torch.bfloat16, device="cuda")
    wide[:, :k] = x
    y = torch.zeros((m, n + 8), dtype=torch.bfloat16, device="cuda")
    announce("dma strided")
    native._check(native.lib().imq_qmv(
        native._ptr(w), native._ptr(s), native._ptr(b), native._ptr(wide), k + 64,
        native._ptr(y), n + 8, m, n, k, 64, 4, 0, native._stream(None)))
    torch.cuda.synchronize()
    _check(oracle, pr, y[:, :n].contiguous(), _rows(n, 17))
    assert not y[:, n:].any()  # columns past N untouched
