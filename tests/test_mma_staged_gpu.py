"""GPU parity of the staged MFMA kernel (qmv_mma_staged_kernel, M >= 3), through the C ABI.

The launch plan takes it when every K is a multiple of 256, x rows are strided (no row
pointer table), the direct-to-LDS kernel declines the launch (M < 5, more tiles of 64 weight
rows than CUs, or K-ranges that would be shorter than 12 groups) and either the launch has
at least 77 tiles, or K >= 4096 and a split workspace is given.  The shapes below are chosen
to meet those conditions (or, for the fallback case, to miss exactly one).  Bars are the oracle's (oracle.check_bf16 /
check_f32): bf16 outputs within 1 bf16 ulp of the exactly computed product plus the fp32
summation allowance; split launches also repeat their bits call after call.
"""

from __future__ import annotations

import numpy as np
import pytest

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


def _check(oracle, pr, y, rows, out_f32=False):
    if out_f32:
        ref, mag = oracle.qmv_f64(pr.w[rows], pr.s[rows], pr.b[rows], pr.x)
        v = oracle.check_f32(y.float().cpu().numpy()[:, rows], ref, mag)
    else:
        v, lit = oracle.check_bf16_both(bf16_bits(y)[:, rows], pr.w[rows], pr.s[rows], pr.b[rows], pr.x)
        assert lit.ok, lit.detail
    assert v.ok, v.detail


def _rows(n, step):
    return np.unique(np.concatenate([np.arange(0, n, step), np.arange(max(0, n - 70), n)]))


@pytest.mark.parametrize("m", [3, 5, 16, 32])
def test_staged_wide_launch_matches_oracle(native, oracle, m):
    """6000 rows = 94 tiles of 64 (the last one ragged: 48 rows), K = 512 (two stages): at
    least 77 tiles, fewer than the direct-to-LDS kernel's 128.  M = 3 at this K takes the
    few-row VALU tile instead; the oracle bar is the same."""
    pr = oracle.synthetic(6000, 512, m, seed=oracle.SEED_BASE + 500 + m)
    w, s, b, x = to_device(pr)
    announce("staged wide", m)
    y = native.qmv(w, s, b, x)
    _check(oracle, pr, y, _rows(6000, 11))


@pytest.mark.parametrize("m,n", [(4, 200), (32, 129)])
def test_staged_split_repeats_bit_identical(native, oracle, m, n):
    """Few rows and K = 8192: the groups are split eight ways (the library asks for a
    workspace), the last split of each tile adds the partials in order; five calls give
    the same bits and meet the oracle."""
    k = 8192
    pr = oracle.synthetic(n, k, m, seed=oracle.SEED_BASE + 520 + m)
    w, s, b, x = to_device(pr)
    probs = (native.Problem * 1)()
    probs[0] = native.Problem(w.data_ptr(), s.data_ptr(), b.data_ptr(), x.data_ptr(), k,
                              0, n, n, k)
    assert native.lib().imq_qmv_grouped_workspace(probs, 1, m) > 0
    announce("staged split", m, n)
    first = native.qmv(w, s, b, x)
    _check(oracle, pr, first, np.arange(n))
    for _ in range(4):
        again = native.qmv(w, s, b, x)
        assert np.array_equal(bf16_bits(again), bf16_bits(first))


def test_staged_grouped_problems(native, oracle):
    """Two weights of 8200 rows sharing one x (129 + 129 tiles, ragged) and a third with its
    own x and K, one launch (268 tiles: more than the direct-to-LDS kernel takes); each
    output meets the oracle."""
    m = 7
    shapes = [(8200, 1024), (8200, 1024), (640, 2048)]
    prs = [oracle.synthetic(n, k, m, seed=oracle.SEED_BASE + 540 + i)
           for i, (n, k) in enumerate(shapes)]
    dev = [to_device(p) for p in prs]
    xs = [dev[0][3], dev[0][3], dev[2][3]]
    announce("staged grouped")
    outs = native.qmv_grouped([d[:3] for d in dev], xs)
    for p, d, o, xx in zip(prs, dev, outs, xs):
        pr = oracle.Problem(p.w, p.s, p.b, bf16_bits(xx), 0)
        _check(oracle, pr, o, _rows(p.w.shape[0], 9))


def test_staged_fp32_output(native, oracle):
    import torch
    pr = oracle.synthetic(16448, 768, 32, seed=oracle.SEED_BASE + 560)  # 257 tiles
    w, s, b, x = to_device(pr)
    announce("staged fp32")
    y = native.qmv(w, s, b, x, out_dtype=torch.float32)
    _check(oracle, pr, y, _rows(16448, 29), out_f32=True)


def test_staged_strided_rows_through_the_abi(native, oracle):
    """imq_qmv with ldx > K (x rows inside a wider buffer) and ldy > N (257 tiles)."""
    import torch
    n, k, m = 16448, 256, 9
    pr = oracle.synthetic(n, k, m, seed=oracle.SEED_BASE + 570)
    w, s, b, x = to_device(pr)
    wide = torch.zeros((m, k + 64), dtype=torch.bfloat16, device="cuda")
    wide[:, :k] = x
    y = torch.zeros((m, n + 8), dtype=torch.bfloat16, device="cuda")
    announce("staged strided")
    native._check(native.lib().imq_qmv(
        native._ptr(w), native._ptr(s), native._ptr(b), native._ptr(wide), k + 64,
        native._ptr(y), n + 8, m, n, k, 64, 4, 0, native._stream(None)))
    torch.cuda.synchronize()
    _check(oracle, pr, y[:, :n].contiguous(), _rows(n, 17))
    assert not y[:, n:].any()  # columns past N untouched


def test_k_not_multiple_of_256_takes_the_other_kernel(native, oracle):
    """8200 rows but K = 320: the plan falls back to qmv_mma_kernel; the oracle bar holds."""
    pr = oracle.synthetic(8200, 320, 9, seed=oracle.SEED_BASE + 580)
    w, s, b, x = to_device(pr)
    announce("K % 256 != 0 fallback")
    y = native.qmv(w, s, b, x)
    _check(oracle, pr, y, _rows(8200, 23))
