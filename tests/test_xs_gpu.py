"""GPU parity of the x-stationary MFMA kernel (qmv_xs_kernel), through the C ABI.

The launch plan takes it for M >= 3 when the launch has at least 8 tiles of 32 weight rows
per CU (2048 tiles on 256 CUs) and every K is a multiple of 256 up to 4096: the LM head
(N = 151936, K = 2560) is the shape it exists for.  Bars are the oracle's (check_bf16 /
check_f32) on sampled rows, which include the ragged last tile; M = 5 and 16 take the
one-m-block form (two tiles of weights in flight), M = 17 and 32 the two-m-block form.
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
    return np.unique(np.concatenate([np.arange(0, n, step), np.arange(max(0, n - 80), n)]))


@pytest.mark.parametrize("m,out_f32", [(5, True), (16, False), (17, True), (32, True), (32, False)])
def test_lm_head_shape_matches_oracle(native, oracle, m, out_f32):
    n, k = 151936, 2560
    pr = oracle.synthetic(n, k, m, seed=oracle.SEED_BASE + 700 + m)
    w, s, b, x = to_device(pr)
    announce("xs lm head", m, out_f32)
    y = native.qmv(w, s, b, x, out_dtype=torch.float32 if out_f32 else torch.bfloat16)
    torch.cuda.synchronize()
    rows = _rows(n, 997)
    if out_f32:
        ref, mag = oracle.qmv_f64(pr.w[rows], pr.s[rows], pr.b[rows], pr.x)
        v = oracle.check_f32(y.cpu().numpy()[:, rows], ref, mag)
    else:
        v, lit = oracle.check_bf16_both(bf16_bits(y)[:, rows], pr.w[rows], pr.s[rows], pr.b[rows], pr.x)
        assert lit.ok, lit.detail
    assert v.ok, v.detail


def test_grouped_many_tiles_repeat_bits(native, oracle):
    """Two weights with different K in one launch (70016 + 4096 rows: >= 2048 tiles, the
    first one ragged), bf16 out; the oracle bar on sampled rows, and a second call gives the
    same bits."""
    m = 8
    shapes = [(70016 + 7, 1024), (4096, 4096)]
    prs = [oracle.synthetic(n, k, m, seed=oracle.SEED_BASE + 720 + i) for i, (n, k) in enumerate(shapes)]
    dev = [to_device(pr) for pr in prs]
    announce("xs grouped", shapes, m)
    outs = native.qmv_grouped([(w, s, b) for (w, s, b, _) in dev], [x for (*_, x) in dev])
    again = native.qmv_grouped([(w, s, b) for (w, s, b, _) in dev], [x for (*_, x) in dev])
    torch.cuda.synchronize()
    for pr, y, y2 in zip(prs, outs, again):
        rows = _rows(pr.n, 331)
        v, lit = oracle.check_bf16_both(bf16_bits(y)[:, rows], pr.w[rows], pr.s[rows], pr.b[rows], pr.x)
        assert v.ok, v.detail
        assert lit.ok, lit.detail
        assert np.array_equal(bf16_bits(y), bf16_bits(y2))
