"""GPU parity of the 256-row band MFMA kernel (qmv_band_kernel), through the C ABI.

The launch plan takes it for 5 <= M <= 32 when neither the x-stationary kernel nor the
direct-to-LDS kernel's whole-K tiles apply, every K is a multiple of 256 and the launch
fills at least half the CUs (256 on MI355X) with bands of 256 weight rows times K-ranges
of at most 16 groups, for single-weight launches (grouped ones keep the plans whose bits
the fused gate/up entry reproduces): 19456 x 2560 (76 bands in three ranges, the last of 8
groups), 20000 x 3840 (79 bands, four ranges, the last of 12 groups, a ragged last band),
8192 x 4096 (eight ranges of 8), and K <= 1024 with more than 170 bands (one range, no
partials): N = 50000 with a ragged last band, N = 45000 at K = 512 with fp32 output.  Rows
m >= M read row M - 1 and are never stored (M = 5, 6, 8, 9, 12, 17, 24, 31).  Bars are the oracle's (check_bf16 with the literal bar / check_f32) on sampled
rows that include the ragged last band; repeated calls give the same bits (the band
counters return to zero).
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
    return np.unique(np.concatenate([np.arange(0, n, step), np.arange(max(0, n - 300), n)]))


def _check(oracle, pr, y, rows, out_f32=False):
    if out_f32:
        ref, mag = oracle.qmv_f64(pr.w[rows], pr.s[rows], pr.b[rows], pr.x)
        v = oracle.check_f32(y.float().cpu().numpy()[:, rows], ref, mag)
    else:
        v, lit = oracle.check_bf16_both(bf16_bits(y)[:, rows], pr.w[rows], pr.s[rows], pr.b[rows], pr.x)
        assert lit.ok, lit.detail
    assert v.ok, v.detail


@pytest.mark.parametrize("n,k,m,out_f32", [
    (19456, 2560, 32, False), (19456, 2560, 16, True),
    (20000, 3840, 24, False), (20000, 3840, 17, True),
    (8192, 4096, 32, False), (8192, 4096, 16, False),
    (50000, 1024, 31, False), (45000, 512, 32, True),
    (50000, 1024, 9, False), (19456, 2560, 12, False), (8192, 4096, 8, True),
    (50000, 1024, 5, False), (19456, 2560, 6, True),
])
def test_band_matches_oracle(native, oracle, n, k, m, out_f32):
    pr = oracle.synthetic(n, k, m, seed=oracle.SEED_BASE + 950 + m + k // 64)
    w, s, b, x = to_device(pr)
    announce("band", n, k, m, out_f32)
    dtype = torch.float32 if out_f32 else torch.bfloat16
    y = native.qmv(w, s, b, x, out_dtype=dtype)
    y2 = native.qmv(w, s, b, x, out_dtype=dtype)
    torch.cuda.synchronize()
    _check(oracle, pr, y, _rows(n, 173), out_f32)
    assert torch.equal(y, y2)
