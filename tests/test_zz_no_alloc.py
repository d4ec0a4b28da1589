"""GPU parity of imq_qmv_grouped_noalloc, the entry point that allocates nothing: its split
partials and counters live in the library's static per-device scratch.  Through the C ABI,
two calls in a row (the second smaller) must give the same bits as imq_qmv_grouped_ws with
a caller workspace of imq_qmv_grouped_workspace bytes (the same plan), and meet the oracle's
bar on sampled rows.  Outputs are bf16, so the bar against the other entry point is
bit-identity."""

from __future__ import annotations

import ctypes

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


def _problems(native, weights, xs, ys):
    probs = (native.Problem * len(weights))()
    for i, ((w, s, b), x, y) in enumerate(zip(weights, xs, ys)):
        n, k = int(w.shape[0]), int(w.shape[1]) * 8
        probs[i] = native.Problem(w.data_ptr(), s.data_ptr(), b.data_ptr(), x.data_ptr(), k,
                                  y.data_ptr(), n, n, k)
    return probs


def _case(native, oracle, shapes, m, seed):
    prs = [oracle.synthetic(n, k, m, seed=seed + i) for i, (n, k) in enumerate(shapes)]
    dev = [to_device(pr) for pr in prs]
    weights = [(w, s, b) for (w, s, b, _) in dev]
    xs = [x for (_, _, _, x) in dev]
    y_ref = [torch.full((m, n), -1.0, dtype=torch.bfloat16, device="cuda") for (n, _) in shapes]
    y_new = [torch.full((m, n), -2.0, dtype=torch.bfloat16, device="cuda") for (n, _) in shapes]
    lib = native.lib()
    stream = ctypes.c_void_p(int(torch.cuda.current_stream().cuda_stream))

    probs = _problems(native, weights, xs, y_ref)
    nbytes = int(lib.imq_qmv_grouped_workspace(probs, len(shapes), m))
    ws = torch.zeros(max(nbytes, 16) // 4, dtype=torch.float32, device="cuda")
    announce("no-alloc reference (grouped_ws)", shapes, m, nbytes)
    assert lib.imq_qmv_grouped_ws(probs, len(shapes), m, 64, 4, 0, ctypes.c_void_p(ws.data_ptr()),
                                  nbytes, stream) == 0, native.last_error()
    torch.cuda.synchronize()

    probs = _problems(native, weights, xs, y_new)
    announce("no-alloc call", shapes, m)
    assert lib.imq_qmv_grouped_noalloc(probs, len(shapes), m, 64, 4, 0, stream) == 0, \
        native.last_error()
    torch.cuda.synchronize()
    for i, (pr, a, b) in enumerate(zip(prs, y_ref, y_new)):
        assert np.array_equal(bf16_bits(a), bf16_bits(b)), f"problem {i} differs"
        rows = np.unique(np.concatenate([np.arange(0, pr.n, 7), np.arange(max(0, pr.n - 40), pr.n)]))
        v, lit = oracle.check_bf16_both(bf16_bits(b)[:, rows], pr.w[rows], pr.s[rows], pr.b[rows], pr.x)
        assert v.ok, v.detail
        assert lit.ok, lit.detail
    return nbytes


def test_noalloc_matches_workspace_entry_twice(native, oracle):
    """A split call (o projection shape at 32 rows) and then a smaller split call (fewer
    rows, fewer weight rows, two problems): both bit-identical to imq_qmv_grouped_ws."""
    first = _case(native, oracle, [(2560, 4096)], 32, oracle.SEED_BASE + 900)
    second = _case(native, oracle, [(640, 4096), (320, 4096)], 8, oracle.SEED_BASE + 910)
    assert first > 0 and second > 0  # both calls used the scratch
    assert second < first


def test_noalloc_direct_to_lds_twice(native, oracle):
    """Launches of the direct-to-LDS kernel, whose split partials and counters go to the
    scratch: 2560 x 9728 at 32 rows (five K-ranges), then a smaller call (4096 x 2048, 16
    rows, three ranges), each bit-identical to imq_qmv_grouped_ws; then K = 3840 x 15360 at
    8 rows (whole-K tiles), which needs no workspace and leaves the scratch alone."""
    first = _case(native, oracle, [(2560, 9728)], 32, oracle.SEED_BASE + 940)
    second = _case(native, oracle, [(4096, 2048)], 16, oracle.SEED_BASE + 950)
    third = _case(native, oracle, [(15360, 3840)], 8, oracle.SEED_BASE + 960)
    assert first > second > 0 and third == 0


def test_noalloc_without_split(native, oracle):
    """Calls that need no workspace (one row; a staged launch of 94 tiles) go through the
    same kernels as the other entry points and never touch the scratch."""
    assert _case(native, oracle, [(2560, 2560)], 1, oracle.SEED_BASE + 920) == 0
    assert _case(native, oracle, [(6000, 512)], 16, oracle.SEED_BASE + 930) == 0
