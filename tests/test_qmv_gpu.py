"""GPU parity of the HIP qmv against the oracle, through the C ABI (ctypes).

Bars (see oracle.check_bf16 / check_f32): dequantised weights bit-exact; bf16 outputs
within 1 bf16 ulp of the exactly computed product (plus an fp32 summation allowance of
2**-20 * sum|w*x| that only matters under cancellation); fp32 outputs within that
allowance and max|y-ref|/max|ref| <= 1e-3.  Shapes cover the benchmark configurations,
tiny and ragged N, every M from 1 to 32, and the reference's exact fixtures.
"""

from __future__ import annotations

import json
import os

import numpy as np
import pytest

from tests.conftest import gpu_available
from tests.gpu_util import announce, bf16_bits, to_device

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not gpu_available(), reason="needs a ROCm GPU")]

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.fixture(scope="module")
def native():
    from ironmule_amd import _native
    code, arch, cus = _native.device_check()
    assert code == 0, f"device {arch} is not supported"
    return _native


def _check(oracle, pr, y, out_f32=False, rows=None):
    w, s, b, x = pr.w, pr.s, pr.b, pr.x
    if rows is not None:
        w, s, b = w[rows], s[rows], b[rows]
    ref, mag = oracle.qmv_f64(w, s, b, x)
    if out_f32:
        got = y.float().cpu().numpy()
        if rows is not None:
            got = got[:, rows]
        v = oracle.check_f32(got, ref, mag)
    else:
        got = bf16_bits(y)
        if rows is not None:
            got = got[:, rows]
        v, lit = oracle.check_bf16_both(got, w, s, b, x)
        assert lit.ok, lit.detail
    assert v.ok, v.detail
    return v


SHAPES = [
    # (N, K): the decode layer's projections, the shared-weight K=3840 shape, tiny/ragged
    (2560, 2560), (4096, 2560), (1024, 2560), (2560, 4096), (9728, 2560), (2560, 9728),
    (64, 3840), (8, 64), (33, 192), (1, 64), (100, 15360), (257, 1024),
]


@pytest.mark.parametrize("n,k", SHAPES)
def test_qmv_batch1_matches_oracle(native, oracle, n, k):
    pr = oracle.synthetic(n, k, 1, seed=oracle.SEED_BASE + n + k)
    w, s, b, x = to_device(pr)
    announce("qmv m=1", n, k)
    y = native.qmv(w, s, b, x)
    _check(oracle, pr, y)


@pytest.mark.parametrize("m", [1, 2, 3, 4, 5, 7, 8, 9, 12, 16, 17, 24, 31, 32])
def test_qmv_every_row_count(native, oracle, m):
    pr = oracle.synthetic(384, 2560, m, seed=oracle.SEED_BASE + 100 + m)
    w, s, b, x = to_device(pr)
    announce("qmv rows", m)
    y = native.qmv(w, s, b, x)
    _check(oracle, pr, y)


@pytest.mark.parametrize("m", [1, 32])
def test_qmv_fp32_output(native, oracle, m):
    import torch
    pr = oracle.synthetic(1000, 2560, m, seed=oracle.SEED_BASE + 3)
    w, s, b, x = to_device(pr)
    announce("qmv fp32 out", m)
    y = native.qmv(w, s, b, x, out_dtype=torch.float32)
    _check(oracle, pr, y, out_f32=True)


def test_multi_equals_stacked_rows(native, oracle):
    pr = oracle.synthetic(1536, 3840, 2, seed=oracle.SEED_BASE + 4)
    w, s, b, x = to_device(pr)
    announce("qmv_multi width 2")
    outs = native.qmv_multi(w, s, b, [x[0], x[1]])
    stacked = native.qmv(w, s, b, x)
    for i in range(2):
        assert np.array_equal(bf16_bits(outs[i])[0], bf16_bits(stacked)[i])
    _check(oracle, pr, stacked)


@pytest.mark.parametrize("m", [1, 2, 5, 32])
def test_grouped_equals_separate_calls(native, oracle, m):
    """q/k/v (one activation) and o/down (their own) in one launch: each output matches
    its own call bit for bit, and the oracle."""
    shapes = [(512, 2560), (128, 2560), (128, 2560), (320, 4096), (96, 9728)]
    probs = [oracle.synthetic(n, k, m, seed=oracle.SEED_BASE + 40 + i)
             for i, (n, k) in enumerate(shapes)]
    dev = [to_device(p) for p in probs]
    xs = [dev[0][3], dev[0][3], dev[0][3], dev[3][3], dev[4][3]]
    announce("grouped", m)
    outs = native.qmv_grouped([d[:3] for d in dev], xs)
    for i, (p, d) in enumerate(zip(probs, dev)):
        single = native.qmv(d[0], d[1], d[2], xs[i])
        if m == 1:
            # one kernel serves both (every x fits the streaming kernel's LDS): same
            # arithmetic, same bits.  At M > 1 the grouped call's three activations can
            # exceed that LDS budget and take the MFMA kernel, whose fp32 summation order
            # differs; both calls must then meet the oracle bound on their own.
            assert np.array_equal(bf16_bits(outs[i]), bf16_bits(single)), i
        pr = oracle.Problem(p.w, p.s, p.b, bf16_bits(xs[i]), 0)
        _check(oracle, pr, outs[i])
        _check(oracle, pr, single)


@pytest.mark.parametrize("m", [3, 4])
def test_few_row_tile_rows_equal_one_row_calls(native, oracle, m):
    """Three and four rows with every K <= 4096 take the few-row tile (the one-row tile
    serving several activation rows from one weight read), in a grouped launch and with
    the pointer table of qmv_multi: each output row equals the one-row call on that row,
    bit for bit, and the oracle."""
    shapes = [(512, 2560), (128, 2560), (320, 4096), (33, 192)]
    probs = [oracle.synthetic(n, k, m, seed=oracle.SEED_BASE + 60 + i)
             for i, (n, k) in enumerate(shapes)]
    dev = [to_device(p) for p in probs]
    xs = [dev[0][3], dev[0][3], dev[2][3], dev[3][3]]
    announce("few-row grouped", m)
    outs = native.qmv_grouped([d[:3] for d in dev], xs)
    for i, (p, d) in enumerate(zip(probs, dev)):
        for r in range(m):
            one = native.qmv(d[0], d[1], d[2], xs[i][r:r + 1].contiguous())
            assert np.array_equal(bf16_bits(outs[i])[r], bf16_bits(one)[0]), (i, r)
        _check(oracle, oracle.Problem(p.w, p.s, p.b, bf16_bits(xs[i]), 0), outs[i])
    announce("few-row qmv_multi", m)
    w, s, b, x = dev[2]
    rows = [x[r].clone() for r in range(m)]  # separate allocations: the pointer table
    multi = native.qmv_multi(w, s, b, rows)
    stacked = native.qmv(w, s, b, x)
    for r in range(m):
        assert np.array_equal(bf16_bits(multi[r])[0], bf16_bits(stacked)[r]), r


@pytest.mark.parametrize("n,k", [(256, 2560), (64, 15360), (33, 192)])
def test_dequant_is_bit_exact(native, oracle, n, k):
    import torch
    pr = oracle.synthetic(n, k, 1, seed=oracle.SEED_BASE + 5 + n)
    w, s, b, _ = to_device(pr)
    announce("dequant", n, k)
    want = oracle.dequant_f32(pr.w, pr.s, pr.b)
    got = native.dequant(w, s, b, torch.float32).cpu().numpy()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    got16 = native.dequant(w, s, b, torch.bfloat16)
    assert np.array_equal(bf16_bits(got16), oracle.f32_to_bf16(want))
    goth = native.dequant(w, s, b, torch.float16).cpu()
    assert torch.equal(goth, torch.from_numpy(want).to(torch.float16))


def test_golden_fixtures(native, oracle):
    import torch
    data = json.load(open(os.path.join(HERE, "golden", "qmv_golden.json")))
    for p in data["problems"]:
        w = np.array([[int(h, 16) for h in row] for row in p["w"]], dtype=np.uint32)
        pr = oracle.Problem(w, np.array(p["scales"], dtype=np.uint16),
                            np.array(p["biases"], dtype=np.uint16),
                            np.array(p["x"], dtype=np.uint16), 0)
        tw, ts, tb, tx = to_device(pr)
        announce("golden", p["name"])
        d = native.dequant(tw, ts, tb, torch.float32).cpu().numpy()
        assert np.array_equal(d, np.array(p["dequant_f32"], dtype=np.float32)), p["name"]
        y = native.qmv(tw, ts, tb, tx)
        exact = np.array(p["y_f64"])
        _, mag = oracle.qmv_f64(pr.w, pr.s, pr.b, pr.x)
        v = oracle.check_bf16(bf16_bits(y), exact, mag)
        assert v.ok, (p["name"], v.detail)
        lit = oracle.check_bf16_literal(bf16_bits(y), oracle.qmv_dequant_f32(pr.w, pr.s, pr.b, pr.x),
                                        exact, mag)
        print(p["name"], lit.detail)
        assert lit.ok, (p["name"], lit.detail)


@pytest.mark.parametrize("m", [1, 2, 4, 8, 16, 32])
def test_shared_weight_config_full_size(native, oracle, m):
    """The shared-weight configuration at its own shape, K=3840, N=15360, over its M sweep
    (the weight read once for all M requests; each M takes its own launch plan); rows
    sampled for the oracle, including the last ones."""
    pr = oracle.synthetic(15360, 3840, m, seed=oracle.SEED_BASE + 2)
    w, s, b, x = to_device(pr)
    announce("shared K3840 N15360", m)
    y = native.qmv(w, s, b, x)
    rows = np.unique(np.concatenate([np.arange(0, 15360, 37), np.arange(15300, 15360)]))
    _check(oracle, pr, y, rows=rows)


def test_lm_head_full_size(native, oracle):
    import torch
    pr = oracle.synthetic(151936, 2560, 1, seed=oracle.SEED_BASE + 3)
    w, s, b, x = to_device(pr)
    announce("lm head N151936 fp32")
    y = native.qmv(w, s, b, x, out_dtype=torch.float32)
    rows = np.concatenate([np.arange(0, 151936, 101), np.arange(151936 - 64, 151936)])
    _check(oracle, pr, y, out_f32=True, rows=rows)


def test_output_written_exactly_once_regardless_of_prior_contents(native, oracle):
    import torch
    pr = oracle.synthetic(777, 2560, 3, seed=oracle.SEED_BASE + 9)
    w, s, b, x = to_device(pr)
    announce("out prefilled with NaN")
    out = torch.full((3, 777), float("nan"), dtype=torch.bfloat16, device="cuda")
    native.qmv(w, s, b, x, out=out)
    assert not torch.isnan(out).any()
    _check(oracle, pr, out)


def test_python_errors(native):
    import torch
    w = torch.zeros((8, 8), dtype=torch.int32, device="cuda")
    s = torch.zeros((8, 1), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError):
        native.qmv(w, s, s, torch.zeros((33, 64), dtype=torch.bfloat16, device="cuda"))
    with pytest.raises(ValueError):
        native.qmv(w, s, s, torch.zeros((1, 64), dtype=torch.float32, device="cuda"))


@pytest.mark.parametrize("m,n,k", [(3, 300, 9728), (32, 2560, 4096), (17, 129, 2560)])
def test_split_groups_repeat_bit_identical(native, oracle, m, n, k):
    """Few rows, long K: the groups are split over workgroups whose partials the last one of
    each tile adds in order.  The split is really taken (the library asks for a
    workspace), five calls in a row give the same bits (the tile counters return to zero
    after every call) and every call meets the oracle bound."""
    import ctypes
    pr = oracle.synthetic(n, k, m, seed=oracle.SEED_BASE + 60 + m)
    w, s, b, x = to_device(pr)
    probs = (native.Problem * 1)()
    probs[0] = native.Problem(w.data_ptr(), s.data_ptr(), b.data_ptr(), x.data_ptr(), k,
                              0, n, n, k)
    assert native.lib().imq_qmv_grouped_workspace(probs, 1, m) > 0
    del ctypes
    announce("split groups", m, n, k)
    first = native.qmv(w, s, b, x)
    _check(oracle, pr, first)
    for _ in range(4):
        again = native.qmv(w, s, b, x)
        assert np.array_equal(bf16_bits(again), bf16_bits(first))


def test_split_calls_of_different_shapes_share_a_workspace(native, oracle):
    """Decode-like alternation of split shapes on one stream (so one cached workspace):
    q/k/v-like grouped, o-like, gate/up-like grouped and down-like calls at M = 32, three
    rounds; every output meets the oracle bound and repeats its first round's bits."""
    shapes = [[(4096, 2560), (1024, 2560), (1024, 2560)], [(2560, 4096)],
              [(9728, 2560), (9728, 2560)], [(2560, 9728)]]
    m = 32
    calls = []
    for j, group in enumerate(shapes):
        prs = [oracle.synthetic(n, k, m, seed=oracle.SEED_BASE + 80 + 10 * j + i)
               for i, (n, k) in enumerate(group)]
        dev = [to_device(p) for p in prs]
        calls.append((prs, dev))
    announce("split shapes share a workspace")
    first = None
    for rnd in range(3):
        outs = []
        for prs, dev in calls:
            outs.append(native.qmv_grouped([d[:3] for d in dev], [dev[0][3]] * len(dev)))
        bits = [[bf16_bits(o) for o in group] for group in outs]
        if first is None:
            first = bits
            for (prs, dev), group in zip(calls, outs):
                for p, d, o in zip(prs, dev, group):
                    rows = np.arange(0, p.w.shape[0], 7)
                    pr = oracle.Problem(p.w, p.s, p.b, bf16_bits(dev[0][3]), 0)
                    _check(oracle, pr, o, rows=rows)
        else:
            for a, b in zip(bits, first):
                for x, y in zip(a, b):
                    assert np.array_equal(x, y), rnd


def test_a_graph_keeps_its_workspace_after_the_stream_outgrows_it(native, oracle):
    """Continuous batching's pattern: a graph of a batch-8 split launch is captured on a
    stream, then a batch-32 launch on the same stream needs a larger workspace and a graph
    of it is captured too.  The first graph's workspace must stay allocated: fresh tensors
    filled with junk take whatever memory was freed, and five replays of each graph (with
    eager work between them) still give their eager results' bits."""
    import torch
    n_rows, k = 2560, 4096
    pr = oracle.synthetic(n_rows, k, 32, seed=oracle.SEED_BASE + 95)
    w, s, b, x32 = to_device(pr)
    x8 = x32[:8].contiguous()
    stream = torch.cuda.Stream()
    key = native._workspace_key(w.device, stream)
    announce("graph workspace growth")
    with torch.cuda.stream(stream):
        want8 = native.qmv(w, s, b, x8, stream=stream)
    torch.cuda.synchronize()
    size8 = native._workspaces[key].numel()
    retired = len(native._retired)
    g8 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g8, stream=stream):
        y8 = native.qmv(w, s, b, x8, stream=stream)
    with torch.cuda.stream(stream):
        want32 = native.qmv(w, s, b, x32, stream=stream)
    torch.cuda.synchronize()
    assert native._workspaces[key].numel() > size8 and len(native._retired) == retired + 1
    g32 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g32, stream=stream):
        y32 = native.qmv(w, s, b, x32, stream=stream)
    torch.cuda.synchronize()
    junk = [torch.full((size8,), -7.0e30, device="cuda") for _ in range(8)]
    _check(oracle, pr, want32)
    for rep in range(5):
        with torch.cuda.stream(stream):
            g8.replay()
        torch.cuda.synchronize()
        assert torch.equal(y8.view(torch.int16), want8.view(torch.int16)), rep
        with torch.cuda.stream(stream):
            g32.replay()
        torch.cuda.synchronize()
        assert torch.equal(y32.view(torch.int16), want32.view(torch.int16)), rep
        junk.append(native.qmv(w, s, b, x8))
    del junk
