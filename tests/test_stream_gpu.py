"""GPU parity of the streaming engine (imq_stream_*, include/ironmule_step.h), through
the C ABI.

The bar is bit-identity with the per-kernel path: every output of a streamed program
equals imq_qmv_grouped's on the same inputs (the per-kernel qmv is itself checked against
the oracle in test_qmv_gpu.py; one stage here is also checked against the oracle
directly).  Cases: independent stages (the distinct x rows staged once) at the Qwen3-4B
layer shapes and at small ragged shapes, chained stages whose inputs are earlier
outputs, grids from one workgroup to the resident maximum, repeated launches and graph
replays, and the refusals.
"""

from __future__ import annotations

import numpy as np
import pytest

from tests.conftest import gpu_available
from tests.gpu_util import announce, bf16_bits, to_device

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not gpu_available(), reason="needs a ROCm GPU")]


@pytest.fixture(scope="module")
def env():
    import torch

    from ironmule_amd import _native
    from oracle import oracle as orc
    code, arch, _ = _native.device_check()
    assert code == 0, f"device {arch} is not supported"
    orc.lib()
    return torch, _native, orc


def _weight(orc, n, k, seed):
    w, s, b, _ = to_device(orc.synthetic(n, k, 1, seed=seed))
    return w, s, b


def _row(torch, k, seed):
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    return torch.randn(k, device="cuda", generator=g).to(torch.bfloat16)


def _check_stages(torch, n, stages, run):
    for ws, x, ys, _ in stages:
        want = n.qmv_grouped(ws, [x.reshape(1, -1)] * len(ws))
        for y, yw in zip(ys, want):
            assert torch.equal(y.view(torch.int16), yw.reshape(-1).view(torch.int16)), run


LAYER = [("qkv", (4096, 1024, 1024), 2560), ("o", (2560,), 4096), ("gate_up", (9728, 9728), 2560),
         ("down", (2560,), 9728)]


@pytest.mark.parametrize("workgroups", [0, 1, 37])
def test_independent_layer_stages(env, workgroups):
    """Two Qwen3-4B layers' seven projections as eight independent stages over three x
    rows (K = 2560, 4096, 9728): every output equals the per-kernel call, on three runs."""
    torch, n, orc = env
    announce("stream independent layer", workgroups)
    xs = {k: _row(torch, k, k) for k in (2560, 4096, 9728)}
    stages = []
    for layer in range(2):
        for i, (_, ns, k) in enumerate(LAYER):
            ws = [_weight(orc, nn, k, 1000 * layer + 10 * i + j) for j, nn in enumerate(ns)]
            ys = [torch.full((nn,), 7.0, dtype=torch.bfloat16, device="cuda") for nn in ns]
            stages.append((ws, xs[k], ys, False))
    prog = n.stream_program(stages, workgroups=workgroups)
    info = prog.info()
    assert not info["chained"] and info["stages"] == 8
    if workgroups:
        assert info["workgroups"] == workgroups
    for run in range(3):
        prog.launch()
        torch.cuda.synchronize()
        assert not prog.failed()
        _check_stages(torch, n, stages, run)
    prog.close()


@pytest.mark.parametrize("n_rows,workgroups", [(5000, 1), (5000, 3), (3001, 2), (5000, 9)])
def test_short_last_claimed_run_repeated_launches(env, n_rows, workgroups):
    """One stage whose last claimed run is shorter than the others (5000 rows at K = 2560
    are 1250 tiles: at one workgroup the claimed tail is 2 tiles past a multiple of 8),
    launched eight times on the same claim counters: every launch's output equals the
    per-kernel call.  A counter left behind by one launch would make the next skip runs."""
    torch, n, orc = env
    announce("stream short last run", n_rows, workgroups)
    x = _row(torch, 2560, 5)
    ws = [_weight(orc, n_rows, 2560, 77)]
    ys = [torch.empty(n_rows, dtype=torch.bfloat16, device="cuda")]
    stages = [(ws, x, ys, False)]
    prog = n.stream_program(stages, workgroups=workgroups)
    assert prog.info()["workgroups"] == workgroups
    for run in range(8):
        ys[0].fill_(9.0)
        prog.launch()
        torch.cuda.synchronize()
        _check_stages(torch, n, stages, run)
    prog.close()


def test_independent_ragged_shapes_and_the_oracle(env):
    """Small K (64, 192, 320), N not a multiple of any tile, one weight per stage and
    three per stage; one output is also checked against the oracle's fp64 product."""
    torch, n, orc = env
    announce("stream independent ragged")
    spec = [((17, 5, 64), 64), ((130,), 192), ((1, 33), 320), ((257,), 64), ((3, 3, 3), 192)]
    xs = {k: _row(torch, k, 50 + k) for k in (64, 192, 320)}
    stages = []
    for i, (ns, k) in enumerate(spec):
        ws = [_weight(orc, nn, k, 300 + 10 * i + j) for j, nn in enumerate(ns)]
        ys = [torch.empty(nn, dtype=torch.bfloat16, device="cuda") for nn in ns]
        stages.append((ws, xs[k], ys, False))
    prog = n.stream_program(stages)
    for run in range(2):
        prog.launch()
        torch.cuda.synchronize()
        _check_stages(torch, n, stages, run)
    pr = orc.synthetic(130, 192, 1, seed=310)
    x = bf16_bits(xs[192]).reshape(1, -1)
    verdict, lit = orc.check_bf16_both(bf16_bits(stages[1][2][0]), pr.w, pr.s, pr.b, x)
    assert verdict.ok, verdict.detail
    assert lit.ok, lit.detail
    prog.close()


@pytest.mark.parametrize("shapes", [
    dict(k0=2560, n0=(4096, 1024, 1024), dep=(2560,), k1=2560, n1=(9728, 9728), dep1=(2560,)),
    dict(k0=64, n0=(128, 17), dep=(100,), k1=192, n1=(64, 8, 24), dep1=(7,)),
    dict(k0=256, n0=(320,), dep=(77, 5), k1=1024, n1=(1024, 1000), dep1=(64,)),
])
@pytest.mark.parametrize("workgroups", [0, 3])
def test_chained_stages(env, shapes, workgroups):
    """Stage A (1-3 weights on x0), stage B (waits; reads A's first output), stage C (no
    wait, its own x1), stage D (waits; reads C's first output): every output equals the
    per-kernel call on the same inputs, bit for bit, on three runs."""
    torch, n, orc = env
    announce("stream chained", shapes, workgroups)
    seed = 100
    wa = [_weight(orc, nn, shapes["k0"], seed + i) for i, nn in enumerate(shapes["n0"])]
    ya = [torch.empty(nn, dtype=torch.bfloat16, device="cuda") for nn in shapes["n0"]]
    wb = [_weight(orc, nn, shapes["n0"][0], seed + 10 + i) for i, nn in enumerate(shapes["dep"])]
    yb = [torch.empty(nn, dtype=torch.bfloat16, device="cuda") for nn in shapes["dep"]]
    wc = [_weight(orc, nn, shapes["k1"], seed + 20 + i) for i, nn in enumerate(shapes["n1"])]
    yc = [torch.empty(nn, dtype=torch.bfloat16, device="cuda") for nn in shapes["n1"]]
    wd = [_weight(orc, nn, shapes["n1"][0], seed + 30 + i) for i, nn in enumerate(shapes["dep1"])]
    yd = [torch.empty(nn, dtype=torch.bfloat16, device="cuda") for nn in shapes["dep1"]]
    x0, x1 = _row(torch, shapes["k0"], 1), _row(torch, shapes["k1"], 2)
    stages = [(wa, x0, ya, False), (wb, ya[0], yb, True), (wc, x1, yc, False), (wd, yc[0], yd, True)]
    prog = n.stream_program(stages, workgroups=workgroups)
    assert prog.info()["chained"]
    for run in range(3):
        for t in ya + yb + yc + yd:
            t.fill_(3.0)
        prog.launch()
        torch.cuda.synchronize()
        assert not prog.failed(), run
        _check_stages(torch, n, stages, run)
    prog.close()


def test_chained_layers_replay_in_a_graph(env):
    """Three layers in decode order (q/k/v, o reading q, gate/up, down reading gate), each
    stage waiting for the previous one, captured once and replayed five times with fresh
    inputs between replays: every replay equals the per-kernel calls."""
    torch, n, orc = env
    announce("stream chained graph")
    x = _row(torch, 2560, 9)
    stages = []
    for layer in range(3):
        wq = [_weight(orc, nn, 2560, 2000 + 10 * layer + j) for j, nn in enumerate((4096, 1024, 1024))]
        yq = [torch.empty(nn, dtype=torch.bfloat16, device="cuda") for nn in (4096, 1024, 1024)]
        wo = [_weight(orc, 2560, 4096, 2100 + layer)]
        yo = [torch.empty(2560, dtype=torch.bfloat16, device="cuda")]
        wg = [_weight(orc, 9728, 2560, 2200 + 10 * layer + j) for j in range(2)]
        yg = [torch.empty(9728, dtype=torch.bfloat16, device="cuda") for _ in range(2)]
        wd = [_weight(orc, 2560, 9728, 2300 + layer)]
        yd = [torch.empty(2560, dtype=torch.bfloat16, device="cuda")]
        stages += [(wq, x, yq, layer > 0), (wo, yq[0], yo, True), (wg, yo[0], yg, True),
                   (wd, yg[0], yd, True)]
    prog = n.stream_program(stages)
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        prog.launch(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        prog.launch(stream)
    torch.cuda.synchronize()
    for rep in range(5):
        x.copy_(_row(torch, 2560, 40 + rep))
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            graph.replay()
        torch.cuda.synchronize()
        assert not prog.failed(), rep
        _check_stages(torch, n, stages, rep)
    prog.close()


def test_chained_stage_trace(env):
    """imq_stream_trace: a traced launch of a chained program gives the same outputs as an
    untraced one and, per (stage, wavefront), four stamps in order (start <= input ready <=
    x staged <= done), every stage starting after the previous stage's first wavefront was
    done; a buffer too small is refused, an independent program has no trace, and a NULL
    buffer stops the recording."""
    torch, n, orc = env
    from ironmule_amd._native import NativeError
    announce("stream chained trace")
    x = _row(torch, 2560, 11)
    wq = [_weight(orc, nn, 2560, 2400 + j) for j, nn in enumerate((4096, 1024))]
    yq = [torch.empty(nn, dtype=torch.bfloat16, device="cuda") for nn in (4096, 1024)]
    wo = [_weight(orc, 2560, 4096, 2410)]
    yo = [torch.empty(2560, dtype=torch.bfloat16, device="cuda")]
    wd = [_weight(orc, 64, 2560, 2420)]
    yd = [torch.empty(64, dtype=torch.bfloat16, device="cuda")]
    stages = [(wq, x, yq, False), (wo, yq[0], yo, True), (wd, yo[0], yd, True)]
    prog = n.stream_program(stages, workgroups=5)
    info = prog.info()
    waves = info["workgroups"] * 12
    with pytest.raises(NativeError):
        prog.trace(torch.zeros(3 * waves * 4 - 1, dtype=torch.int64, device="cuda"))
    buf = torch.zeros(3 * waves * 4, dtype=torch.int64, device="cuda")
    prog.trace(buf)
    prog.launch()
    torch.cuda.synchronize()
    assert not prog.failed()
    _check_stages(torch, n, stages, 0)
    t = buf.view(3, waves, 4).cpu().numpy()
    assert (t > 0).all()
    assert (np.diff(t, axis=2) >= 0).all()
    for s in (1, 2):
        assert t[s, :, 1].min() >= t[s - 1, :, 3].min()
    prog.trace(None)
    buf.zero_()
    prog.launch()
    torch.cuda.synchronize()
    assert not buf.any()
    _check_stages(torch, n, stages, 1)
    prog.close()
    ind = n.stream_program([([_weight(orc, 64, 2560, 2430)], x, [yd[0]], False)])
    with pytest.raises(NativeError, match="chained"):
        ind.trace(torch.zeros(1024, dtype=torch.int64, device="cuda"))
    ind.close()


def test_refusals(env):
    torch, n, orc = env
    from ironmule_amd._native import NativeError
    w = _weight(orc, 64, 2560, 1)
    x = _row(torch, 2560, 1)
    y = torch.empty(64, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(NativeError, match="nothing to wait for"):
        n.stream_program([([w], x, [y], True)])
    big = _weight(orc, 8, 16384, 2)
    xb = _row(torch, 16384, 2)
    yb = torch.empty(8, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(NativeError, match="10240"):
        n.stream_program([([big], xb, [yb], False)])
    # an independent stage that reads an output of the program
    w2 = _weight(orc, 16, 64, 3)
    y2 = torch.empty(16, dtype=torch.bfloat16, device="cuda")
    w1 = _weight(orc, 64, 2560, 4)
    with pytest.raises(NativeError, match="waits for nothing"):
        n.stream_program([([w1], x, [y], False), ([w2], y, [y2], False)])
    # nine distinct x rows
    stages = []
    for i in range(9):
        xi = _row(torch, 64, 70 + i)
        stages.append(([_weight(orc, 4, 64, 80 + i)], xi, [torch.empty(4, dtype=torch.bfloat16, device="cuda")], False))
    with pytest.raises(NativeError, match="exceed"):
        n.stream_program(stages)
