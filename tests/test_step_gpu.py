"""GPU parity of the persistent engine (include/ironmule_step.h), through the C ABI.

Every output of a qmv program equals imq_qmv / imq_qmv_grouped's on the same inputs, bit
for bit.  The decode program folds every RMSNorm but the first layer's input norm into the
projections around it (the o and down stages write x' = bf16(h * w_next) and per-tile sums
of squares; the next stage scales its outputs by 1/rms), so its two forms (one persistent
launch, one launch per stage) give each other's bits, its logits are checked against the
decode oracle with those rounding points, and against the per-kernel `decode_step` (RMSNorm
launches at batch 1) it agrees to the folding's rounding level, with the first layer's KV
written identically.
"""

from __future__ import annotations

import numpy as np
import pytest

from tests.conftest import gpu_available
from tests.gpu_util import announce, to_device

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


@pytest.mark.parametrize("shapes", [
    # (K of stage 0 = K of the q/k/v-like stage, N's), then a dependent stage per entry
    dict(k0=2560, n0=(4096, 1024, 1024), dep=(2560,), k1=2560, n1=(9728, 9728), dep1=(2560,)),
    dict(k0=64, n0=(128, 17), dep=(100,), k1=192, n1=(64, 8, 24), dep1=(7,)),
    dict(k0=256, n0=(320,), dep=(77, 5), k1=1024, n1=(1024, 1000), dep1=(64,)),
])
def test_qmv_program_chain_matches_per_kernel_calls(env, shapes):
    """Stage A (1-3 weights on x0), stage B (waits; reads A's first output), stage C (no
    wait, its own x1), stage D (waits; reads C's first output): every output equals the
    per-kernel call on the same inputs, bit for bit, on two runs."""
    torch, n, orc = env
    announce("qmv program", shapes)
    seed = 100
    wa = [_weight(orc, nn, shapes["k0"], seed + i) for i, nn in enumerate(shapes["n0"])]
    ya = [torch.empty(nn, dtype=torch.bfloat16, device="cuda") for nn in shapes["n0"]]
    kb = shapes["n0"][0]
    wb = [_weight(orc, nn, kb, seed + 10 + i) for i, nn in enumerate(shapes["dep"])]
    yb = [torch.empty(nn, dtype=torch.bfloat16, device="cuda") for nn in shapes["dep"]]
    wc = [_weight(orc, nn, shapes["k1"], seed + 20 + i) for i, nn in enumerate(shapes["n1"])]
    yc = [torch.empty(nn, dtype=torch.bfloat16, device="cuda") for nn in shapes["n1"]]
    kd = shapes["n1"][0]
    wd = [_weight(orc, nn, kd, seed + 30 + i) for i, nn in enumerate(shapes["dep1"])]
    yd = [torch.empty(nn, dtype=torch.bfloat16, device="cuda") for nn in shapes["dep1"]]
    x0, x1 = _row(torch, shapes["k0"], 1), _row(torch, shapes["k1"], 2)
    prog = n.qmv_program([(wa, x0, ya, False), (wb, ya[0], yb, True), (wc, x1, yc, False),
                          (wd, yc[0], yd, True)])
    for run in range(4):
        prog.launch(staged=run % 2 == 1)
        torch.cuda.synchronize()
        assert not prog.failed()
        for ws, x, ys in ((wa, x0, ya), (wb, ya[0], yb), (wc, x1, yc), (wd, yc[0], yd)):
            want = n.qmv_grouped(ws, [x.reshape(1, -1)] * len(ws))
            for y, yw in zip(ys, want):
                assert torch.equal(y.view(torch.int16), yw.reshape(-1).view(torch.int16)), run
    info = prog.info()
    assert info["stages"] == 4 and info["workgroups"] >= 1
    prog.close()


def _tiny():
    from ironmule_amd.decode import DecoderConfig
    return DecoderConfig(hidden=256, layers=2, heads=4, kv_heads=2, head_dim=128,
                         intermediate=512, vocab=512, eps=1e-6, theta=1e6)


def _twin_states(torch, cfg, capacity, seed):
    from ironmule_amd.decode import DecodeState
    a = DecodeState(cfg, batch=1, slots=3, capacity=capacity, max_len=capacity, device="cuda")
    b = DecodeState(cfg, batch=1, slots=3, capacity=capacity, max_len=capacity, device="cuda")
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    for pa, pb in zip(a.k_pool + a.v_pool, b.k_pool + b.v_pool):
        pa.copy_(torch.randn(pa.shape, device="cuda", generator=g).to(torch.bfloat16))
        pb.copy_(pa)
    return a, b


# max|dlogit| / max|logit| of the program against the per-kernel step with RMSNorm launches:
# the folded norms round x before the 1/rms scaling instead of after it (observed 2.3e-4 to
# 4.8e-4 on the tiny and the Qwen3-4B-shaped decoders)
FOLD_BAR = 1e-3


def _compare_steps(torch, weights, cfg, capacity, requests, seed, forms=True):
    """For each request (token, slot, position) in turn: the staged program (one launch per
    stage) and, with `forms`, the persistent one on a twin state give each other's logits,
    h and KV pools bit for bit; against decode_step on a third twin the logits agree within
    FOLD_BAR with the same argmax, and the first layer's KV pools bit for bit."""
    from ironmule_amd.decode import PersistentDecode, decode_step
    ref, per = _twin_states(torch, cfg, capacity, seed)
    engine = PersistentDecode(weights, per, staged=True)
    other = None
    if forms:
        _, per2 = _twin_states(torch, cfg, capacity, seed)
        other = PersistentDecode(weights, per2, staged=False)
    for step, (tok, slot, pos) in enumerate(requests):
        for st in (ref, per) + ((per2,) if forms else ()):
            st.set_requests([tok], [slot], [pos])
        want = decode_step(weights, ref)
        got = engine.step()
        got2 = other.step() if forms else None
        torch.cuda.synchronize()
        assert not engine.failed(), step
        if forms:
            assert not other.failed(), step
            assert torch.equal(got, got2), step
            assert torch.equal(per.h, per2.h), step
            for i in range(cfg.layers):
                assert torch.equal(per.k_pool[i], per2.k_pool[i]), (step, i)
                assert torch.equal(per.v_pool[i], per2.v_pool[i]), (step, i)
        rel = float((got - want).abs().max() / want.abs().max())
        print(f"[observed] program against decode_step, step {step}: max|dlogit|/max|logit| = {rel:.3e}",
              flush=True)
        assert rel <= FOLD_BAR, (step, rel)
        assert int(got.argmax()) == int(want.argmax()), step
        assert torch.equal(per.k_pool[0], ref.k_pool[0]), step
        assert torch.equal(per.v_pool[0], ref.v_pool[0]), step
    return engine, per


def test_decode_program_forms_and_decode_step_tiny(env):
    torch, n, orc = env
    from ironmule_amd.decode import random_weights
    announce("program decode, tiny decoder")
    cfg = _tiny()
    weights = random_weights(cfg, "cuda", seed=5)
    # first token of a slot, a chunk boundary, the last position, then a continuing request
    _compare_steps(torch, weights, cfg, 80, [(5, 1, 0), (17, 0, 63), (300, 2, 64), (511, 2, 79),
                                             (42, 1, 1)], seed=11)


def test_decode_program_tiny_against_the_oracle(env):
    """The persistent logits against the float64 decode oracle with the same rounding
    points (every RMSNorm but the first layer's input norm folded)."""
    torch, n, orc = env
    from ironmule_amd.decode import DecodeState, PersistentDecode, random_weights
    from oracle import decode_oracle as do
    from tests.test_decode_gpu import _oracle_model, _vals
    announce("persistent decode vs oracle, tiny decoder")
    cfg = _tiny()
    weights = random_weights(cfg, "cuda", seed=6)
    state = DecodeState(cfg, batch=1, slots=2, capacity=70, max_len=70, device="cuda")
    gen = torch.Generator(device="cuda")
    gen.manual_seed(1006)
    for kp, vp in zip(state.k_pool, state.v_pool):
        kp.copy_(torch.randn(kp.shape, device="cuda", generator=gen).to(torch.bfloat16))
        vp.copy_(torch.randn(vp.shape, device="cuda", generator=gen).to(torch.bfloat16))
    keys = [_vals(kp) for kp in state.k_pool]
    values = [_vals(vp) for vp in state.v_pool]
    model = _oracle_model(torch, do, orc, weights)
    engine = PersistentDecode(weights, state)
    tok, slot, pos = 77, 1, 66
    for step in range(2):
        state.set_requests([tok], [slot], [pos])
        got = engine.step().cpu().numpy().astype(np.float64)
        assert not engine.failed()
        ref = do.decode_step(model, keys, values, [tok], [slot], [pos], round_bf16=True,
                             fold_norms=True, fold_first=False, fold_final=True)
        rel = np.abs(got - ref).max() / np.abs(ref).max()
        print(f"[observed] persistent decode step {step}: max|dlogit|/max|logit| = {rel:.3e}", flush=True)
        assert rel <= 5e-7, (step, rel)  # observed 1.0e-7
        tok, pos = int(np.argmax(got[0])), pos + 1


def test_decode_program_forms_and_decode_step_qwen3_4b_shapes(env):
    """Two Qwen3-4B-shaped layers with the full 151,936-token head and a 512-token
    context, at the first and a later position."""
    torch, n, orc = env
    from ironmule_amd.decode import DecoderConfig, random_weights
    announce("program decode, qwen3-4b shapes, 2 layers")
    cfg = DecoderConfig(layers=2)
    weights = random_weights(cfg, "cuda", seed=9)
    engine, state = _compare_steps(torch, weights, cfg, 520,
                                   [(11, 0, 512), (151935, 0, 513), (7, 2, 0)], seed=3)
    info = engine.program.info()
    assert info["stages"] == 2 * 5 + 1 and info["workgroups"] >= 256


def test_decode_program_matches_decode_step_full_36_layers(env):
    """The full synthetic Qwen3-4B step (36 layers, the 151,936-token head, a 512-token
    context): the staged batch-1 program behind the bench's batch-1 figure agrees with the
    per-kernel step over two consecutive steps (its oracle check at this size is in
    test_decode_full_gpu.py)."""
    torch, n, orc = env
    from ironmule_amd.decode import DecoderConfig, random_weights
    announce("program decode, qwen3-4b, 36 layers, staged")
    cfg = DecoderConfig()
    assert cfg.layers == 36
    weights = random_weights(cfg, "cuda", seed=21)
    engine, state = _compare_steps(torch, weights, cfg, 520, [(11, 0, 512), (4097, 0, 513)],
                                   seed=5, forms=False)
    assert engine.program.info()["stages"] == 36 * 5 + 1
    del engine, state, weights
    torch.cuda.empty_cache()


@pytest.mark.parametrize("staged", [False, True])
def test_decode_program_replays_in_a_graph(env, staged):
    """Captured in a HIP graph (embedding, counter reset, the program's launches) and
    replayed: every replay gives the eager result's bits, with eager work between."""
    torch, n, orc = env
    from ironmule_amd.decode import PersistentDecode, random_weights
    announce("program decode in a graph, staged", staged)
    cfg = _tiny()
    weights = random_weights(cfg, "cuda", seed=12)
    ref, per = _twin_states(torch, cfg, 80, seed=4)
    engine = PersistentDecode(weights, per, staged=staged)
    per.set_requests([9], [0], [40])
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        first = engine.step(stream=stream).clone()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        engine.step(stream=stream)
    for _ in range(3):
        per.logits.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(per.logits, first)
        assert not engine.failed()


def test_decode_program_refuses_unsupported_descriptions(env):
    torch, n, orc = env
    from dataclasses import replace

    from ironmule_amd.decode import DecodeState, PersistentDecode, random_weights
    announce("persistent decode refusals")
    cfg = _tiny()
    weights = random_weights(cfg, "cuda", seed=1)
    with pytest.raises(ValueError, match="batch 1"):
        PersistentDecode(weights, DecodeState(cfg, batch=2, slots=2, capacity=16, max_len=16,
                                              device="cuda"))
    state = DecodeState(cfg, batch=1, slots=1, capacity=16, max_len=16, device="cuda")
    for bad in (replace(cfg, hidden=100), replace(cfg, kv_heads=3), replace(cfg, heads=40)):
        with pytest.raises(n.NativeError) as err:
            n.decode_program(bad, weights.layers, weights.norm, weights.embed, state.k_pool,
                             state.v_pool, state.positions, state.slot_ids, state.h,
                             state.logits, 16)
        assert err.value.code == n.IMQ_EINVAL
