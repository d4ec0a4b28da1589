"""The full C5 decode step against the decode oracle: 36 Qwen3-4B layers, the tied
151,936-token head and a 512-token context.

Batch 32 runs the per-kernel step (every layer's RMSNorms folded into the projections,
fused attention), batch 1 the staged program (five launches per layer, every RMSNorm but
the first layer's input norm folded).  Two sampled requests of the batch-32 step and the
batch-1 request are recomputed by the oracle in float64 with each step's bf16 rounding
points (`decode_oracle.decode_step(round_bf16=True, fold_norms=True, ...)`), their slots'
KV pools copied to the host before the step, the layers dequantised one at a time.  The bar
on each request's logits is max|got - ref| / max|ref|; the observed values are printed.
The argmax token must agree as well.  At 4 and 8 requests two Qwen3-4B-shaped layers and
the head are held to the same bar (the o and down projections as K-range planes with their
own epilogue launch, the attention reading the q/k/v planes).
"""

from __future__ import annotations

import numpy as np
import pytest

from tests.conftest import gpu_available
from tests.gpu_util import announce, logit_error, oracle_decoder

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not gpu_available(), reason="needs a ROCm GPU")]

CONTEXT = 512
# max|dlogit| / max|logit| of one request at 36 layers against the oracle with the step's
# own rounding points: about twice what was observed (batch 32: 4.3e-6 and 8.0e-6; batch 1:
# 4.6e-6; against the unfolded rounding points the batch-32 step was at 3.9e-5 and 5.1e-5)
BAR = {32: 2e-5, 1: 1e-5}
# the same at two layers and 4 or 8 requests: observed 2.4e-7 to 1.9e-5 (at two layers one
# bf16 tie of an intermediate, rounded the other way than the oracle's, moves the logits by
# about 1e-5 of their range; over 36 layers such differences average out)
BAR_TWO_LAYERS = 4e-5


def _vals(t):
    return t.float().cpu().numpy().astype(np.float64)


def test_full_decode_step_matches_the_oracle():
    import torch

    from ironmule_amd.decode import DecodeState, DecoderConfig, PersistentDecode, decode_step, random_weights
    from oracle import decode_oracle as do
    from oracle import oracle as orc
    orc.lib()
    cfg = DecoderConfig()
    assert cfg.layers == 36 and cfg.vocab == 151936
    weights = random_weights(cfg, "cuda", seed=21)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(22)

    # batch 32, per-kernel step; requests at positions 505..512 in permuted slots
    b32 = DecodeState(cfg, batch=32, slots=32, capacity=CONTEXT + 8, max_len=CONTEXT + 8, device="cuda")
    for pool in b32.k_pool + b32.v_pool:
        pool.copy_(torch.randn(pool.shape, device="cuda", generator=gen).to(torch.bfloat16))
    tokens32 = [(7919 * r + 11) % cfg.vocab for r in range(32)]
    slots32 = [(5 * r + 3) % 32 for r in range(32)]
    pos32 = [CONTEXT - (r % 8) for r in range(32)]
    sample = [0, 21]
    # batch 1, staged program
    b1 = DecodeState(cfg, batch=1, slots=2, capacity=CONTEXT + 8, max_len=CONTEXT + 8, device="cuda")
    for pool in b1.k_pool + b1.v_pool:
        pool.copy_(torch.randn(pool.shape, device="cuda", generator=gen).to(torch.bfloat16))
    tokens1, slots1, pos1 = [151000], [1], [CONTEXT]

    # the oracle's pools: the sampled slots of both states, before the steps write them
    src = [(b32, slots32[r]) for r in sample] + [(b1, slots1[0])]
    keys = [np.stack([_vals(st.k_pool[i][sl]) for st, sl in src]) for i in range(cfg.layers)]
    values = [np.stack([_vals(st.v_pool[i][sl]) for st, sl in src]) for i in range(cfg.layers)]

    announce("full decode step, batch 32 per-kernel")
    b32.set_requests(tokens32, slots32, pos32)
    got32 = decode_step(weights, b32).clone()
    torch.cuda.synchronize()
    announce("full decode step, batch 1 staged program")
    b1.set_requests(tokens1, slots1, pos1)
    prog = PersistentDecode(weights, b1, staged=True)
    got1 = prog.step().clone()
    torch.cuda.synchronize()
    assert not prog.failed()

    announce("decode oracle, 36 layers, 3 requests")
    model = oracle_decoder(do, orc, weights, lazy=True)
    ref32 = do.decode_step(model, [k[:2] for k in keys], [v[:2] for v in values],
                           [tokens32[r] for r in sample], [0, 1], [pos32[r] for r in sample],
                           round_bf16=True, fold_norms=True, fold_first=True, fold_final=False)
    ref1 = do.decode_step(model, [k[2:] for k in keys], [v[2:] for v in values], tokens1, [0],
                          pos1, round_bf16=True, fold_norms=True, fold_first=False, fold_final=True)
    ref = np.concatenate([ref32, ref1])
    got = [_vals(got32[r]) for r in sample] + [_vals(got1[0])]
    names = [f"batch 32 request {r}" for r in sample] + ["batch 1 staged"]
    errs = [logit_error(g, ref[j]) for j, g in enumerate(got)]
    for name, e, g, j in zip(names, errs, got, range(3)):
        print(f"[observed] full decode step {name}: max|dlogit|/max|logit| = {e:.3e}, "
              f"argmax {int(np.argmax(g))} vs oracle {int(np.argmax(ref[j]))}", flush=True)
    for name, e, g, j in zip(names, errs, got, range(3)):
        assert e <= BAR[32 if j < 2 else 1], (name, e)
        assert int(np.argmax(g)) == int(np.argmax(ref[j])), name


@pytest.mark.parametrize("batch", [4, 8])
def test_decode_step_at_small_batches_matches_the_oracle(batch):
    """Two Qwen3-4B-shaped layers and the tied head at 4 and 8 requests (512-token context):
    the per-kernel step with the folded norms, the o and down projections as K-range planes
    with their residual epilogue launched on its own, and the fused attention reading the
    q/k/v planes (four-wavefront workgroups at 4 requests, twelve at 8), against the oracle
    with the step's rounding points on two sampled requests."""
    import dataclasses

    import torch

    from ironmule_amd import _native
    from ironmule_amd.decode import DecodeState, DecoderConfig, decode_step, random_weights
    from oracle import decode_oracle as do
    from oracle import oracle as orc
    orc.lib()
    cfg = dataclasses.replace(DecoderConfig(), layers=2)
    weights = random_weights(cfg, "cuda", seed=31 + batch)
    # the launches this test is about: o and down split K, so they run as planes + epilogue
    for name, k in (("o", cfg.heads * cfg.head_dim), ("down", cfg.intermediate)):
        x = torch.empty((batch, k), dtype=torch.bfloat16, device="cuda")
        assert 2 <= _native.residual_split_planes(weights.layers[0][name], x) <= _native.RESIDUAL_MAX_PLANES
    gen = torch.Generator(device="cuda")
    gen.manual_seed(32 + batch)
    st = DecodeState(cfg, batch=batch, slots=batch + 1, capacity=CONTEXT + 8, max_len=CONTEXT + 8, device="cuda")
    for pool in st.k_pool + st.v_pool:
        pool.copy_(torch.randn(pool.shape, device="cuda", generator=gen).to(torch.bfloat16))
    tokens = [(104729 * r + 7) % cfg.vocab for r in range(batch)]
    slots = [(3 * r + 1) % (batch + 1) for r in range(batch)]
    pos = [CONTEXT - 3 * r for r in range(batch)]
    sample = [0, batch - 1]
    keys = [np.stack([_vals(st.k_pool[i][slots[r]]) for r in sample]) for i in range(cfg.layers)]
    values = [np.stack([_vals(st.v_pool[i][slots[r]]) for r in sample]) for i in range(cfg.layers)]
    announce("decode step, two qwen3-4b layers", batch)
    st.set_requests(tokens, slots, pos)
    got = decode_step(weights, st).clone()
    torch.cuda.synchronize()
    model = oracle_decoder(do, orc, weights)
    ref = do.decode_step(model, keys, values, [tokens[r] for r in sample], [0, 1], [pos[r] for r in sample],
                         round_bf16=True, fold_norms=True, fold_first=True, fold_final=False)
    for j, r in enumerate(sample):
        g = _vals(got[r])
        e = logit_error(g, ref[j])
        print(f"[observed] two-layer decode step batch {batch} request {r}: max|dlogit|/max|logit| = {e:.3e}",
              flush=True)
        assert e <= BAR_TWO_LAYERS, (batch, r, e)
        assert int(np.argmax(g)) == int(np.argmax(ref[j])), (batch, r)
