"""GPU parity of the prompt prefill (decode.prefill) against the decode oracle run one
token at a time, on a small decoder (2 layers, hidden 256, 4/2 heads of 128).

Bars (the decode step's): the last position's logits within max|logit - ref| / max|ref|
<= 5e-4 (1e-4 for the decode step after it) of the oracle with the same bf16 rounding points; every key and value written to
the request's KV slot within 5% of that layer's largest oracle entry; nothing written to
other slots; and a decode step continuing at position T meets the logit bar again.
Prompts of 7 tokens take the qmv kernel, 40 and 96 tokens the fp16 dequantise + GEMM path.
"""

from __future__ import annotations

import numpy as np
import pytest

from tests.conftest import gpu_available
from tests.gpu_util import announce, oracle_decoder

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not gpu_available(), reason="needs a ROCm GPU")]


@pytest.fixture(scope="module")
def env():
    import torch

    from ironmule_amd import _native
    from oracle import decode_oracle as do
    from oracle import oracle as orc
    code, arch, _ = _native.device_check()
    assert code == 0, f"device {arch} is not supported"
    orc.lib()
    return torch, do, orc


def _vals(t):
    return t.float().cpu().numpy().astype(np.float64)


def _rel(got, ref):
    return float(np.abs(got - ref).max() / np.abs(ref).max())


@pytest.mark.parametrize("count", [7, 40, 96])
def test_prefill_matches_the_oracle_decoded_token_by_token(env, count):
    torch, do, orc = env
    from ironmule_amd.decode import (DecodeState, DecoderConfig, decode_step, prefill,
                                     random_weights)
    announce("prefill", count)
    cfg = DecoderConfig(hidden=256, layers=2, heads=4, kv_heads=2, head_dim=128,
                        intermediate=512, vocab=512, eps=1e-6, theta=1e6)
    weights = random_weights(cfg, "cuda", seed=50 + count)
    cap, slot, slots = 128, 2, 3
    state = DecodeState(cfg, batch=1, slots=slots, capacity=cap, max_len=cap, device="cuda")
    tokens = np.random.default_rng(count).integers(0, cfg.vocab, count).tolist()
    got = prefill(weights, state, tokens, slot).cpu().numpy().astype(np.float64)

    model = oracle_decoder(do, orc, weights)
    keys = [np.zeros((slots, cfg.kv_heads, cap, cfg.head_dim)) for _ in range(cfg.layers)]
    values = [np.zeros_like(k) for k in keys]
    for pos, tok in enumerate(tokens):
        ref = do.decode_step(model, keys, values, [tok], [slot], [pos], round_bf16=True)[0]
    print(f"[observed] prefill last position: max|dlogit|/max|logit| = {_rel(got, ref):.3e}", flush=True)
    assert _rel(got, ref) <= 5e-4, _rel(got, ref)  # observed 7.0e-8 .. 2.0e-4
    for i in range(cfg.layers):
        for pool, want in ((state.k_pool[i], keys[i]), (state.v_pool[i], values[i])):
            have = _vals(pool)
            assert np.abs(have[slot, :, :count] - want[slot, :, :count]).max() <= \
                0.05 * np.abs(want[slot, :, :count]).max(), i
            others = [s for s in range(slots) if s != slot]
            assert not have[others].any() and not have[slot, :, count:].any()

    # the request continues with a decode step at position `count`
    nxt = int(np.argmax(got))
    state.set_requests([nxt], [slot], [count])
    step = decode_step(weights, state)[0].cpu().numpy().astype(np.float64)
    ref2 = do.decode_step(model, keys, values, [nxt], [slot], [count], round_bf16=True)[0]
    print(f"[observed] decode step after prefill: max|dlogit|/max|logit| = {_rel(step, ref2):.3e}", flush=True)
    assert _rel(step, ref2) <= 1e-4, _rel(step, ref2)  # observed 6.0e-8 .. 5.2e-5


def test_prefill_rejects_bad_prompts(env):
    torch, do, orc = env
    from ironmule_amd.decode import DecodeState, DecoderConfig, prefill, random_weights
    cfg = DecoderConfig(hidden=256, layers=1, heads=4, kv_heads=2, head_dim=128,
                        intermediate=512, vocab=512)
    weights = random_weights(cfg, "cuda", seed=3)
    state = DecodeState(cfg, batch=1, slots=1, capacity=16, max_len=16, device="cuda")
    with pytest.raises(ValueError):
        prefill(weights, state, [], 0)
    with pytest.raises(ValueError):
        prefill(weights, state, [1] * 17, 0)
    with pytest.raises(ValueError):
        prefill(weights, state, [1, 2], 1)
