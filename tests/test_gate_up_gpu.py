"""GPU parity of imq_qmv_gate_up_silu, the gate and up projections with SiLU * up in one
launch, through the C ABI.

Where the grouped launch over (gate, up) takes the staged MFMA kernel (more 64-row tiles
than CUs), the fused launch computes each output from the same row sums: it must equal
imq_qmv_grouped followed by imq_silu_mul bit for bit, at the batch-32 decode shape, at 5
rows, and with a ragged last tile.  A small ragged case is checked against the oracle's
exact product (silu in float64 on the bf16-rounded projections); rows outside 5..32 and K
not a multiple of 256 are refused."""

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


def _pair(oracle, n, k, m, seed):
    pg = oracle.synthetic(n, k, m, seed=seed)
    pu = oracle.synthetic(n, k, m, seed=seed + 1)
    pu = oracle.Problem(pu.w, pu.s, pu.b, pg.x, 0)
    dg, du = to_device(pg), to_device(pu)
    return pg, pu, dg[:3], du[:3], dg[3]


@pytest.mark.parametrize("n,k,m", [(9728, 2560, 32), (9728, 2560, 5), (8200, 1024, 7)])
def test_fused_equals_grouped_then_silu(native, oracle, n, k, m):
    _, _, gate, up, x = _pair(oracle, n, k, m, oracle.SEED_BASE + 1000 + m)
    announce("gate/up silu vs grouped", n, k, m)
    g, u = native.qmv_grouped([gate, up], [x, x])
    ref = native.silu_mul(g, u, torch.empty_like(g))
    out = native.gate_up_silu(gate, up, x, torch.full_like(g, 7.0))
    again = native.gate_up_silu(gate, up, x, torch.empty_like(g))
    torch.cuda.synchronize()
    assert np.array_equal(bf16_bits(out), bf16_bits(ref))
    assert torch.equal(out, again)


def test_ragged_matches_oracle(native, oracle):
    n, k, m = 1000, 512, 9
    pg, pu, gate, up, x = _pair(oracle, n, k, m, oracle.SEED_BASE + 1020)
    announce("gate/up silu ragged", n, k, m)
    out = native.gate_up_silu(gate, up, x, torch.empty((m, n), dtype=torch.bfloat16, device="cuda"))
    torch.cuda.synchronize()
    g64, _ = oracle.qmv_f64(pg.w, pg.s, pg.b, pg.x)
    u64, _ = oracle.qmv_f64(pu.w, pu.s, pu.b, pu.x)
    g = oracle.bf16_to_f32(oracle.f32_to_bf16(g64.astype(np.float32))).astype(np.float64)
    u = oracle.bf16_to_f32(oracle.f32_to_bf16(u64.astype(np.float32))).astype(np.float64)
    ref = g / (1.0 + np.exp(-g)) * u
    got = oracle.bf16_to_f32(bf16_bits(out)).astype(np.float64)
    # each projection within one bf16 ulp of its exact value, then one more rounding
    err = np.abs(got - ref)
    assert err.max() <= 2.0 ** -6 * np.abs(ref).max(), err.max()


def test_refusals(native, oracle):
    from ironmule_amd._native import NativeError
    _, _, gate, up, x = _pair(oracle, 512, 512, 4, oracle.SEED_BASE + 1030)
    announce("gate/up silu refusals")
    with pytest.raises(NativeError):
        native.gate_up_silu(gate, up, x, torch.empty((4, 512), dtype=torch.bfloat16, device="cuda"))
    _, _, gate, up, x = _pair(oracle, 512, 320, 8, oracle.SEED_BASE + 1031)
    with pytest.raises(NativeError):
        native.gate_up_silu(gate, up, x, torch.empty((8, 512), dtype=torch.bfloat16, device="cuda"))
