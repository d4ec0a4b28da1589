"""GPU parity of the MoE gather qmv (imq_gather_qmv) and its routing (hip_native.
gather_matmul, NativeQuantizedSwitchLinear), through the C ABI.

Bars: each pair's row equals imq_qmv on the selected expert's weights, bit for bit (the
one-row tile is shared), and meets the oracle's bound (oracle.gather_qmv_f64); an index
outside the expert stack gives zeros; the routed module agrees with the library path
(fp32 dequantise + batched product) within the reference's probe tolerance (1e-2,
ironmule/cuda_native.py:253-268).
"""

from __future__ import annotations

import numpy as np
import pytest

from tests.conftest import gpu_available
from tests.gpu_util import announce, bf16_bits

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not gpu_available(), reason="needs a ROCm GPU")]


@pytest.fixture(scope="module")
def env():
    import torch

    from ironmule_amd import _native, hip_native
    from oracle import oracle as orc
    code, arch, _ = _native.device_check()
    assert code == 0, f"device {arch} is not supported"
    orc.lib()
    return torch, _native, hip_native, orc


def _stack(torch, orc, e, n, k, seed):
    probs = [orc.synthetic(n, k, 1, seed=seed + i) for i in range(e)]
    w = np.stack([p.w for p in probs]).view(np.int32)
    s = np.stack([p.s for p in probs])
    b = np.stack([p.b for p in probs])
    to = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    return (to(w), to(s).view(torch.bfloat16), to(b).view(torch.bfloat16),
            (np.stack([p.w for p in probs]), s, b))


def _rows(torch, r, k, seed):
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    return torch.randn((r, k), device="cuda", generator=g).to(torch.bfloat16)


@pytest.mark.parametrize("e,n,k,pairs,xs", [(8, 512, 2560, 16, 1), (8, 768, 2560, 16, 8),
                                            (4, 130, 192, 7, 1), (3, 64, 9728, 5, 5)])
def test_gather_matches_per_expert_calls_and_the_oracle(env, e, n, k, pairs, xs):
    torch, n_, _, orc = env
    announce("gather", e, n, k, pairs, xs)
    w, s, b, host = _stack(torch, orc, e, n, k, orc.SEED_BASE + 400 + e)
    x = _rows(torch, -(-pairs // xs), k, 7)
    idx = torch.tensor([(3 * p + 1) % e for p in range(pairs)], dtype=torch.int32, device="cuda")
    y = n_.gather_qmv(w, s, b, x, idx, rows_per_x=xs)
    torch.cuda.synchronize()
    for p in range(pairs):
        ex = int(idx[p])
        single = n_.qmv(w[ex], s[ex], b[ex], x[p // xs].reshape(1, -1))
        assert torch.equal(y[p].view(torch.int16), single[0].view(torch.int16)), p
    ref, mag = orc.gather_qmv_f64(host[0], host[1], host[2], bf16_bits(x), idx.cpu().numpy(), xs)
    verdict = orc.check_bf16(bf16_bits(y), ref, mag)
    assert verdict.ok, verdict.detail
    ref32 = orc.gather_qmv_dequant_f32(host[0], host[1], host[2], bf16_bits(x), idx.cpu().numpy(), xs)
    lit = orc.check_bf16_literal(bf16_bits(y), ref32, ref, mag)
    print(lit.detail)
    assert lit.ok, lit.detail


def test_gather_fp32_output_and_invalid_experts(env):
    torch, n_, _, orc = env
    announce("gather fp32 + invalid index")
    w, s, b, host = _stack(torch, orc, 4, 256, 1024, orc.SEED_BASE + 450)
    x = _rows(torch, 6, 1024, 9)
    idx = torch.tensor([0, 3, 4, -1, 2, 1000], dtype=torch.int32, device="cuda")
    y = n_.gather_qmv(w, s, b, x, idx, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert not y[2].any() and not y[3].any() and not y[5].any()
    ref, mag = orc.gather_qmv_f64(host[0], host[1], host[2], bf16_bits(x),
                                  np.array([0, 3, 99, 99, 2, 99]), 1)
    verdict = orc.check_f32(y.cpu().numpy(), ref, mag)
    assert verdict.ok, verdict.detail


def test_gather_matmul_routing_down_and_gate_up(env):
    """Down (one activation row per (token, expert) pair) and gate/up (a token's row shared
    by its top-k experts) through gather_matmul: the kernel's result equals the per-pair
    qmv and agrees with the library path within 1e-2; more than GATHER_MAX pairs take the
    library path."""
    torch, n_, hn, orc = env
    from ironmule_amd.quantized import library_gather_matmul
    announce("gather_matmul routing")
    w, s, b, _ = _stack(torch, orc, 8, 384, 2560, orc.SEED_BASE + 470)
    tokens, top = 4, 8
    indices = torch.tensor([[(t * 3 + j) % 8 for j in range(top)] for t in range(tokens)],
                           dtype=torch.int32, device="cuda")
    xg = _rows(torch, tokens, 2560, 11).reshape(tokens, 1, 1, 2560)
    xd = _rows(torch, tokens * top, 2560, 12).reshape(tokens, top, 1, 2560)
    for x in (xg, xd):
        y = hn.gather_matmul(x, w, s, b, indices)
        assert tuple(y.shape) == (tokens, top, 1, 384)
        lib_y = library_gather_matmul(x, w, s, b, indices)
        rel = (y.float() - lib_y.float()).abs().max() / lib_y.float().abs().max()
        assert float(rel) <= 1e-2
        for t in range(tokens):
            for j in range(top):
                ex = int(indices[t, j])
                row = x[t, 0 if x is xg else j].reshape(1, -1)
                single = n_.qmv(w[ex], s[ex], b[ex], row)
                assert torch.equal(y[t, j, 0].view(torch.int16), single[0].view(torch.int16))
    many = torch.zeros((9, 8), dtype=torch.int32, device="cuda")  # 72 pairs > GATHER_MAX
    xm = _rows(torch, 9, 2560, 13).reshape(9, 1, 1, 2560)
    y = hn.gather_matmul(xm, w, s, b, many)
    lib_y = library_gather_matmul(xm, w, s, b, many)
    assert torch.equal(y, lib_y)


def test_switch_linear_install(env):
    """install() probes a QuantizedSwitchLinear (one token against its first eight experts)
    and swaps it to NativeQuantizedSwitchLinear, whose call runs the gather kernel."""
    torch, n_, hn, orc = env
    from ironmule_amd.quantized import QuantizedSwitchLinear
    announce("switch linear install")
    w, s, b, _ = _stack(torch, orc, 8, 256, 1024, orc.SEED_BASE + 490)
    model = torch.nn.Sequential(QuantizedSwitchLinear(w, s, b))
    info = hn.install(model, {"gcnArchName": "gfx950:sramecc+:xnack-"})
    assert info["modules"] == 1 and info["probe_rel_error"] <= 1e-2
    assert isinstance(model[0], hn.NativeQuantizedSwitchLinear)
    indices = torch.tensor([[1, 5]], dtype=torch.int32, device="cuda")
    x = _rows(torch, 1, 1024, 3).reshape(1, 1, 1, 1024)
    y = model[0](x, indices)
    single = n_.qmv(w[5], s[5], b[5], x.reshape(1, -1))
    assert torch.equal(y[0, 1, 0].view(torch.int16), single[0].view(torch.int16))
