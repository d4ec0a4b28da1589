"""The reference's call surface on the GPU: every entry point reaches the gfx950 kernels
through the C ABI and meets the oracle's bound; fallbacks reach the original module."""

from __future__ import annotations

from types import SimpleNamespace

import numpy as np
import pytest
import torch

from tests.conftest import gpu_available
from tests.gpu_util import announce, bf16_bits, to_device

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not gpu_available(), reason="needs a ROCm GPU")]

IDENTITY = SimpleNamespace(identity_sha256="ab" * 32, architecture="gemma3")
GFX950 = {"gcnArchName": "gfx950"}


def _module(oracle, n, k, seed):
    from ironmule_amd.quantized import QuantizedLinear
    pr = oracle.synthetic(n, k, 1, seed=seed)
    w, s, b, x = to_device(pr)
    return pr, QuantizedLinear(w, s, b), x


def _bound(oracle, pr, y, x_bits=None):
    x = pr.x if x_bits is None else x_bits
    v, lit = oracle.check_bf16_both(bf16_bits(y), pr.w, pr.s, pr.b, x)
    assert v.ok, v.detail
    assert lit.ok, lit.detail


def test_k3840_run_and_module(oracle):
    from ironmule_amd import _native, qmv_k3840
    pr, mod, x = _module(oracle, 1024, 3840, 7)
    announce("qmv_k3840.run")
    y = qmv_k3840.run(qmv_k3840.K3840, mod.weight, mod.scales, mod.biases, x, 1024, 3840)
    assert y.shape == (1, 1024)
    _bound(oracle, pr, y)
    assert torch.equal(y, _native.qmv(mod.weight, mod.scales, mod.biases, x))
    y2 = qmv_k3840.run(qmv_k3840.PORT, mod.weight, mod.scales, mod.biases, x, 1024, 3840)
    assert torch.equal(y, y2)
    swapped = qmv_k3840.K3840QuantizedLinear(mod)
    assert torch.equal(swapped(x[None])[0], y)
    wide = torch.randn((1, 3, 3840), device="cuda").to(torch.bfloat16)
    assert torch.equal(swapped(wide), mod(wide))  # the library path, byte for byte


def test_enable_then_disable(oracle):
    from ironmule_amd import qmv_k3840
    _, mod, x = _module(oracle, 512, 3840, 8)
    holder = torch.nn.Module()
    holder.proj = mod
    announce("enable/disable")
    record = qmv_k3840.enable(holder, IDENTITY)
    assert record["admitted"] == 1 and isinstance(holder.proj, qmv_k3840.K3840QuantizedLinear)
    assert torch.equal(holder.proj(x[None]), mod(x[None]))
    assert qmv_k3840.disable(holder) == 1 and holder.proj is mod


def test_variant_install_gate_and_uninstall(oracle):
    from ironmule_amd import qmv_variant
    pr, mod, x = _module(oracle, 1024, 3840, 9)
    holder = torch.nn.Module()
    holder.proj = mod
    announce("variant install")
    gate, record = qmv_variant.install(holder, IDENTITY)
    assert record["admitted"] == 1 and record["mismatched"] == 0
    assert not gate.active
    shut = holder.proj(x[None])
    gate.open("test")
    opened = holder.proj(x[None])
    assert torch.equal(shut, opened)
    _bound(oracle, pr, opened)
    gate.kill("test")
    gate.open("again")
    assert not gate.active
    assert qmv_variant.uninstall(holder) == 1 and holder.proj is mod


@pytest.mark.parametrize("width", [1, 2, 5, 32])
def test_run_shared(oracle, width):
    from ironmule_amd import qmv_shared
    pr = oracle.synthetic(768, 3840, width, seed=10 + width)
    w, s, b, x = to_device(pr)
    vectors = [x[i:i + 1] for i in range(width)]
    announce("run_shared", width)
    outs = qmv_shared.run_shared(w, s, b, vectors, 768)
    assert len(outs) == width
    singles = [qmv_shared.run_shared(w, s, b, [v], 768)[0] for v in vectors]
    for i in range(width):
        _bound(oracle, oracle.Problem(pr.w, pr.s, pr.b, pr.x[i:i + 1], 0), outs[i])
        if width <= 2:
            assert torch.equal(outs[i], singles[i])


@pytest.mark.parametrize("k", [4096, 15360])
def test_run_fast(oracle, k):
    from ironmule_amd import qmv_fast_shared
    pr = oracle.synthetic(512, k, 2, seed=20 + k)
    w, s, b, x = to_device(pr)
    announce("run_fast", k)
    outs = qmv_fast_shared.run_fast(w, s, b, [x[0:1], x[1:2]], 512, k)
    for i in range(2):
        _bound(oracle, oracle.Problem(pr.w, pr.s, pr.b, pr.x[i:i + 1], 0), outs[i])
    with pytest.raises(ValueError):
        qmv_fast_shared.run_fast(w, s, b, [x[0:1]], 512, 3840)


def test_paired_projections_share_the_sweep(oracle):
    from ironmule_amd import paired
    _, mod, _ = _module(oracle, 256, 3840, 30)
    xs = [torch.randn((1, 1, 3840), device="cuda").to(torch.bfloat16) for _ in range(2)]
    announce("paired")
    shared = paired.project_pair(mod, xs, share=True)
    alone = paired.project_pair(mod, xs, share=False)
    for a, b in zip(shared, alone):
        assert a.shape == (1, 1, 256) and torch.equal(a, b)


def test_native_plan_install_and_routing(oracle):
    from ironmule_amd import _native, hip_native
    from ironmule_amd.quantized import QuantizedEmbedding, QuantizedLinear
    pr = oracle.synthetic(640, 2560, 1, seed=40)
    w, s, b, x = to_device(pr)

    class Model(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.proj = QuantizedLinear(w, s, b)
            self.embed_tokens = QuantizedEmbedding(w, s, b)

    model = Model()
    announce("native install")
    record = hip_native.install(model, GFX950)
    assert record["modules"] == 2 and record["probe_rel_error"] <= hip_native.PROBE_TOLERANCE
    y = model.proj(x[None])
    _bound(oracle, pr, y)
    assert torch.equal(model.embed_tokens.as_linear(x[None]), y)
    # more than 32 rows: dequantise to fp16 and one GEMM, within the probe tolerance
    rows = torch.randn((1, 40, 2560), device="cuda").to(torch.bfloat16)
    got = model.proj(rows).float()
    ref = rows.float() @ _native.dequant(w, s, b, torch.float32).T
    assert float((got - ref).abs().max() / ref.abs().max()) < 1e-2
    # non-bf16 activations take the library path (fp32 dequantise-then-matmul)
    fp32 = model.proj(rows.float())
    assert float((fp32 - ref).abs().max() / ref.abs().max()) < 1e-5
