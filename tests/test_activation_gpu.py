"""The admission knob and the activation gate on the GPU, through the C ABI.

An engine built with `k3840_matvec` admits the K=3840 kernel once and serves decode rows
from it; `close` restores the model.  An activation installed on a model runs the variant
while its gate is open for a qualified class, the original module otherwise, and after a
kill (here: a reported correctness error) the original module again, with the kill on
disk outranking the opt-in flag of a new activation.  Outputs are held to the oracle's
bar."""

from __future__ import annotations

import dataclasses
from types import SimpleNamespace

import pytest
import torch

from tests.conftest import gpu_available
from tests.gpu_util import announce, bf16_bits, to_device

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not gpu_available(), reason="needs a ROCm GPU")]

IDENTITY = SimpleNamespace(identity_sha256="ef" * 32, architecture="qwen3", revision="r1")


def _model(oracle, n, seed):
    from ironmule_amd.quantized import QuantizedLinear
    pr = oracle.synthetic(n, 3840, 1, seed=seed)
    w, s, b, x = to_device(pr)
    holder = torch.nn.Module()
    holder.proj = QuantizedLinear(w, s, b)
    return pr, holder, x


def _bar(oracle, pr, y):
    v, lit = oracle.check_bf16_both(bf16_bits(y), pr.w, pr.s, pr.b, pr.x)
    assert v.ok, v.detail
    assert lit.ok, lit.detail


def test_engine_admits_once_and_close_restores(oracle):
    from ironmule_amd import engine, qmv_k3840
    pr, model, x = _model(oracle, 1024, 31)
    original = model.proj
    announce("engine admit_k3840")
    eng = engine.load_engine(model, engine.Knobs(k3840_matvec=True), IDENTITY)
    assert eng.k3840_admission["admitted"] == 1
    assert isinstance(model.proj, qmv_k3840.K3840QuantizedLinear)
    y = model.proj(x[None])[0]
    _bar(oracle, pr, y)
    assert eng.admit_k3840(IDENTITY) is None
    assert eng.close() == 1 and model.proj is original
    off = engine.load_engine(model, identity=IDENTITY)
    assert off.k3840_admission is None and model.proj is original


def test_open_gate_runs_the_variant_and_a_kill_restores_the_module(oracle, tmp_path, monkeypatch):
    from ironmule_amd import activation as act
    from ironmule_amd import qmv_variant
    pr, model, x = _model(oracle, 1024, 32)
    original = model.proj
    context = act.context_here(model_id="synthetic", identity=IDENTITY, projection_widths=(1024,))
    controller = act.StaticController(dataclasses.asdict(context))
    controller.qualify(qmv_variant.QUALIFIED_ACTION_ID, "decode_short", 12)
    state = tmp_path / "activation.json"
    a = act.LearnedDispatchActivation(controller, context, enabled=True, state_path=state)
    announce("activation install_on")
    adm = a.install_on(model, IDENTITY)
    assert adm.admitted, adm.reason
    assert isinstance(model.proj, qmv_variant.GatedVariantLinear) and not a.gate.active

    calls = []
    real = qmv_variant.GatedVariantLinear.decode
    monkeypatch.setattr(qmv_variant.GatedVariantLinear, "decode",
                        lambda self, row: calls.append(1) or real(self, row))
    row = x[None]

    # shut: the original module serves
    shut = model.proj(row)[0]
    assert calls == []
    # open for the qualified class on the interactive route: the variant serves
    y, rec = a.serve("decode_short", "interactive", lambda: model.proj(row)[0])
    assert rec.effective_action == act.CANDIDATE and len(calls) == 1
    _bar(oracle, pr, y)
    assert torch.equal(y, shut)
    # another route shuts it again
    model_out, rec = a.serve("decode_short", "batch", lambda: model.proj(row)[0])
    assert rec.effective_action == act.REFERENCE and len(calls) == 1

    # a candidate dispatch that reports a correctness error kills
    a.serve("decode_short", "interactive", lambda: model.proj(row)[0],
            telemetry=lambda: SimpleNamespace(fallbacks=0, correctness_errors=1))
    assert len(calls) == 2 and a.gate.killed and model.proj is original
    after = model.proj(row)[0]
    assert len(calls) == 2
    _bar(oracle, pr, after)
    again = act.LearnedDispatchActivation(controller, context, enabled=True, state_path=state)
    assert not again.enabled and not again.install_on(model, IDENTITY).admitted
    assert model.proj is original
