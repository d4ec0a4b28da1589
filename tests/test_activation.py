"""The engine's K=3840 admission knob and the activation layer's gate, on the CPU.

Mirrors the behaviour ironmule/runtime.py:434-449 and ironmule/activation.py:151-384
state: the knob is off by default and admits once; a refusal raises with the model
untouched; the activation is off by default, checks every admission axis in order,
installs with the gate shut, opens it only for qualified classes on the interactive
route, and kills on fallbacks, correctness errors, exceptions or a controller that stops
qualifying; a kill is written to disk and outranks the opt-in flag in a new process.
Nothing here launches a kernel: installation is replaced by a recording stand-in where a
test needs one to succeed."""

from __future__ import annotations

import dataclasses
import json
import subprocess
import sys
from types import SimpleNamespace

import pytest
import torch

from ironmule_amd import activation as act
from ironmule_amd import engine as eng
from ironmule_amd import qmv_k3840, qmv_variant
from ironmule_amd.quantized import QuantizedLinear

IDENTITY = SimpleNamespace(identity_sha256="cd" * 32, architecture="qwen3", revision="r1")
CLASS = "decode_short"
ACTION = qmv_variant.QUALIFIED_ACTION_ID


def _projection(n: int = 64, k: int = 3840) -> QuantizedLinear:
    return QuantizedLinear(torch.zeros((n, k // 8), dtype=torch.int32),
                           torch.ones((n, k // 64), dtype=torch.bfloat16),
                           torch.zeros((n, k // 64), dtype=torch.bfloat16))


class _Holder(torch.nn.Module):
    def __init__(self) -> None:
        super().__init__()
        self.proj = _projection()


CONTEXT = act.ActivationContext(
    hardware_fingerprint="0123456789abcdef", gpu_architecture="gfx950", model_id="synthetic",
    model_identity_sha256=IDENTITY.identity_sha256, model_revision="r1", quantization_bits=4,
    quantization_group_size=64, hidden_size=3840, projection_widths=(64, 15360),
    library="libironmule_qmv abi 1", torch="2.10")


def _controller(context=CONTEXT, classes=(CLASS,)):
    c = act.StaticController(dataclasses.asdict(context))
    for cls in classes:
        c.qualify(ACTION, cls, 12)
    return c


# ------------------------------------------------------------------ engine knob

def test_knob_is_off_by_default_and_admits_nothing():
    assert eng.BASELINE.k3840_matvec is False and eng.Knobs() == eng.BASELINE
    assert eng.BASELINE.key() == "k3840_matvec=False"
    model = _Holder()
    before = model.proj
    engine = eng.load_engine(model, identity=IDENTITY)
    assert engine.k3840_admission is None and not engine.k3840_pending
    assert engine.admit_k3840(IDENTITY) is None
    assert model.proj is before and engine.close() == 0


@pytest.mark.parametrize("identity", [None, SimpleNamespace(identity_sha256="xyz", architecture="qwen3"),
                                      SimpleNamespace(identity_sha256="cd" * 32, architecture="llama")])
def test_refused_admission_raises_and_leaves_the_model(identity):
    model = _Holder()
    before = model.proj
    with pytest.raises(qmv_k3840.K3840Unsupported):
        eng.load_engine(model, eng.Knobs(k3840_matvec=True), identity)
    assert model.proj is before
    engine = eng.Engine(model, eng.Knobs(k3840_matvec=True))
    with pytest.raises(qmv_k3840.K3840Unsupported):
        engine.admit_k3840(identity)
    assert engine.k3840_pending and engine.k3840_admission is None and model.proj is before


def test_refused_without_a_device_even_with_a_good_identity(monkeypatch):
    monkeypatch.setattr(qmv_k3840, "_device_problem", lambda: "no gfx950 device here")
    model = _Holder()
    with pytest.raises(qmv_k3840.K3840Unsupported, match="no gfx950"):
        eng.load_engine(model, eng.Knobs(k3840_matvec=True), IDENTITY)
    assert isinstance(model.proj, QuantizedLinear)


def test_admission_runs_once_and_close_restores(monkeypatch):
    calls = []
    monkeypatch.setattr(qmv_k3840, "enable", lambda m, i: calls.append(("enable", i)) or {"admitted": 1})
    monkeypatch.setattr(qmv_k3840, "disable", lambda m: calls.append(("disable",)) or 1)
    engine = eng.load_engine(_Holder(), eng.Knobs(k3840_matvec=True), IDENTITY)
    assert engine.k3840_admission == {"admitted": 1} and engine.model_identity is IDENTITY
    assert engine.admit_k3840(IDENTITY) is None  # never again on this engine
    assert engine.close() == 1 and engine.close() == 0
    assert calls == [("enable", IDENTITY), ("disable",)]


# ------------------------------------------------------------------ activation: admission

def test_activation_is_off_by_default(tmp_path):
    a = act.LearnedDispatchActivation(_controller(), CONTEXT, state_path=tmp_path / "state")
    assert not a.enabled and "default is off" in a.disabled_reason
    adm = a.admit()
    assert not adm.admitted and adm.checked == {"opt_in": False}
    rec = a.for_dispatch(CLASS, "interactive")
    assert rec.effective_action == act.REFERENCE
    assert act.OFF.as_dict()["default_enabled"] is False


def _mismatch(name, value):
    return dataclasses.replace(CONTEXT, **{name: value})


@pytest.mark.parametrize("context,stored,reason", [
    (_mismatch("hardware_fingerprint", "ffff"), CONTEXT, "on hardware_fingerprint"),
    (_mismatch("model_identity_sha256", ""), _mismatch("model_identity_sha256", ""), "on model_identity_sha256"),
    (_mismatch("model_revision", "r2"), CONTEXT, "on model_revision"),
    (_mismatch("library", "libironmule_qmv abi 2"), CONTEXT, "on library"),
    (_mismatch("torch", "2.9"), CONTEXT, "on torch"),
    (_mismatch("gpu_architecture", "gfx942"), CONTEXT, "gpu architecture"),
    (_mismatch("quantization_bits", 8), _mismatch("quantization_bits", 8), "quantisation"),
    (_mismatch("quantization_group_size", 32), _mismatch("quantization_group_size", 32), "quantisation"),
    (_mismatch("hidden_size", 2560), _mismatch("hidden_size", 2560), "K is 2560"),
    (_mismatch("projection_widths", (40, 72)), _mismatch("projection_widths", (40, 72)), "whole number of 32"),
])
def test_every_axis_refuses_on_its_own(tmp_path, context, stored, reason):
    a = act.LearnedDispatchActivation(_controller(stored), context, enabled=True,
                                      state_path=tmp_path / "state")
    adm = a.admit()
    assert not adm.admitted and reason in adm.reason, adm.reason
    assert not act.kill_path(tmp_path / "state").exists()  # a refused admission is not a kill


def test_the_first_disagreeing_axis_is_the_reason(tmp_path):
    context = dataclasses.replace(CONTEXT, model_revision="r9", hidden_size=2560)
    adm = act.LearnedDispatchActivation(_controller(), context, enabled=True).admit()
    assert "model_revision" in adm.reason


def test_admission_needs_a_qualified_class():
    a = act.LearnedDispatchActivation(_controller(classes=()), CONTEXT, enabled=True)
    adm = a.admit()
    assert not adm.admitted and "qualifies no workload class" in adm.reason
    good = act.LearnedDispatchActivation(_controller(classes=("b", "a")), CONTEXT, enabled=True).admit()
    assert good.admitted and good.workload_classes == ("a", "b")
    assert good.checked["admitted_n"] == [64, 15360]
    assert good.checked["correctness_contract"] == qmv_variant.CORRECTNESS_CONTRACT


def test_no_controller_is_no_admission():
    adm = act.LearnedDispatchActivation(None, CONTEXT, enabled=True).admit()
    assert not adm.admitted and adm.reason == "no local controller"


# ------------------------------------------------------------------ activation: the gate

def test_prepared_gate_starts_shut_and_opens_only_for_qualified_interactive(tmp_path):
    a = act.LearnedDispatchActivation(_controller(), CONTEXT, enabled=True, state_path=tmp_path / "s")
    assert a.prepare().admitted and a.gate is not None and not a.gate.active
    rec = a.for_dispatch(CLASS, "interactive")
    assert rec.effective_action == act.CANDIDATE and rec.evidence_count == 12 and a.gate.active
    assert a.for_dispatch(CLASS, "interactive") is rec  # built once per (class, route)
    other = a.for_dispatch(CLASS, "throughput")
    assert other.effective_action == act.REFERENCE and "outside" in other.activation_reason
    assert not a.gate.active
    a.for_dispatch(CLASS, "interactive")
    unq = a.for_dispatch("long_prompt", "interactive")
    assert unq.effective_action == act.REFERENCE and not a.gate.active
    assert unq.local_learning_state == act.UNKNOWN


def test_monitor_requalification_shuts_without_killing(tmp_path):
    monitor = SimpleNamespace(requalification_required=False)
    a = act.LearnedDispatchActivation(_controller(), CONTEXT, enabled=True,
                                      state_path=tmp_path / "s", monitor=monitor)
    a.prepare()
    a.for_dispatch(CLASS, "interactive")
    monitor.requalification_required = True
    rec = a.for_dispatch(CLASS, "interactive")
    assert rec.local_learning_state == act.REQUALIFICATION_REQUIRED and not a.gate.active
    assert not a.gate.killed and not act.kill_path(tmp_path / "s").exists()
    monitor.requalification_required = False
    assert a.for_dispatch(CLASS, "interactive").effective_action == act.CANDIDATE


def test_a_controller_that_stops_qualifying_kills(tmp_path):
    ctl = _controller()
    a = act.LearnedDispatchActivation(ctl, CONTEXT, enabled=True, state_path=tmp_path / "s")
    a.prepare()
    a.for_dispatch(CLASS, "interactive")
    ctl.withdraw(ACTION, CLASS)
    rec = a.for_dispatch(CLASS, "interactive")
    assert rec.effective_action == act.REFERENCE and a.gate.killed and not a.enabled
    assert "no longer qualifies" in act.read_kill(tmp_path / "s")["reason"]
    a.gate.open("try")
    assert not a.gate.active


def test_a_controller_change_that_still_qualifies_rebuilds_records(tmp_path):
    ctl = _controller()
    a = act.LearnedDispatchActivation(ctl, CONTEXT, enabled=True, state_path=tmp_path / "s")
    a.prepare()
    first = a.for_dispatch(CLASS, "interactive")
    ctl.qualify(ACTION, CLASS, 20)
    second = a.for_dispatch(CLASS, "interactive")
    assert second is not first and second.evidence_count == 20 and a.gate.active


@pytest.mark.parametrize("telemetry,killed", [
    (SimpleNamespace(fallbacks=0, correctness_errors=0), False),
    (SimpleNamespace(fallbacks=2, correctness_errors=0), True),
    (SimpleNamespace(fallbacks=0, correctness_errors=1), True),
    (SimpleNamespace(), False),
])
def test_after_dispatch_kills_on_fallbacks_or_errors(tmp_path, telemetry, killed):
    a = act.LearnedDispatchActivation(_controller(), CONTEXT, enabled=True, state_path=tmp_path / "s")
    a.prepare()
    rec = a.for_dispatch(CLASS, "interactive")
    event = a.after_dispatch(rec, telemetry)
    assert (event is not None) == killed and a.gate.killed == killed
    assert act.kill_path(tmp_path / "s").exists() == killed
    # a reference dispatch never kills
    b = act.LearnedDispatchActivation(_controller(), CONTEXT, enabled=True)
    b.prepare()
    assert b.after_dispatch(b.for_dispatch(CLASS, "batch"), SimpleNamespace(fallbacks=5)) is None


def test_an_exception_in_a_candidate_dispatch_kills_and_propagates(tmp_path):
    a = act.LearnedDispatchActivation(_controller(), CONTEXT, enabled=True, state_path=tmp_path / "s")
    a.prepare()

    def boom():
        raise ValueError("bad")

    with pytest.raises(ValueError):
        a.serve(CLASS, "interactive", boom)
    assert a.gate.killed and "ValueError" in act.read_kill(tmp_path / "s")["reason"]
    result, rec = a.serve(CLASS, "interactive", lambda: 7)
    assert result == 7 and rec.effective_action == act.REFERENCE


def test_refused_install_kills_and_leaves_the_model(tmp_path, monkeypatch):
    def refuse(model, identity):
        raise qmv_variant.VariantUnsupported("missed its bound")

    monkeypatch.setattr(act, "install", refuse)
    model = _Holder()
    before = model.proj
    a = act.LearnedDispatchActivation(_controller(), CONTEXT, enabled=True, state_path=tmp_path / "s")
    adm = a.install_on(model, IDENTITY)
    assert not adm.admitted and "installation refused" in adm.reason
    assert model.proj is before and not a.enabled
    assert a.events[-1]["persisted_to"] == str(act.kill_path(tmp_path / "s"))


def test_install_puts_the_gate_shut_and_kill_uninstalls(tmp_path, monkeypatch):
    installed = []

    def fake_install(model, identity):
        gate = qmv_variant.VariantGate()
        installed.append(model)
        return gate, {"admitted": 1}

    monkeypatch.setattr(act, "install", fake_install)
    monkeypatch.setattr(act, "uninstall", lambda model: 1 if model is installed[0] else 0)
    a = act.LearnedDispatchActivation(_controller(), CONTEXT, enabled=True, state_path=tmp_path / "s")
    model = _Holder()
    assert a.install_on(model, IDENTITY).admitted and not a.gate.active
    assert a.status()["installed"] == {"admitted": 1}
    event = a.kill("planted")
    assert event["projections_restored"] == 1 and a.status()["gate"]["killed"]


# ------------------------------------------------------------------ the persisted kill

def test_kill_outranks_the_flag_in_a_new_process(tmp_path):
    state = tmp_path / "state.json"
    a = act.LearnedDispatchActivation(_controller(), CONTEXT, enabled=True, state_path=state)
    a.prepare()
    a.kill("correctness errors", {"n": 1})
    stored = json.loads(act.kill_path(state).read_text())
    assert stored["schema"] == act.SCHEMA and stored["detail"] == {"n": 1}
    code = ("import sys; from ironmule_amd import activation as a; "
            "x = a.LearnedDispatchActivation(None, a.ActivationContext(), enabled=True, "
            "state_path=sys.argv[1]); print(int(x.enabled), x.disabled_reason)")
    out = subprocess.run([sys.executable, "-c", code, str(state)], capture_output=True, text=True,
                         check=True, cwd=str(__import__("pathlib").Path(__file__).parents[1]))
    assert out.stdout.startswith("0 a persisted kill record is present: correctness errors"), out.stdout


@pytest.mark.parametrize("body", ["{not json", "[1, 2]"])
def test_an_unreadable_kill_record_counts_as_a_kill(tmp_path, body):
    state = tmp_path / "s"
    act.kill_path(state).write_text(body)
    a = act.LearnedDispatchActivation(_controller(), CONTEXT, enabled=True, state_path=state)
    assert not a.enabled and a.killed_at_start is not None
    assert not a.admit().admitted


def test_write_kill_is_atomic_and_leaves_no_partial(tmp_path):
    path = act.write_kill(tmp_path / "deep" / "s", "why")
    assert path.exists() and not list(path.parent.glob("*.partial"))
