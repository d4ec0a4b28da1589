"""The switch that lets a locally qualified K=3840 variant serve decode, and takes it away.

Mirrors the gate-driving part of ironmule/activation.py: `ActivationContext`,
`Admission`, `ActivationRecord`, `OFF`, the persisted kill (`kill_path`, `read_kill`,
`write_kill`) and `LearnedDispatchActivation` with `admit`, `install_on`, `prepare`,
`for_dispatch`, `after_dispatch`, `kill` and `status` (activation.py:113-148, 151-384).
The learner that qualifies workload classes from A/B evidence (ironmule/local_learner.py)
and the drift monitor (ironmule/monitoring.py) are not part of this build; the activation
reads them through the few members listed under "Controller" below, so the reference's
own learner and monitor objects, or `StaticController` here, can be passed in.

What it does:

* Off by default.  Only a caller passing `enabled=True`, with no kill record on disk,
  and a controller that qualifies at least one workload class for the variant on this
  machine's context gets anything but the reference path.
* `install_on(model, identity)` checks every admission axis first, then installs the
  variant (`qmv_variant.install`) with its gate shut.  An install that fails kills.
* `for_dispatch(workload_class, route)` opens the gate for a class the controller
  qualifies on an eligible route and shuts it for everything else.  The record for a
  (class, route) pair is built once and reused until the controller's digest changes.
* `after_dispatch(record, telemetry)` kills on fallbacks or correctness errors reported
  for a candidate dispatch; `serve` also kills when the candidate dispatch raises.
* A kill shuts the gate for the rest of the process, puts the original modules back and
  writes `<state>.kill` atomically.  That file outranks `enabled=True` in every later
  process; nothing here removes it.  An unreadable kill file counts as a kill.

Controller (the members read): `digest` (str, changes whenever its state does);
`as_dict()` with "digest" and "context" (the machine and model it was measured on);
`recommendation(action_id, workload_class)` with `.local_learning_state` and
`.evidence_count`; and the mapping `_recommendations` keyed by (action_id,
workload_class).  Monitor: `requalification_required` (bool).

The context pins differ from the reference's in two fields: the reference pins the MLX
and mlx_lm versions its byte identity was measured under; here `library` (this HIP
library's ABI version) and `torch` stand in their place.
"""

from __future__ import annotations

import hashlib
import json
import os
import tempfile
from dataclasses import dataclass, field
from pathlib import Path
from typing import Any, Callable, Mapping

from . import qmv_k3840
from .qmv_variant import (CORRECTNESS_CONTRACT, QUALIFIED_ACTION_ID, QUALIFIED_GEOMETRY,
                          VariantGate, VariantUnsupported, install, uninstall)

SCHEMA = "ironmule.local_activation.v1"
REFERENCE = "reference"
CANDIDATE = "candidate"
# the controller and monitor states the activation reads (ironmule/local_learner.py:49-52,
# ironmule/monitoring.py:53)
UNKNOWN = "UNKNOWN"
CANDIDATE_QUALIFIED = "CANDIDATE_QUALIFIED"
REQUALIFICATION_REQUIRED = "REQUALIFICATION_REQUIRED"
#: The variant is qualified for single-token decode on the sequential route only.
ELIGIBLE_ROUTES = ("interactive",)
TARGET_K = qmv_k3840.TARGET_K
ROWS_PER_GROUP = QUALIFIED_GEOMETRY[0] * QUALIFIED_GEOMETRY[1]
#: Context fields a controller's stored context must match exactly (and be non-empty).
PINNED_CONTEXT = ("hardware_fingerprint", "model_identity_sha256", "model_revision",
                  "library", "torch")


@dataclass(frozen=True)
class ActivationContext:
    """What the admission compares against the controller's stored context."""

    hardware_fingerprint: str = ""
    gpu_architecture: str = ""
    model_id: str = ""
    model_identity_sha256: str = ""
    model_revision: str = ""
    quantization_bits: int = 0
    quantization_group_size: int = 0
    hidden_size: int = 0
    projection_widths: tuple[int, ...] = ()
    library: str = ""
    torch: str = ""


def hardware_fingerprint() -> str:
    """16 hex digits naming this GPU: sha256 of its architecture, CU count, name and
    memory size (needs the HIP library and a device)."""
    import torch

    from . import _native
    code, arch, cus = _native.device_check()
    props = torch.cuda.get_device_properties(torch.cuda.current_device())
    facts = {"arch": arch, "code": code, "cus": cus, "name": props.name,
             "memory": int(props.total_memory)}
    return hashlib.sha256(json.dumps(facts, sort_keys=True).encode()).hexdigest()[:16]


def context_here(*, model_id: str = "", identity: Any = None, bits: int = 4,
                 group_size: int = 64, hidden_size: int = TARGET_K,
                 projection_widths: tuple[int, ...] = ()) -> ActivationContext:
    """This machine's context for a model (needs the HIP library and a device)."""
    import torch

    from . import _native
    _, arch, _ = _native.device_check()
    return ActivationContext(
        hardware_fingerprint=hardware_fingerprint(), gpu_architecture=arch, model_id=model_id,
        model_identity_sha256=getattr(identity, "identity_sha256", "") or "",
        model_revision=getattr(identity, "revision", "") or "",
        quantization_bits=int(bits), quantization_group_size=int(group_size),
        hidden_size=int(hidden_size), projection_widths=tuple(projection_widths),
        library=f"libironmule_qmv abi {int(_native.lib().imq_abi_version())}",
        torch=torch.__version__)


@dataclass(frozen=True)
class Admission:
    """Whether the variant may be installed at all, and the axis that decided it."""

    admitted: bool
    reason: str
    action_id: str = ""
    controller_digest: str = ""
    workload_classes: tuple[str, ...] = ()
    checked: Mapping[str, Any] = field(default_factory=dict)

    def as_dict(self) -> dict[str, Any]:
        return {"admitted": self.admitted, "reason": self.reason, "action_id": self.action_id,
                "controller_digest": self.controller_digest,
                "workload_classes": list(self.workload_classes), "checked": dict(self.checked)}


@dataclass(frozen=True)
class ActivationRecord:
    """What one dispatch was allowed to run, and on which controller state."""

    base_action: str
    effective_action: str
    local_learning_state: str
    evidence_count: int
    controller_digest: str
    activation_reason: str
    workload_class: str = ""

    def as_dict(self) -> dict[str, Any]:
        return {"base_action": self.base_action, "effective_action": self.effective_action,
                "local_learning_state": self.local_learning_state,
                "evidence_count": self.evidence_count,
                "controller_digest": self.controller_digest,
                "activation_reason": self.activation_reason,
                "workload_class": self.workload_class,
                "opt_in_required": True, "default_enabled": False}


OFF = ActivationRecord(REFERENCE, REFERENCE, UNKNOWN, 0, "",
                       "local learned dispatch is not enabled; the default is off")


def _reference_record(reason: str, workload_class: str, state: str = UNKNOWN,
                      evidence: int = 0, digest: str = "") -> ActivationRecord:
    return ActivationRecord(REFERENCE, REFERENCE, state, evidence, digest, reason, workload_class)


# ------------------------------------------------------------------ the persisted kill

def kill_path(state_path: Path) -> Path:
    """The kill record beside a state file: `<state>.kill`."""
    state_path = Path(state_path)
    return state_path.with_name(state_path.name + ".kill")


def read_kill(state_path: Path) -> dict[str, Any] | None:
    """The kill record, or None when there is none.  A record that cannot be read or is
    not a JSON object still counts as a kill."""
    path = kill_path(state_path)
    if not path.exists():
        return None
    try:
        stored = json.loads(path.read_text(encoding="utf-8"))
    except (OSError, ValueError):
        return {"schema": SCHEMA, "reason": "the kill record is unreadable; that counts as "
                                            "killed, not as absent"}
    if not isinstance(stored, Mapping):
        return {"schema": SCHEMA, "reason": "the kill record is not a JSON object"}
    return dict(stored)


def write_kill(state_path: Path, reason: str, detail: Mapping[str, Any] | None = None) -> Path:
    """Write the kill record atomically (a temporary file renamed over it)."""
    path = kill_path(state_path)
    path.parent.mkdir(parents=True, exist_ok=True)
    body = json.dumps({"schema": SCHEMA, "reason": reason, "detail": dict(detail or {}),
                       "effect": "the locally qualified variant stays off on this machine "
                                 "until this file is removed by hand"},
                      indent=2, sort_keys=True)
    fd, partial = tempfile.mkstemp(dir=str(path.parent), suffix=".partial")
    try:
        with os.fdopen(fd, "w", encoding="utf-8") as out:
            out.write(body)
        os.replace(partial, path)
    except BaseException:
        Path(partial).unlink(missing_ok=True)
        raise
    return path


# ------------------------------------------------------------------ a fixed controller

@dataclass(frozen=True)
class Recommendation:
    local_learning_state: str
    evidence_count: int = 0


_NO_STATE = Recommendation(UNKNOWN, 0)


class StaticController:
    """A controller whose qualification comes from outside (for example a measured A/B
    run): a context and a table of (action, workload class) -> state.  Its digest is the
    sha256 of both, so `qualify` and `withdraw` change it."""

    def __init__(self, context: Mapping[str, Any]) -> None:
        self._context = dict(context)
        self._recommendations: dict[tuple[str, str], Recommendation] = {}
        self._digest = ""

    def qualify(self, action_id: str, workload_class: str, evidence: int) -> None:
        self._set(action_id, workload_class, Recommendation(CANDIDATE_QUALIFIED, int(evidence)))

    def withdraw(self, action_id: str, workload_class: str, state: str = "REFERENCE_ONLY") -> None:
        self._set(action_id, workload_class, Recommendation(state, 0))

    def _set(self, action_id: str, workload_class: str, rec: Recommendation) -> None:
        self._recommendations[(action_id, workload_class)] = rec
        self._digest = ""

    def recommendation(self, action_id: str, workload_class: str) -> Recommendation:
        return self._recommendations.get((action_id, workload_class), _NO_STATE)

    @property
    def digest(self) -> str:
        if not self._digest:
            rows = sorted([a, c, r.local_learning_state, r.evidence_count]
                          for (a, c), r in self._recommendations.items())
            body = json.dumps({"context": self._context, "rows": rows}, sort_keys=True)
            self._digest = hashlib.sha256(body.encode()).hexdigest()
        return self._digest

    def as_dict(self) -> dict[str, Any]:
        return {"digest": self.digest, "context": dict(self._context)}


def _qualified_classes(learner: Any, action_id: str) -> tuple[str, ...]:
    return tuple(sorted(
        workload_class for (action, workload_class) in getattr(learner, "_recommendations", {})
        if action == action_id
        and learner.recommendation(action, workload_class).local_learning_state == CANDIDATE_QUALIFIED))


# ------------------------------------------------------------------ the activation

class LearnedDispatchActivation:
    """One substitution (reference -> the installed variant), for qualified classes only,
    and one way out (a kill that outlives the process)."""

    def __init__(self, learner: Any, context: ActivationContext, *, enabled: bool = False,
                 state_path: Path | None = None, action_id: str = QUALIFIED_ACTION_ID,
                 monitor: Any = None) -> None:
        self.learner = learner
        self.context = context
        self.action_id = action_id
        self.monitor = monitor
        self.state_path = Path(state_path) if state_path is not None else None
        self.gate: VariantGate | None = None
        self.installed: dict[str, Any] | None = None
        self.admission: Admission | None = None
        self.events: list[dict[str, Any]] = []
        self._model: Any = None
        self._records: dict[tuple[str, str], ActivationRecord] = {}
        self._digest = ""
        self.killed_at_start = read_kill(self.state_path) if self.state_path is not None else None
        # a kill on disk outranks the caller's flag
        self.enabled = bool(enabled) and self.killed_at_start is None
        if not enabled:
            self.disabled_reason = "not enabled by the caller; the default is off"
        elif self.killed_at_start is not None:
            self.disabled_reason = ("a persisted kill record is present: "
                                    f"{self.killed_at_start.get('reason', 'no reason given')}")
        else:
            self.disabled_reason = ""

    # -- admission ------------------------------------------------------------
    def _axes(self, stored: Mapping[str, Any]) -> list[tuple[str, Any, Callable[[], str | None]]]:
        """The admission axes in order: (name, what this runtime has, problem()) where
        problem() is None when the axis agrees, else the refusal's reason."""
        ctx = self.context
        stored_context = stored.get("context", {}) or {}

        def pinned(name: str) -> Callable[[], str | None]:
            def problem() -> str | None:
                want = getattr(ctx, name)
                if not want or stored_context.get(name) != want:
                    return f"controller state does not match this runtime on {name}"
                return None
            return problem

        def architecture() -> str | None:
            if ctx.gpu_architecture and stored_context.get("gpu_architecture") not in ("", ctx.gpu_architecture):
                return "gpu architecture"
            return None

        def quantization() -> str | None:
            if (ctx.quantization_bits, ctx.quantization_group_size) != (4, 64):
                return "quantisation: the kernel is built for 4 bits at group size 64"
            return None

        def reduction() -> str | None:
            if ctx.hidden_size and ctx.hidden_size != TARGET_K:
                return f"K is {ctx.hidden_size}, the kernel is built for {TARGET_K}"
            return None

        def widths() -> str | None:
            if ctx.projection_widths and not any(w % ROWS_PER_GROUP == 0 for w in ctx.projection_widths):
                return f"no projection width is a whole number of {ROWS_PER_GROUP} rows"
            return None

        return ([(name, getattr(ctx, name), pinned(name)) for name in PINNED_CONTEXT]
                + [("gpu_architecture", ctx.gpu_architecture, architecture),
                   ("quantization", {"bits": ctx.quantization_bits,
                                     "group_size": ctx.quantization_group_size}, quantization),
                   ("k", ctx.hidden_size, reduction),
                   ("projection_widths", list(ctx.projection_widths), widths)])

    def admit(self) -> Admission:
        """Every axis in order, before anything is installed; the first that disagrees is
        the reason."""
        checked: dict[str, Any] = {"opt_in": self.enabled}
        if not self.enabled:
            return Admission(False, self.disabled_reason, checked=checked)
        if self.learner is None:
            return Admission(False, "no local controller", checked=checked)
        stored = self.learner.as_dict()
        digest = stored["digest"]
        checked["controller_digest"] = digest
        for name, value, problem in self._axes(stored):
            checked[name] = value
            reason = problem()
            if reason is not None:
                return Admission(False, reason, controller_digest=digest, checked=checked)
        checked["admitted_n"] = [w for w in self.context.projection_widths if w % ROWS_PER_GROUP == 0]
        checked["action_id"] = self.action_id
        checked["correctness_contract"] = CORRECTNESS_CONTRACT
        classes = _qualified_classes(self.learner, self.action_id)
        checked["local_preference"] = CANDIDATE_QUALIFIED if classes else "not qualified"
        if not classes:
            return Admission(False, "the local controller qualifies no workload class for this "
                                    "action", controller_digest=digest, checked=checked)
        return Admission(True, "every admission axis agrees and the local controller qualifies "
                               "at least one workload class", action_id=self.action_id,
                         controller_digest=digest, workload_classes=classes, checked=checked)

    # -- installation ---------------------------------------------------------
    def install_on(self, model: Any, identity: Any) -> Admission:
        """Install the variant if admission passes, with its gate shut.  A refused
        install kills (and leaves the model as it was)."""
        admission = self.admit()
        if not admission.admitted:
            return admission
        try:
            gate, record = install(model, identity)
        except (VariantUnsupported, RuntimeError) as error:
            self.kill(f"the variant could not be installed: {type(error).__name__}: {error}")
            return Admission(False, f"installation refused: {error}",
                             controller_digest=admission.controller_digest,
                             checked=dict(admission.checked))
        self.gate, self.installed, self._model = gate, record, model
        self.admission = admission
        self._digest = admission.controller_digest
        return admission

    def prepare(self) -> Admission:
        """Admission without a model: a shut gate and nothing installed behind it."""
        admission = self.admit()
        if admission.admitted:
            self.gate = VariantGate()
            self.admission = admission
            self._digest = admission.controller_digest
        return admission

    # -- per dispatch ---------------------------------------------------------
    def for_dispatch(self, workload_class: str, route: str) -> ActivationRecord:
        """Open the gate for the dispatch about to run, or shut it, and say why.  After
        the first dispatch of a (class, route) pair this is a digest compare, a dict
        lookup and at most one gate write."""
        if not self.enabled or self.gate is None or self.learner is None:
            return _reference_record(self.disabled_reason or "no variant is installed", workload_class)
        if self.gate.killed:
            return self._killed_record(workload_class)
        if self.monitor is not None and self.monitor.requalification_required:
            if self.gate.active:
                self.gate.close("requalification is required")
            return _reference_record("passive monitoring requires a requalification before this "
                                     "action is used again", workload_class,
                                     state=REQUALIFICATION_REQUIRED)
        digest = self.learner.digest
        if digest != self._digest:
            # the controller changed: re-read it and drop every record built on the old state
            self._records.clear()
            state = self.learner.recommendation(self.action_id, workload_class).local_learning_state
            if state != CANDIDATE_QUALIFIED and self._digest:
                self.kill("the controller state changed and no longer qualifies this action")
                return self._killed_record(workload_class)
            self._digest = digest
            self.admission = Admission(True, "admitted on the current controller state",
                                       action_id=self.action_id, controller_digest=digest)
        record = self._records.get((workload_class, route))
        if record is None:
            record = self._records[(workload_class, route)] = self._record_for(workload_class, route, digest)
        if record.effective_action == CANDIDATE:
            if not self.gate.active:
                self.gate.open(record.activation_reason)
        elif self.gate.active:
            self.gate.close(record.activation_reason)
        return record

    def _record_for(self, workload_class: str, route: str, digest: str) -> ActivationRecord:
        rec = self.learner.recommendation(self.action_id, workload_class)
        state, evidence = rec.local_learning_state, rec.evidence_count
        if route not in ELIGIBLE_ROUTES:
            return _reference_record(f"route {route!r} is outside {list(ELIGIBLE_ROUTES)}",
                                     workload_class, state, evidence, digest)
        if state != CANDIDATE_QUALIFIED:
            return _reference_record(f"workload class {workload_class!r} is {state}",
                                     workload_class, state, evidence, digest)
        return ActivationRecord(REFERENCE, CANDIDATE, state, evidence, digest,
                                f"the local controller qualifies {workload_class!r} on "
                                f"{evidence} accepted sessions", workload_class)

    def _killed_record(self, workload_class: str) -> ActivationRecord:
        return _reference_record(f"killed: {self.gate.reason if self.gate else 'unknown'}",
                                 workload_class)

    def after_dispatch(self, record: ActivationRecord, telemetry: Any) -> dict[str, Any] | None:
        """After a candidate dispatch: nothing, or a kill when the telemetry reports
        fallbacks or correctness errors."""
        if record.effective_action != CANDIDATE:
            return None
        reasons = [f"{n} {what}" for n, what in
                   ((getattr(telemetry, "fallbacks", 0), "fallbacks in the candidate path"),
                    (getattr(telemetry, "correctness_errors", 0), "correctness errors")) if n]
        return self.kill("; ".join(reasons)) if reasons else None

    def serve(self, workload_class: str, route: str, call: Callable[[], Any],
              telemetry: Callable[[], Any] | None = None) -> tuple[Any, ActivationRecord]:
        """One dispatch: set the gate, run `call`, then `after_dispatch` on `telemetry()`.
        A candidate dispatch that raises kills before the exception propagates."""
        record = self.for_dispatch(workload_class, route)
        try:
            result = call()
        except BaseException as error:
            if record.effective_action == CANDIDATE:
                self.kill(f"an exception in the candidate path: {type(error).__name__}")
            raise
        if telemetry is not None:
            self.after_dispatch(record, telemetry())
        return result, record

    def kill(self, reason: str, detail: Mapping[str, Any] | None = None) -> dict[str, Any]:
        """Shut the gate for good, put the original modules back and persist the kill."""
        if self.gate is not None:
            self.gate.kill(reason)
        self._records.clear()
        restored = uninstall(self._model) if self._model is not None else 0
        self.enabled = False
        self.disabled_reason = f"killed: {reason}"
        persisted = str(write_kill(self.state_path, reason, detail)) if self.state_path is not None else None
        event = {"killed": True, "reason": reason, "projections_restored": restored,
                 "detail": dict(detail or {}), "persisted_to": persisted}
        self.events.append(event)
        return event

    def status(self) -> dict[str, Any]:
        gate = None if self.gate is None else {"active": self.gate.active, "killed": self.gate.killed,
                                                "reason": self.gate.reason}
        return {"schema": SCHEMA, "enabled": self.enabled, "default_enabled": False,
                "disabled_reason": self.disabled_reason, "action_id": self.action_id,
                "installed": self.installed, "gate": gate, "killed_at_start": self.killed_at_start,
                "requalification_required": (self.monitor.requalification_required
                                             if self.monitor is not None else None),
                "events": list(self.events)}
