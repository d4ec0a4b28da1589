"""The engine's admission of the K=3840 decode kernel: an opt-in knob, acted on once at load.

Mirrors the part of ironmule/runtime.py and ironmule/tune.py that reaches the hot path:
`Knobs.k3840_matvec` (runtime.py:35, off by default), `Engine.admit_k3840`
(runtime.py:434-449) and the one place that calls it, right after the model is loaded
and before any token (tune.py:426-429).  The rest of the reference's engine (KV caches,
prefill/decode bodies, speculation, wired memory, the other knobs) belongs to the
runtime this build leaves out; an `Engine` here holds a torch model whose projections are
`QuantizedLinear`s and does only what admission needs.

The rules the reference states and this keeps:

* the knob is off by default, and an engine built without it never touches the model;
* admission happens at most once per engine, with the model's identity, and never on the
  per-token path (`admit_k3840` after the first call returns None);
* a refusal raises `qmv_k3840.K3840Unsupported` with the model unchanged: a caller that
  asked for the kernel must not silently get something else, and decides itself whether
  to continue without it;
* the admission record says what was swapped; `close` puts the original modules back.
"""

from __future__ import annotations

import threading
from dataclasses import asdict, dataclass
from typing import Any

import torch

from . import qmv_k3840


@dataclass(frozen=True)
class Knobs:
    """Engine switches that reach the qmv path.  Only `k3840_matvec` does: it asks for
    the K=3840 decode kernel, admitted at load only."""

    k3840_matvec: bool = False

    def as_dict(self) -> dict[str, Any]:
        return asdict(self)

    def key(self) -> str:
        return "|".join(f"{name}={value}" for name, value in sorted(self.as_dict().items()))


BASELINE = Knobs()


class Engine:
    """A loaded model and its knobs.  `admit_k3840` is pending from construction until it
    has run once, so an engine built directly (without `load_engine`) runs the library
    path until someone admits the kernel with the model's identity."""

    def __init__(self, model: torch.nn.Module, knobs: Knobs = BASELINE) -> None:
        self.model = model
        self.knobs = knobs
        self.model_identity: Any = None
        self.k3840_admission: dict[str, Any] | None = None
        self._k3840_pending = bool(knobs.k3840_matvec)
        self._lock = threading.Lock()
        self._closed = False

    @property
    def k3840_pending(self) -> bool:
        return self._k3840_pending

    def admit_k3840(self, identity: Any) -> dict[str, Any] | None:
        """Admit the opt-in kernel, once, before any token: the admission record, or None
        when the knob is off or admission already ran.  A refusal raises
        K3840Unsupported, the model is left as it was and the admission stays pending."""
        with self._lock:
            if not self._k3840_pending:
                return None
            if self._closed:
                raise RuntimeError("the engine is closed")
            record = qmv_k3840.enable(self.model, identity)
            self._k3840_pending = False
            self.k3840_admission = record
            return record

    def close(self) -> int:
        """Put back every module the admission swapped, at most once.  Returns how many."""
        with self._lock:
            if self._closed:
                return 0
            self._closed = True
            if self.k3840_admission is None:
                return 0
            return qmv_k3840.disable(self.model)


def load_engine(model: torch.nn.Module, knobs: Knobs = BASELINE, identity: Any = None) -> Engine:
    """An engine over an already built model, with the kernel admitted if the knob asks
    for it.  Admission runs here because it needs the identity, and only here."""
    engine = Engine(model, knobs)
    engine.model_identity = identity
    engine.admit_k3840(identity)
    return engine
