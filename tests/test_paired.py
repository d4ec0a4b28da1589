"""The pairing scheduler on the CPU (PairedGroupedExecutor over a recording backend): pairs
form only from two ready requests with one KV capacity, everything else steps alone,
nothing waits for a partner, and the round-robin order serves every request (the rules of
ironmule/paired_research.py:245-272).  Nothing here launches a kernel."""

from __future__ import annotations

import pytest

from ironmule_amd.paired import PAIR_WIDTH, PairedBackend, PairedGroupedExecutor, Session


class Recording(PairedBackend):
    """Next token = previous + 1 (+ 100 when paired), and a log of every call."""

    def __init__(self):
        super().__init__(model=None, share=True)
        self.calls = []

    def step(self, state, token, capacity):
        self.calls.append(("solo", state, token, capacity))
        return None, token + 1

    def step_pair(self, states, tokens, capacity):
        self.calls.append(("pair", tuple(states), tuple(tokens), capacity))
        return [(None, t + 101) for t in tokens]


def _sessions(*specs):
    return [Session(rid=name, tokens=[first], max_tokens=n, state=name, capacity=cap)
            for name, first, n, cap in specs]


def test_two_ready_requests_step_as_a_pair():
    backend = Recording()
    ex = PairedGroupedExecutor(backend, share=True)
    a, b = _sessions(("a", 0, 3, 0), ("b", 10, 3, 0))
    ex.run([a, b], capacity=64)
    assert a.tokens == [0, 101, 202] and b.tokens == [10, 111, 212]
    assert ex.paired_steps == 2 and ex.solo_steps == 0
    assert [c[0] for c in backend.calls] == ["pair", "pair"] and backend.calls[0][3] == 64


def test_a_lone_request_steps_alone_at_once():
    backend = Recording()
    ex = PairedGroupedExecutor(backend, share=True)
    (a,) = _sessions(("a", 0, 4, 0))
    ex.run([a], capacity=32)
    assert a.tokens == [0, 1, 2, 3] and ex.paired_steps == 0 and ex.solo_steps == 3


def test_different_capacities_never_pair():
    backend = Recording()
    ex = PairedGroupedExecutor(backend, share=True)
    a, b = _sessions(("a", 0, 2, 16), ("b", 5, 2, 32))
    ex.run([a, b], capacity=64)
    assert ex.paired_steps == 0 and ex.solo_steps == 2
    assert [(c[0], c[3]) for c in backend.calls] == [("solo", 16), ("solo", 32)]


def test_three_requests_rotate_and_finish():
    """A pair, then the third with the first again: served requests go to the back, and a
    finished request leaves its partner to step alone."""
    backend = Recording()
    ex = PairedGroupedExecutor(backend, share=True)
    a, b, c = _sessions(("a", 0, 3, 0), ("b", 10, 2, 0), ("c", 20, 2, 0))
    ex.run([a, b, c], capacity=8)
    assert [call[1] for call in backend.calls] == [("a", "b"), ("c", "a")]
    assert a.done and b.done and c.done
    assert ex.paired_steps == 2 and ex.solo_steps == 0


def test_width_one_never_pairs_and_widths_are_bounded():
    backend = Recording()
    ex = PairedGroupedExecutor(backend, share=True, max_width=1)
    a, b = _sessions(("a", 0, 2, 0), ("b", 10, 2, 0))
    ex.run([a, b], capacity=8)
    assert ex.paired_steps == 0 and ex.solo_steps == 2
    assert PAIR_WIDTH == 2
    with pytest.raises(ValueError):
        PairedGroupedExecutor(backend, share=True, max_width=0)
    with pytest.raises(ValueError):
        PairedGroupedExecutor(backend, share=True, max_width=33)
