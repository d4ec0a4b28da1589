"""The split workspace cache of the ctypes boundary (ironmule_amd/_native.py), on the CPU:
a (device, stream) keeps one zero-filled workspace, a larger need replaces it, and the one
replaced stays alive (a graph captured earlier may still hold its pointer).  Device
allocation is stood in for by CPU tensors; nothing here launches a kernel."""

from __future__ import annotations

import gc
import weakref

import pytest
import torch

from ironmule_amd import _native


@pytest.fixture
def cpu_workspaces(monkeypatch):
    monkeypatch.setattr(_native, "_workspaces", {})
    monkeypatch.setattr(_native, "_retired", [])
    monkeypatch.setattr(_native, "_workspace_key", lambda device, stream: (0, id(stream)))
    monkeypatch.setattr(_native, "_zeroed", lambda words, index, stream: torch.zeros(words))
    return _native


def test_one_workspace_per_stream_reused_while_it_fits(cpu_workspaces):
    n = cpu_workspaces
    a, b = object(), object()
    w1 = n._workspace(4096, "cuda", a)
    assert w1.numel() * 4 >= 4096 and not w1.any()
    assert n._workspace(1000, "cuda", a) is w1
    assert n._workspace(1000, "cuda", b) is not w1


def test_growth_keeps_the_outgrown_workspace_alive(cpu_workspaces):
    n = cpu_workspaces
    s = object()
    small = n._workspace(1024, "cuda", s)
    ref = weakref.ref(small)
    big = n._workspace(1 << 20, "cuda", s)
    assert big is not small and big.numel() * 4 >= 1 << 20
    del small
    gc.collect()
    assert ref() is not None and ref() in n._retired
    assert n._workspace(4096, "cuda", s) is big  # a smaller need reuses the larger one
