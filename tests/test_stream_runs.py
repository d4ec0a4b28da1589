"""CPU check of the streaming engine's run plan and claim protocol.

`tests/stream_runs_sim.cpp` compiles ironmule_amd/csrc/stream_runs.h (the header the
independent-stage kernel uses for its plan and its two cursors) with g++ and simulates
the kernel's wavefronts under random interleavings over several launches that share the
claim counters.  It requires every tile computed once by the wavefront that loaded it and
every claim counter back at zero after each launch.  The same simulation with the old
rule for the last claimed run's length (every claimed run dyn_run tiles long) must fail:
that rule left a counter behind whenever the last run was short.
"""

from __future__ import annotations

import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
SOURCE = os.path.join(HERE, "stream_runs_sim.cpp")


@pytest.fixture(scope="module")
def sim(tmp_path_factory):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ is not installed")
    exe = str(tmp_path_factory.mktemp("sim") / "stream_runs_sim")
    subprocess.run([gxx, "-O2", "-std=c++17", "-Wall", "-Werror", SOURCE, "-o", exe], check=True)
    return exe


def _run(exe, *args):
    return subprocess.run([exe, *map(str, args)], capture_output=True, text=True, timeout=300)


@pytest.mark.parametrize("seed", [1, 7, 20261201])
def test_claim_protocol(sim, seed):
    """Fixed cases (one workgroup over 1250 tiles, the 20480-tile layer program at 1 and
    37 workgroups, tiny programs) and 150 random (tiles, grid, claimed run, claimed share)
    cases, 6 launches each."""
    proc = _run(sim, seed, 150, 6)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    assert proc.stdout.startswith("ok "), proc.stdout


def test_old_last_run_length_is_caught(sim):
    """With the last claimed run as long as the others, the wavefront that draws it can
    leave the loop before its load cursor makes its failed claim; the simulation must see
    the counter left behind."""
    proc = _run(sim, "--old-length", 1, 150, 6)
    assert proc.returncode == 1, proc.stdout + proc.stderr
    assert "counter left at" in proc.stdout or "computed 0 times" in proc.stdout, proc.stdout
