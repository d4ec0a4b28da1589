"""CPU check of the streaming engine's run plan and claim protocol.

`tests/stream_runs_sim.cpp` compiles ironmule_amd/csrc/stream_runs.h (the header the
independent-stage kernel uses for its plan and its two cursors) with g++ and simulates
the kernel's wavefronts under random interleavings over several launches that share the
claim counters.  It requires every tile computed once by the wavefront that loaded it and
every claim counter back at zero after each launch, over random tile counts, grids of 4-
and 12-wavefront workgroups, claimed shares, and long and short (tail) claimed run
lengths.  The same simulation with run lengths that ignore where a shard's tiles end must
fail: that rule left a counter behind whenever a last run was short.
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
    37 workgroups, the 20- and 36-layer headline programs at 256 x 12 wavefronts, tiny
    programs) and 80 random cases, 4 launches each."""
    proc = _run(sim, seed, 80, 4)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    assert proc.stdout.startswith("ok "), proc.stdout


def test_run_lengths_that_ignore_the_shard_end_are_caught(sim):
    """With every claimed run as long as its kind, a shard's last run either stops short of
    the wavefront's failed claim (a counter left behind) or runs into the next shard's
    tiles (computed twice); the simulation must report one of them."""
    proc = _run(sim, "--old-length", 1, 150, 4)
    assert proc.returncode == 1, proc.stdout + proc.stderr
    assert proc.stdout.startswith("FAIL") and ("counter left at" in proc.stdout
                                               or "computed" in proc.stdout), proc.stdout
