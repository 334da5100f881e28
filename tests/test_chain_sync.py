"""The one-launch chain's grid barrier protocol, checked on the CPU with threads
(tests/chain_sync_sim.cpp over llm-kv260_amd/csrc/chain_sync.h, the kernel's
own state layout and epoch arithmetic): no workgroup passes a barrier before
every workgroup finished the step, across launches and across 2^32, and a
wait that gives up ends every workgroup's wait and leaves a clean state for
the next launch. A planted bug (polling for the previous epoch) must fail."""

from __future__ import annotations

import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def sim(tmp_path_factory):
    exe = str(tmp_path_factory.mktemp("chain_sync") / "chain_sync_sim")
    subprocess.run(["g++", "-O2", "-std=c++17", "-pthread", "-Wall", "-Wextra", "-Werror",
                    "-I", os.path.join(ROOT, "llm-kv260_amd", "csrc"),
                    os.path.join(ROOT, "tests", "chain_sync_sim.cpp"), "-o", exe], check=True)
    return exe


def run(exe, G, n, launches, spin, stall=-1, gen0=0, plant=0):
    p = subprocess.run([exe, str(G), str(n), str(launches), str(spin), str(stall), hex(gen0), str(plant)],
                       capture_output=True, text=True, timeout=120)
    return p.returncode, p.stdout


@pytest.mark.parametrize("G", [1, 7, 64, 256])
def test_barrier_orders_every_step(sim, G):
    rc, out = run(sim, G, 65, 4, 10**7)
    assert rc == 0, out
    assert "early passes in all: 0" in out


def test_barrier_across_the_32_bit_wrap(sim):
    rc, out = run(sim, 64, 65, 4, 10**7, gen0=0xFFFFFF80)
    assert rc == 0, out
    assert "gen 4294967232 -> 0" in out


def test_give_up_restores_the_state(sim):
    """Launch 1 stalls one workgroup past the others' spin limit: every wait
    ends, one timeout is counted, the counters, GEN and ABORT are cleared,
    and launch 2 runs normally from there."""
    rc, out = run(sim, 64, 10, 3, 20000, stall=1)
    assert rc == 0, out
    lines = out.splitlines()
    assert "gave up 0" not in lines[1] and lines[1].endswith("ok"), out
    assert "gen 0 -> 9" in lines[2], out


def test_planted_bug_is_caught(sim):
    rc, out = run(sim, 64, 65, 2, 10**7, plant=1)
    assert rc == 1, out
    early = int(out.strip().splitlines()[-1].split(":")[1])
    assert early > 0, out
