"""The chain plan's packet ring, checked on the CPU with threads
(tests/plan_ring_sim.cpp over llm-kv260_amd/csrc/plan_ring.h, the launch
loop's own wait): a producer writing many times the ring's size through a
slow consumer never overwrites an untaken packet and leaves no hole; a
launch that runs far longer than the give-up bound but keeps progressing
never gives up; a consumer that stops gives up the launch with every slot it
took written, so the queue drains cleanly once the consumer resumes. The old
bound (measured from the launch's start) must fail the long-launch case."""

from __future__ import annotations

import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def sim(tmp_path_factory):
    exe = str(tmp_path_factory.mktemp("plan_ring") / "plan_ring_sim")
    subprocess.run(["g++", "-O2", "-std=c++17", "-pthread", "-Wall", "-Wextra", "-Werror",
                    "-I", os.path.join(ROOT, "llm-kv260_amd", "csrc"),
                    os.path.join(ROOT, "tests", "plan_ring_sim.cpp"), "-o", exe], check=True)
    return exe


def run(exe, size, packets, n, per_us, stall_at=-1, stall_ms=0, stall_s=10.0, plant=0):
    p = subprocess.run([exe, str(size), str(packets), str(n), str(per_us), str(stall_at), str(stall_ms),
                        str(stall_s), str(plant)], capture_output=True, text=True, timeout=120)
    return p.returncode, p.stdout.strip()


@pytest.mark.parametrize("size,n", [(8, 3), (16, 16), (64, 65)])
def test_wrapping_many_times_keeps_every_packet(sim, size, n):
    rc, out = run(sim, size, 20000, n, 0)
    assert rc == 0, out
    assert out.startswith("written 20000 read 20000 result OK errors 0"), out


def test_long_launch_that_progresses_never_gives_up(sim):
    """2,000 packets at 100 us each through an 8-slot ring: 0.2 s of launch
    against a 0.05 s bound on a stall."""
    rc, out = run(sim, 8, 2000, 5, 100, stall_s=0.05)
    assert rc == 0, out
    assert "result OK" in out and "written 2000 read 2000" in out, out


def test_stalled_consumer_gives_up_without_a_hole(sim):
    """The consumer stops before packet 40 for 0.5 s; the launch gives up
    after 0.1 s without progress, having written exactly the packets that fit,
    and the consumer takes every one of them when it resumes."""
    rc, out = run(sim, 16, 1000, 4, 0, stall_at=40, stall_ms=500, stall_s=0.1)
    assert rc == 0, out
    assert "result STALLED" in out, out
    written = int(out.split()[1])
    assert written == 40 + 16, out        # packets 0..39 taken, then a full ring


def test_planted_old_bound_is_caught(sim):
    """The bound measured from the launch's start gives up a launch that is
    progressing: the same long launch as above ends STALLED."""
    rc, out = run(sim, 8, 2000, 5, 100, stall_s=0.05, plant=1)
    assert "result STALLED" in out, out
