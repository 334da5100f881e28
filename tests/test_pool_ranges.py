"""The udmabuf pools' host-current ranges (llm-kv260_amd/csrc/pool_ranges.h,
used by shim.hip's lazy clean and invalidate), checked on the CPU against a
byte map (tests/pool_ranges_sim.cpp): random adds, removes and window
queries keep the set disjoint, merged and equal to the bytes marked; an add
that does not merge touching ranges (planted) is caught."""

from __future__ import annotations

import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def sim(tmp_path_factory):
    exe = str(tmp_path_factory.mktemp("pool_ranges") / "pool_ranges_sim")
    subprocess.run(["g++", "-O2", "-std=c++17", "-Wall", "-Wextra", "-Werror",
                    "-I", os.path.join(ROOT, "llm-kv260_amd", "csrc"),
                    os.path.join(ROOT, "tests", "pool_ranges_sim.cpp"), "-o", exe], check=True)
    return exe


def run(exe, size, ops, seed, plant=0):
    p = subprocess.run([exe, str(size), str(ops), str(seed), str(plant)], capture_output=True, text=True,
                       timeout=120)
    return p.returncode, p.stdout.strip()


@pytest.mark.parametrize("size,seed", [(64, 1), (256, 2), (4096, 3)])
def test_random_operations_match_a_byte_map(sim, size, seed):
    rc, out = run(sim, size, 20000, seed)
    assert rc == 0 and out == "ops 20000 ok", out


def test_planted_unmerged_add_is_caught(sim):
    rc, out = run(sim, 64, 20000, 1, plant=1)
    assert rc == 1 and "unmerged" in out, out
