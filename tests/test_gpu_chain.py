"""The decode chain as one launch (w4a8_chain_gemv with every k in 2048..8192):
each step byte for byte against the oracle, against the one-kernel-per-step
mode, with a real step-to-step data dependency, inside a HIP graph, and the
bounded waits' give-up path forced from the host.

Every output buffer is poisoned with 0xAA first.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

import c_oracle as C
import q4_0_oracle as O
from gpu_helpers import assert_bytes_equal, dev, host, poisoned_f32

pytestmark = pytest.mark.gpu

ONE_LAUNCH, PER_STEP = 0, 1


class Step(ctypes.Structure):
    _fields_ = [("w", ctypes.c_void_p), ("x", ctypes.c_void_p), ("y", ctypes.c_void_p),
                ("rows", ctypes.c_int), ("k", ctypes.c_int)]


def _stream():
    import torch
    return torch.cuda.current_stream().cuda_stream


@pytest.fixture
def lib(gpu):
    """The library in one-launch mode with the default spin limit; the defaults
    (one launch per step) are restored after the test."""
    L = gpu.lib()
    assert L.w4a8_chain_set_mode(ONE_LAUNCH) == 0
    assert L.w4a8_chain_set_spin_limit(0) == 0
    assert L.w4a8_chain_timeouts() >= 0          # clear any count left by an earlier test
    yield L
    L.w4a8_chain_set_mode(PER_STEP)
    L.w4a8_chain_set_spin_limit(0)


def _independent(shapes, seed0):
    """Steps with their own weights and activations, and the oracle's outputs."""
    mats, xs, ys, wants = [], [], [], []
    for i, (rows, k) in enumerate(shapes):
        w = O.normal_f32((rows, k), seed0 + i, 0.02)
        x = O.normal_f32((1, k), seed0 + 500 + i)[0]
        blocks = C.quantize_q4_0(w)
        xq, xd = C.quantize_q8_0(x)
        mats.append(dev(blocks))
        xs.append(dev(x))
        ys.append(poisoned_f32(rows))
        wants.append(C.gemv_q4_0(blocks, k, xq, xd))
    steps = (Step * len(shapes))(*[Step(mats[i].data_ptr(), xs[i].data_ptr(), ys[i].data_ptr(), r, k)
                                   for i, (r, k) in enumerate(shapes)])
    return steps, (mats, xs), ys, wants


def _run(gpu, L, steps, n):
    gpu.check("w4a8_chain_gemv", L.w4a8_chain_gemv(ctypes.cast(steps, ctypes.c_void_p), n, _stream()))


SHAPES = {
    # layer shapes and a ragged LM-head-like tail (rounds of eight tiles per workgroup)
    "llama_layer": [(3072, 2048), (2048, 2048), (16384, 2048), (2048, 8192), (20000, 2048)],
    # one row, ragged rows, a tile of fewer than 64 chunks (k = 6144: two rows of 24 chunks)
    "ragged": [(1, 2048), (5, 4096), (300, 6144), (257, 8192), (9, 2048), (4097, 4096)],
    "single": [(64, 2048)],
}


@pytest.mark.parametrize("name", sorted(SHAPES))
def test_one_launch_matches_oracle_and_per_step(gpu, lib, name):
    shapes = SHAPES[name]
    steps, keep, ys, wants = _independent(shapes, 700)
    _run(gpu, lib, steps, len(shapes))
    one = [host(y).copy() for y in ys]
    assert lib.w4a8_chain_timeouts() == 0
    for i, (got, want) in enumerate(zip(one, wants)):
        assert_bytes_equal(got, want, f"{name} step {i} {shapes[i]}")
    for y in ys:
        y.fill_(float("nan"))
    assert lib.w4a8_chain_set_mode(PER_STEP) == 0
    _run(gpu, lib, steps, len(shapes))
    for i, y in enumerate(ys):
        assert_bytes_equal(host(y), one[i], f"{name} step {i}: per-step mode")


def test_one_launch_max_steps(gpu, lib):
    """96 steps (W4A8_CHAIN_MAX_STEPS) alternating k = 2048 and 8192."""
    shapes = [(64 + 32 * (i % 5), 2048 if i % 2 == 0 else 8192) for i in range(96)]
    steps, keep, ys, wants = _independent(shapes, 3000)
    _run(gpu, lib, steps, len(shapes))
    for i, (y, want) in enumerate(zip(ys, wants)):
        assert_bytes_equal(host(y), want, f"step {i}")
    assert lib.w4a8_chain_timeouts() == 0


def test_one_launch_data_dependency(gpu, lib):
    """x of every step after the first IS the previous step's y: the chain must
    read it only once every workgroup has written it. The oracle runs the same
    chain step by step on the CPU; both modes must match it byte for byte,
    and stay exact over repeated launches."""
    shapes = [(2048, 2048), (8192, 2048), (2048, 8192), (2048, 2048), (3072, 2048), (2048, 3072), (2048, 2048)]
    for (r0, _), (_, k1) in zip(shapes, shapes[1:]):
        assert r0 == k1
    blocks = [C.quantize_q4_0(O.normal_f32((r, k), 40 + i, 0.02)) for i, (r, k) in enumerate(shapes)]
    x0 = O.normal_f32((1, shapes[0][1]), 39)[0]
    wants, x = [], x0
    for b, (r, k) in zip(blocks, shapes):
        xq, xd = C.quantize_q8_0(x)
        x = C.gemv_q4_0(b, k, xq, xd)
        wants.append(x)
    mats = [dev(b) for b in blocks]
    xin = dev(x0)
    ys = [poisoned_f32(r) for r, _ in shapes]
    xs = [xin] + ys[:-1]
    steps = (Step * len(shapes))(*[Step(mats[i].data_ptr(), xs[i].data_ptr(), ys[i].data_ptr(), r, k)
                                   for i, (r, k) in enumerate(shapes)])
    for mode in (ONE_LAUNCH, PER_STEP, ONE_LAUNCH):
        assert lib.w4a8_chain_set_mode(mode) == 0
        for rep in range(3):
            for y in ys:
                y.fill_(float("nan"))
            _run(gpu, lib, steps, len(shapes))
            for i, (y, want) in enumerate(zip(ys, wants)):
                assert_bytes_equal(host(y), want, f"mode {mode} launch {rep} step {i}")
    assert lib.w4a8_chain_timeouts() == 0


def test_one_launch_graph_replays(gpu, lib):
    """The one-launch chain captured into a HIP graph: every replay, with eager
    work and synchronisations between them, equals the eager launch."""
    import torch
    shapes = SHAPES["llama_layer"]
    steps, keep, ys, wants = _independent(shapes, 900)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        _run(gpu, lib, steps, len(shapes))
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        gpu.check("w4a8_chain_gemv", lib.w4a8_chain_gemv(ctypes.cast(steps, ctypes.c_void_p), len(shapes),
                                                         torch.cuda.current_stream().cuda_stream))
    for rep in range(4):
        for y in ys:
            y.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for i, (y, want) in enumerate(zip(ys, wants)):
            assert_bytes_equal(host(y), want, f"replay {rep} step {i}")
        junk = torch.randn(1 << 20, device="cuda") * 2.0   # eager work between replays
        del junk
    assert lib.w4a8_chain_timeouts() == 0


def test_one_launch_give_up_and_recover(gpu, lib):
    """Forced from the host: with a spin limit of one poll, workgroups give up
    at the barriers, every kernel still ends, the launch is counted as timed
    out, and the barrier state is restored -- the next launch at the default
    limit is byte-exact and counts nothing."""
    shapes = [(2048, 2048), (16384, 2048), (2048, 8192)] * 8
    steps, keep, ys, wants = _independent(shapes, 1200)
    assert lib.w4a8_chain_set_spin_limit(1) == 0
    _run(gpu, lib, steps, len(shapes))
    _run(gpu, lib, steps, len(shapes))
    assert lib.w4a8_chain_timeouts() >= 1
    assert lib.w4a8_chain_set_spin_limit(0) == 0
    for rep in range(2):
        for y in ys:
            y.fill_(float("nan"))
        _run(gpu, lib, steps, len(shapes))
        for i, (y, want) in enumerate(zip(ys, wants)):
            assert_bytes_equal(host(y), want, f"after recovery, launch {rep} step {i}")
    assert lib.w4a8_chain_timeouts() == 0


def test_chain_mode_rejects_unknown(gpu, lib):
    assert lib.w4a8_chain_set_mode(2) == -2
    assert lib.w4a8_chain_set_mode(-1) == -2
