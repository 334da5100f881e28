"""GPU parity at the five workload configurations' full sizes.

Every output is compared with the oracle's SHA-256 in tests/golden/configs.json
(written by tests/golden/make_fixtures.py from the same seeded inputs), so a
single differing bit anywhere in a 128256-row LM head or a 65-matrix decode
step fails. The weights are quantized on the GPU by the engine's own Q4_0
kernel, and their digests are checked too.
"""

from __future__ import annotations

import ctypes
import hashlib
import json
import os

import numpy as np
import pytest

from gpu_helpers import dev, host, poisoned_f32
from kv260gemv import configs as cf

pytestmark = pytest.mark.gpu

with open(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "configs.json")) as _f:
    FIX = json.load(_f)


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def device_blocks(gpu, m: cf.Matrix):
    """Q4_0 rows of the seeded weights, quantized on the GPU chunk by chunk."""
    import torch
    out = torch.empty((m.rows, m.k // 32 * 18), dtype=torch.uint8, device="cuda")
    for r0, w in cf.weight_chunks(m):
        out[r0:r0 + w.shape[0]] = gpu.quantize_q4_0(dev(w))
    return out


class Step(ctypes.Structure):
    _fields_ = [("w", ctypes.c_void_p), ("x", ctypes.c_void_p), ("y", ctypes.c_void_p),
                ("rows", ctypes.c_int), ("k", ctypes.c_int)]


def step_array(mats, xs, ys, shapes):
    return (Step * len(shapes))(*[Step(mats[i].data_ptr(), xs[i].data_ptr(), ys[i].data_ptr(), r, k)
                                  for i, (r, k) in enumerate(shapes)])


def check_matrix(gpu, m: cf.Matrix, rec: dict, blocks=None):
    """Every M=1 entry point on one configuration matrix, against its digests."""
    import torch
    if blocks is None:
        blocks = device_blocks(gpu, m)
    assert sha(host(blocks)) == rec["q4_0"], f"{m.name}: Q4_0 weights"
    x = dev(cf.activation(m))
    xq, xd = gpu.quantize_q8_0(x)
    assert sha(host(xq)) == rec["xq"] and sha(host(xd).view(np.uint16)) == rec["xd"], f"{m.name}: Q8_0"
    outs = {
        "gemv_q4_0": gpu.gemv_q4_0(blocks, m.k, xq, xd),
        "gemv_engine": gpu.gemv_engine(blocks, m.k, gpu.quantize_q8_0_engine(x), out=poisoned_f32(m.rows)),
        "gemv_q4_0_f32": gpu.gemv_q4_0_f32(blocks, m.k, x, out=poisoned_f32(m.rows)),
    }
    qb = torch.cat([xd.view(torch.uint8).reshape(-1, 2), xq.view(torch.uint8).reshape(-1, 32)], dim=1)
    outs["gemv_q8_0_blocks"] = gpu.gemv_q8_0_blocks(blocks, m.k, qb.contiguous().reshape(-1),
                                                    out=poisoned_f32(m.rows))
    for name, y in outs.items():
        got = host(y)
        assert sha(got) == rec["y"], f"{m.name} {name}: y differs (head {got[:4].view(np.uint32)})"
    return blocks


def test_config0_o_proj(gpu):
    check_matrix(gpu, cf.O_PROJ, FIX["config0"][0])


def test_config1_layer_shapes_and_batch(gpu):
    import torch
    mats, xs, ys = [], [], []
    for m, rec in zip(cf.LAYER_SHAPES, FIX["config1"]):
        mats.append(check_matrix(gpu, m, rec))
        xs.append(dev(cf.activation(m)))
        ys.append(poisoned_f32(m.rows))
    shapes = [(m.rows, m.k) for m in cf.LAYER_SHAPES]
    steps = step_array(mats, xs, ys, shapes)
    gpu.check("w4a8_gemv_batch", gpu.lib().w4a8_gemv_batch(ctypes.cast(steps, ctypes.c_void_p), len(shapes),
                                                          torch.cuda.current_stream().cuda_stream))
    for y, rec in zip(ys, FIX["config1"]):
        assert sha(host(y)) == rec["y"], f"batch {rec['name']}"


def test_config2_lm_head_three_copies(gpu):
    """128256 x 2048 logits, byte-exact and the same greedy token, from each of three
    weight copies (443 MB, past the 256 MB Infinity Cache)."""
    m, rec = cf.LM_HEAD, FIX["config2"][0]
    base = check_matrix(gpu, m, rec)
    copies = [base, base.clone(), base.clone()]
    x_eng = gpu.quantize_q8_0_engine(dev(cf.activation(m)))
    y = poisoned_f32(m.rows)
    for rep in range(6):
        c = copies[rep % 3]
        y.fill_(float("nan"))
        gpu.gemv_engine(c, m.k, x_eng, out=y)
        got = host(y)
        assert sha(got) == rec["y"], f"copy {rep % 3}"
        assert int(np.argmax(got)) == rec["argmax"]


@pytest.fixture(scope="module")
def chain_blocks(gpu):
    """Config 3's 65 weight matrices, quantized on the GPU once for every
    config-3 test and checked against their digests."""
    mats = []
    for m, rec in zip(cf.decode_chain(), FIX["config3"]):
        b = device_blocks(gpu, m)
        assert sha(host(b)) == rec["q4_0"], f"{m.name}: Q4_0 weights"
        mats.append(b)
    return mats


def test_config3_decode_chain_400_steps(gpu, chain_blocks):
    """The 65-matrix chain: byte-exact after step 0 and after step 399, through the
    dependent chain entry point, and once through the batch."""
    import torch
    chain, recs = cf.decode_chain(), FIX["config3"]
    mats = chain_blocks
    xs = [dev(cf.activation(m)) for m in chain]
    ys = [poisoned_f32(m.rows) for m in chain]
    shapes = [(m.rows, m.k) for m in chain]
    steps = step_array(mats, xs, ys, shapes)
    ptr = ctypes.cast(steps, ctypes.c_void_p)
    L = gpu.lib()
    stream = torch.cuda.current_stream().cuda_stream

    def check(what):
        for m, y, rec in zip(chain, ys, recs):
            assert sha(host(y)) == rec["y"], f"{what}: {m.name}"
        assert int(np.argmax(host(ys[-1]))) == recs[-1]["argmax"]

    gpu.check("w4a8_chain_gemv", L.w4a8_chain_gemv(ptr, len(chain), stream))
    check("chain step 0")
    for y in ys:
        y.fill_(float("nan"))
    for _ in range(399):
        gpu.check("w4a8_chain_gemv", L.w4a8_chain_gemv(ptr, len(chain), stream))
    check("chain step 399")
    for y in ys:
        y.fill_(float("nan"))
    gpu.check("w4a8_gemv_batch", L.w4a8_gemv_batch(ptr, len(chain), stream))
    check("batch")


def test_config3_chain_plan_400_passes(gpu, chain_blocks):
    """The headline issuer at full size: config 3's 65 matrices as a chain plan,
    one pass, then 400 passes in one launch (26,000 packets, past the queue's
    16,384-slot ring, so the launch waits for room in it), then two passes of
    the timed launch; all 65 digests after each. The timed launch's stamps:
    every dispatch's span is positive, and each dispatch starts after the one
    before it ended (the packets' barrier bits)."""
    import torch
    chain, recs = cf.decode_chain(), FIX["config3"]
    xs = [dev(cf.activation(m)) for m in chain]
    ys = [poisoned_f32(m.rows) for m in chain]
    steps = step_array(chain_blocks, xs, ys, [(m.rows, m.k) for m in chain])
    L = gpu.lib()
    torch.cuda.synchronize()
    plan = ctypes.c_void_p()
    gpu.check("w4a8_chain_plan_create", L.w4a8_chain_plan_create(ctypes.cast(steps, ctypes.c_void_p), len(chain),
                                                                 ctypes.byref(plan)))
    try:
        for passes in (1, 400):
            for y in ys:
                y.fill_(float("nan"))
            torch.cuda.synchronize()
            gpu.check("w4a8_chain_plan_launch", L.w4a8_chain_plan_launch(plan, passes))
            gpu.check("w4a8_chain_plan_wait", L.w4a8_chain_plan_wait(plan, 60000))
            for m, y, rec in zip(chain, ys, recs):
                assert sha(host(y)) == rec["y"], f"plan, {passes} passes: {m.name}"
        for y in ys:
            y.fill_(float("nan"))
        grid = [L.w4a8_chain_plan_workgroups(plan, j) for j in range(len(chain))]
        assert L.w4a8_chain_plan_workgroups(plan, -1) == sum(grid) and min(grid) > 0
        stamps = torch.zeros(2 * 2 * sum(grid), dtype=torch.int64, device="cuda")
        torch.cuda.synchronize()
        gpu.check("w4a8_chain_plan_launch_timed", L.w4a8_chain_plan_launch_timed(plan, 2, stamps.data_ptr()))
        gpu.check("w4a8_chain_plan_wait", L.w4a8_chain_plan_wait(plan, 60000))
        for m, y, rec in zip(chain, ys, recs):
            assert sha(host(y)) == rec["y"], f"timed plan: {m.name}"
        wg = host(stamps).view(np.uint64).reshape(-1, 2).astype(np.int64)
        assert (wg > 0).all() and (wg[:, 1] >= wg[:, 0]).all(), "every workgroup stamps its slot"
        first = np.concatenate(([0], np.cumsum(grid * 2)[:-1]))
        st = np.stack([np.minimum.reduceat(wg[:, 0], first), np.maximum.reduceat(wg[:, 1], first)], axis=1)
        span = st[:, 1] - st[:, 0]
        assert (span > 0).all(), span
        assert (st[1:, 0] >= st[:-1, 1]).all(), "a dispatch started before the previous one ended"
        hz = ctypes.c_int64()
        gpu.check("w4a8_wall_clock_hz", L.w4a8_wall_clock_hz(ctypes.byref(hz)))
        us = span / hz.value * 1e6
        assert us.max() < 1000.0, us.max()
    finally:
        gpu.check("w4a8_chain_plan_destroy", L.w4a8_chain_plan_destroy(plan))


def test_config3_overlapped_plan_400_passes(gpu, chain_blocks):
    """Config 3's 65 matrices as an overlapped plan (each step's workgroups
    start during the step before and wait for it in the kernel): all 65
    digests after one pass and after 400 passes in one launch."""
    import torch
    chain, recs = cf.decode_chain(), FIX["config3"]
    xs = [dev(cf.activation(m)) for m in chain]
    ys = [poisoned_f32(m.rows) for m in chain]
    steps = step_array(chain_blocks, xs, ys, [(m.rows, m.k) for m in chain])
    L = gpu.lib()
    torch.cuda.synchronize()
    plan = ctypes.c_void_p()
    gpu.check("w4a8_chain_plan_create_overlapped",
              L.w4a8_chain_plan_create_overlapped(ctypes.cast(steps, ctypes.c_void_p), len(chain), ctypes.byref(plan)))
    try:
        for passes in (1, 400):
            for y in ys:
                y.fill_(float("nan"))
            torch.cuda.synchronize()
            gpu.check("w4a8_chain_plan_launch", L.w4a8_chain_plan_launch(plan, passes))
            gpu.check("w4a8_chain_plan_wait", L.w4a8_chain_plan_wait(plan, 60000))
            for m, y, rec in zip(chain, ys, recs):
                assert sha(host(y)) == rec["y"], f"overlapped plan, {passes} passes: {m.name}"
    finally:
        gpu.check("w4a8_chain_plan_destroy", L.w4a8_chain_plan_destroy(plan))


def test_config3_one_launch_chain(gpu, chain_blocks):
    """The 65-matrix chain as one cooperative launch (W4A8_CHAIN_ONE_LAUNCH):
    byte-exact after the first launch and after 50 more, no wait given up."""
    import torch
    chain, recs = cf.decode_chain(), FIX["config3"]
    mats = chain_blocks
    xs = [dev(cf.activation(m)) for m in chain]
    ys = [poisoned_f32(m.rows) for m in chain]
    steps = step_array(mats, xs, ys, [(m.rows, m.k) for m in chain])
    ptr = ctypes.cast(steps, ctypes.c_void_p)
    L = gpu.lib()
    stream = torch.cuda.current_stream().cuda_stream
    assert L.w4a8_chain_set_mode(0) == 0
    try:
        assert L.w4a8_chain_timeouts() >= 0
        for launches, what in ((1, "first launch"), (50, "after 51 launches")):
            for y in ys:
                y.fill_(float("nan"))
            for _ in range(launches):
                gpu.check("w4a8_chain_gemv", L.w4a8_chain_gemv(ptr, len(chain), stream))
            for m, y, rec in zip(chain, ys, recs):
                assert sha(host(y)) == rec["y"], f"{what}: {m.name}"
        assert L.w4a8_chain_timeouts() == 0
    finally:
        L.w4a8_chain_set_mode(1)


def test_config3_prefill24(gpu, chain_blocks):
    """A 24-token prompt through the chain's 65 matrices (quantize the rows, then
    the M > 1 GEMM), every output byte-exact against the oracle's digests."""
    chain, recs = cf.decode_chain(), FIX["config3_prefill24"]
    for j, (m, b, rec) in enumerate(zip(chain, chain_blocks, recs)):
        x_rows = gpu.quantize_q8_0_engine(dev(cf.prefill_activation(j, cf.PREFILL_M, m.k)))
        assert sha(host(x_rows)[:, :m.k]) == rec["xq"], m.name
        y = poisoned_f32((cf.PREFILL_M, m.rows))
        gpu.gemm_engine(b, m.k, x_rows, out=y)
        got = host(y)
        assert sha(got) == rec["y"], f"prefill {m.name}: head {got.reshape(-1)[:4].view(np.uint32)}"


def test_config4_m_sweep(gpu):
    """M = 1 .. 64 activation rows through the int8-MFMA path, each row byte-exact."""
    recs = {(r["name"], r["m"]): r for r in FIX["config4"]}
    for m in cf.GEMM_SHAPES:
        blocks = device_blocks(gpu, m)
        for mrows in cf.GEMM_M:
            rec = recs[(m.name, mrows)]
            x_rows = gpu.quantize_q8_0_engine(dev(cf.gemm_activation(mrows, m.k)))
            assert sha(host(x_rows)[:, :m.k]) == rec["xq"], (m.name, mrows)
            y = poisoned_f32((mrows, m.rows))
            gpu.gemm_engine(blocks, m.k, x_rows, out=y)
            got = host(y)
            assert sha(got) == rec["y"], f"{m.name} M={mrows}: head {got.reshape(-1)[:4].view(np.uint32)}"
