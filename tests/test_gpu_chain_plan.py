"""The decode chain as a plan (w4a8_chain_plan_*: raw AQL dispatches on the
library's own queue, no cache fences between steps): each step byte for byte
against the oracle and against w4a8_chain_gemv, over several passes and
launches; a step-to-step data dependency inside a pass and one that runs from
the last step of a pass into the first step of the next (the coherent-read
and write-through variants), readers of memory an earlier step already
cached; several launches before one wait; plans made and destroyed in turn.

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


class Step(ctypes.Structure):
    _fields_ = [("w", ctypes.c_void_p), ("x", ctypes.c_void_p), ("y", ctypes.c_void_p),
                ("rows", ctypes.c_int), ("k", ctypes.c_int)]


def _steps(mats, xs, ys, shapes):
    return (Step * len(shapes))(*[Step(mats[i].data_ptr(), xs[i].data_ptr(), ys[i].data_ptr(), r, k)
                                  for i, (r, k) in enumerate(shapes)])


class Plan:
    def __init__(self, gpu, steps, n, overlapped=False):
        import torch
        torch.cuda.synchronize()       # the plan's queue is not ordered with HIP streams
        self.L, self.gpu = gpu.lib(), gpu
        self.p = ctypes.c_void_p()
        create = self.L.w4a8_chain_plan_create_overlapped if overlapped else self.L.w4a8_chain_plan_create
        gpu.check("w4a8_chain_plan_create", create(ctypes.cast(steps, ctypes.c_void_p), n, ctypes.byref(self.p)))

    def run(self, passes=1):
        self.gpu.check("w4a8_chain_plan_launch", self.L.w4a8_chain_plan_launch(self.p, passes))
        self.gpu.check("w4a8_chain_plan_wait", self.L.w4a8_chain_plan_wait(self.p, 30000))

    def close(self):
        self.gpu.check("w4a8_chain_plan_destroy", self.L.w4a8_chain_plan_destroy(self.p))


def _independent(shapes, seed0):
    mats, xs, ys, wants = [], [], [], []
    for i, (rows, k) in enumerate(shapes):
        blocks = C.quantize_q4_0(O.normal_f32((rows, k), seed0 + i, 0.02))
        x = O.normal_f32((1, k), seed0 + 500 + i)[0]
        xq, xd = C.quantize_q8_0(x)
        mats.append(dev(blocks))
        xs.append(dev(x))
        ys.append(poisoned_f32(rows))
        wants.append(C.gemv_q4_0(blocks, k, xq, xd))
    return mats, xs, ys, wants


SHAPES = {
    # the layer shapes and a ragged LM-head-like tail (the large launch shape)
    "llama_layer": [(3072, 2048), (2048, 2048), (16384, 2048), (2048, 8192), (20000, 2048)],
    # one row, ragged rows, a tile of fewer than 64 chunks (k = 6144), k = 16384
    "ragged": [(1, 2048), (5, 4096), (300, 6144), (257, 8192), (9, 2048), (4097, 4096), (33, 16384)],
    "single": [(64, 2048)],
}


@pytest.mark.parametrize("overlapped", [False, True], ids=["barrier", "overlapped"])
@pytest.mark.parametrize("name", sorted(SHAPES))
def test_plan_matches_oracle_and_chain(gpu, name, overlapped):
    import torch
    shapes = SHAPES[name]
    mats, xs, ys, wants = _independent(shapes, 1500)
    steps = _steps(mats, xs, ys, shapes)
    plan = Plan(gpu, steps, len(shapes), overlapped)
    plan.run(1)
    for i, (y, want) in enumerate(zip(ys, wants)):
        assert_bytes_equal(host(y), want, f"{name} step {i} {shapes[i]}")
    for passes in (3, 1):
        for y in ys:
            y.fill_(float("nan"))
        plan.run(passes)
        for i, (y, want) in enumerate(zip(ys, wants)):
            assert_bytes_equal(host(y), want, f"{name} {passes} passes, step {i}")
    plan.close()
    for y in ys:
        y.fill_(float("nan"))
    L = gpu.lib()
    gpu.check("w4a8_chain_gemv", L.w4a8_chain_gemv(ctypes.cast(steps, ctypes.c_void_p), len(shapes),
                                                   torch.cuda.current_stream().cuda_stream))
    for i, (y, want) in enumerate(zip(ys, wants)):
        assert_bytes_equal(host(y), want, f"{name} step {i}: w4a8_chain_gemv")


def _dependent_oracle(blocks, shapes, x0, passes):
    """The chain y_j = W_j q8(y_{j-1}) run `passes` times on the CPU; with
    `cyclic`, pass p + 1 starts from pass p's last output."""
    x, outs = x0, None
    for _ in range(passes):
        outs = []
        for b, (r, k) in zip(blocks, shapes):
            xq, xd = C.quantize_q8_0(x)
            x = C.gemv_q4_0(b, k, xq, xd)
            outs.append(x)
    return outs


@pytest.mark.parametrize("overlapped", [False, True], ids=["barrier", "overlapped"])
def test_plan_dependency_inside_a_pass(gpu, overlapped):
    """x of every step after the first IS the previous step's y (overlapped:
    each step's workgroups start early and must wait for that y)."""
    shapes = [(2048, 2048), (8192, 2048), (2048, 8192), (2048, 2048), (3072, 2048), (2048, 3072), (2048, 2048)]
    blocks = [C.quantize_q4_0(O.normal_f32((r, k), 60 + i, 0.02)) for i, (r, k) in enumerate(shapes)]
    x0 = O.normal_f32((1, shapes[0][1]), 59)[0]
    wants = _dependent_oracle(blocks, shapes, x0, 1)
    mats = [dev(b) for b in blocks]
    xin = dev(x0)
    ys = [poisoned_f32(r) for r, _ in shapes]
    plan = Plan(gpu, _steps(mats, [xin] + ys[:-1], ys, shapes), len(shapes), overlapped)
    for passes in (1, 4, 2):
        for y in ys:
            y.fill_(float("nan"))
        plan.run(passes)
        for i, (y, want) in enumerate(zip(ys, wants)):
            assert_bytes_equal(host(y), want, f"{passes} passes, step {i}")
    plan.close()


@pytest.mark.parametrize("overlapped", [False, True], ids=["barrier", "overlapped"])
def test_plan_dependency_across_passes(gpu, overlapped):
    """The first step reads the last step's output: each pass continues from
    the previous one, within a launch and across launches."""
    shapes = [(8192, 2048), (2048, 8192), (3072, 2048), (2048, 3072)]
    blocks = [C.quantize_q4_0(O.normal_f32((r, k), 80 + i, 0.02)) for i, (r, k) in enumerate(shapes)]
    x0 = O.normal_f32((1, 2048), 79)[0]
    mats = [dev(b) for b in blocks]
    ys = [poisoned_f32(r) for r, _ in shapes]
    ys[-1].copy_(dev(x0))                  # the first pass starts from x0
    plan = Plan(gpu, _steps(mats, [ys[-1]] + ys[:-1], ys, shapes), len(shapes), overlapped)
    plan.run(3)
    wants = _dependent_oracle(blocks, shapes, x0, 3)
    for i, (y, want) in enumerate(zip(ys, wants)):
        assert_bytes_equal(host(y), want, f"after 3 passes, step {i}")
    plan.run(2)
    x = np.asarray(wants[-1])
    wants = _dependent_oracle(blocks, shapes, x, 2)
    for i, (y, want) in enumerate(zip(ys, wants)):
        assert_bytes_equal(host(y), want, f"after 3 + 2 passes, step {i}")
    plan.close()


def test_plan_reader_paths(gpu):
    """Steps reading other steps' outputs where an earlier step of the pass
    has already brought that memory into an L2: a second reader of one
    output, and an output sharing an L2 line with an earlier step's input (one
    arena, the two 16 bytes apart across a line), besides plain readers."""
    import torch
    k = 2048
    blocks = [C.quantize_q4_0(O.normal_f32((k, k), 120 + i, 0.02)) for i in range(5)]
    mats = [dev(b) for b in blocks]
    xa = O.normal_f32((1, k), 119)[0]
    arena = torch.full((2 * k + 1024,), float("nan"), dtype=torch.float32, device="cuda")
    x_in = arena[16:16 + k]                          # bytes 64 .. 8256
    y_p = arena[16 + k + 4:16 + 2 * k + 4]           # from byte 8272: same 256-byte line as x_in's end
    x_in.copy_(dev(xa))
    y0, y2, y3, y4 = (poisoned_f32(k) for _ in range(4))
    # step: (x, y); 1 reads y0, 3 reads y0 again, 2 reads y_p (its first line
    # shared with step 0's input), 4 reads y2
    io = [(x_in, y0), (y0, y_p), (y_p, y2), (y0, y3), (y2, y4)]
    steps = (Step * 5)(*[Step(mats[i].data_ptr(), x.data_ptr(), y.data_ptr(), k, k) for i, (x, y) in enumerate(io)])
    def q(v):
        return C.quantize_q8_0(np.asarray(v, dtype=np.float32))
    w0 = C.gemv_q4_0(blocks[0], k, *q(xa))
    w1 = C.gemv_q4_0(blocks[1], k, *q(w0))
    w2 = C.gemv_q4_0(blocks[2], k, *q(w1))
    w3 = C.gemv_q4_0(blocks[3], k, *q(w0))
    w4 = C.gemv_q4_0(blocks[4], k, *q(w2))
    plan = Plan(gpu, steps, 5)
    for passes in (1, 3):
        for y in (y0, y_p, y2, y3, y4):
            y.fill_(float("nan"))
        torch.cuda.synchronize()
        plan.run(passes)
        for name, y, want in (("y0", y0, w0), ("y_p", y_p, w1), ("y2", y2, w2), ("y3", y3, w3), ("y4", y4, w4)):
            assert_bytes_equal(host(y), want, f"{passes} passes, {name}")
    plan.close()


def test_plan_steps_sharing_one_output_buffer(gpu):
    """Three steps of different shapes write one buffer, as the reference's
    caller gives every engine call the same y (board/tp/tp_llama.cpp:301):
    gate|up's 16384 rows, then q|k|v's 3072 and o's 2048 over its start; two
    readers then take k = 2048 slices of it as x (rows 0..2047, o's; rows
    2048..4095, q|k|v's and then gate|up's). Each step maps its rows to other
    workgroups (and XCDs), so the later writer's bytes must win everywhere:
    byte-exact against the C oracle over 1 and 3 passes."""
    import torch
    k = 2048
    shapes = [(16384, k), (3072, k), (k, k)]
    mats, xs, _, wants = _independent(shapes, 2100)
    shared = poisoned_f32(16384)
    rd_blocks = [C.quantize_q4_0(O.normal_f32((k, k), 2150 + i, 0.02)) for i in range(2)]
    rd_mats = [dev(b) for b in rd_blocks]
    rd_ys = [poisoned_f32(k) for _ in range(2)]
    final = np.array(wants[0], copy=True)
    final[:3072] = wants[1]
    final[:k] = wants[2]
    rd_want = [C.gemv_q4_0(rd_blocks[i], k, *C.quantize_q8_0(np.ascontiguousarray(final[i * k:(i + 1) * k])))
               for i in range(2)]
    steps = (Step * 5)(*[Step(mats[i].data_ptr(), xs[i].data_ptr(), shared.data_ptr(), r, kk)
                         for i, (r, kk) in enumerate(shapes)],
                       *[Step(rd_mats[i].data_ptr(), shared[i * k:].data_ptr(), rd_ys[i].data_ptr(), k, k)
                         for i in range(2)])
    plan = Plan(gpu, steps, 5)
    for passes in (1, 3):
        shared.fill_(float("nan"))
        for y in rd_ys:
            y.fill_(float("nan"))
        torch.cuda.synchronize()
        plan.run(passes)
        assert_bytes_equal(host(shared), final, f"{passes} passes: the shared buffer")
        for i in range(2):
            assert_bytes_equal(host(rd_ys[i]), rd_want[i], f"{passes} passes: reader {i}")
    plan.close()


def test_plan_several_launches_one_wait(gpu):
    """Launches queue up; one wait covers them all; two plans share the queue."""
    shapes_a = [(2048, 2048), (16384, 2048)]
    shapes_b = [(2048, 8192), (3072, 2048)]
    ma, xa, ya, wa = _independent(shapes_a, 1700)
    mb, xb, yb, wb = _independent(shapes_b, 1800)
    pa = Plan(gpu, _steps(ma, xa, ya, shapes_a), 2)
    pb = Plan(gpu, _steps(mb, xb, yb, shapes_b), 2)
    L = gpu.lib()
    for _ in range(3):
        gpu.check("launch a", L.w4a8_chain_plan_launch(pa.p, 2))
        gpu.check("launch b", L.w4a8_chain_plan_launch(pb.p, 1))
    gpu.check("wait b", L.w4a8_chain_plan_wait(pb.p, 30000))
    gpu.check("wait a", L.w4a8_chain_plan_wait(pa.p, 30000))
    for y, want in zip(ya + yb, wa + wb):
        assert_bytes_equal(host(y), want, "queued launches")
    pa.close()
    pb.close()


def test_overlapped_plan_timed_launch_and_checks(gpu):
    """An overlapped plan's timed launch (barrier bits, no overlap) gives the
    same outputs and leaves the flags consistent: a plain launch after it is
    still byte-exact. Only plain GEMV steps are accepted."""
    import torch
    shapes = SHAPES["llama_layer"]
    mats, xs, ys, wants = _independent(shapes, 1550)
    plan = Plan(gpu, _steps(mats, xs, ys, shapes), len(shapes), overlapped=True)
    L = gpu.lib()
    stamps = torch.zeros(2 * 2 * L.w4a8_chain_plan_workgroups(plan.p, -1), dtype=torch.int64, device="cuda")
    for y in ys:
        y.fill_(float("nan"))
    torch.cuda.synchronize()
    gpu.check("launch_timed", L.w4a8_chain_plan_launch_timed(plan.p, 2, stamps.data_ptr()))
    gpu.check("wait", L.w4a8_chain_plan_wait(plan.p, 30000))
    for i, (y, want) in enumerate(zip(ys, wants)):
        assert_bytes_equal(host(y), want, f"timed, step {i}")
    for y in ys:
        y.fill_(float("nan"))
    torch.cuda.synchronize()
    plan.run(3)
    for i, (y, want) in enumerate(zip(ys, wants)):
        assert_bytes_equal(host(y), want, f"after the timed launch, step {i}")
    plan.close()
    p = ctypes.c_void_p()
    bad = _steps(mats, xs, ys, [(64, 1024)])
    assert L.w4a8_chain_plan_create_overlapped(ctypes.cast(bad, ctypes.c_void_p), 1, ctypes.byref(p)) == -2


def test_plan_argument_checks(gpu):
    L = gpu.lib()
    shapes = [(64, 2048)]
    mats, xs, ys, _ = _independent(shapes, 1900)
    steps = _steps(mats, xs, ys, shapes)
    p = ctypes.c_void_p()
    assert L.w4a8_chain_plan_create(ctypes.cast(steps, ctypes.c_void_p), 0, ctypes.byref(p)) == -2
    bad = _steps(mats, xs, ys, [(64, 1024)])         # k < 2048
    assert L.w4a8_chain_plan_create(ctypes.cast(bad, ctypes.c_void_p), 1, ctypes.byref(p)) == -2
    plan = Plan(gpu, steps, 1)
    assert L.w4a8_chain_plan_launch(plan.p, 0) == -2
    assert L.w4a8_chain_plan_wait(plan.p, 0) == 0       # nothing launched: done at once
    plan.close()


# ------------------------------------------------------------- producers


def _blocks(rows, k, seed):
    return dev(C.quantize_q4_0(O.normal_f32((rows, k), seed, 0.02)))


def _run_steps(gpu, steps, passes):
    import torch
    L = gpu.lib()
    arr = (gpu.PlanStep * len(steps))(*steps)
    torch.cuda.synchronize()
    p = ctypes.c_void_p()
    gpu.check("w4a8_chain_plan_create_steps", L.w4a8_chain_plan_create_steps(ctypes.cast(arr, ctypes.c_void_p),
                                                                             len(steps), ctypes.byref(p)))
    gpu.check("launch", L.w4a8_chain_plan_launch(p, passes))
    gpu.check("wait", L.w4a8_chain_plan_wait(p, 30000))
    gpu.check("destroy", L.w4a8_chain_plan_destroy(p))


def test_plan_producer_steps_match_the_stream_entry_points(gpu):
    """A decode step with its producers: q|k|v and gate|up read rmsnorm(x),
    down reads gate|up's silu * up output, the LM head picks its row; the same
    steps without the rmsnorm. Every output and the picked row against the
    stream entry points, over two passes."""
    import torch
    k, n_ff, vocab = 2048, 8192, 20000
    g = torch.Generator(device="cuda")
    g.manual_seed(7)
    resid = torch.randn(k, generator=g, device="cuda")
    attn = torch.randn(k, generator=g, device="cuda")
    norm = torch.randn(k, generator=g, device="cuda")
    W = {"qkv": _blocks(3072, k, 11), "o": _blocks(k, k, 12), "gu": _blocks(2 * n_ff, k, 13),
         "down": _blocks(k, n_ff, 14), "lm": _blocks(vocab, k, 15)}
    for with_norm in (True, False):
        nw = norm if with_norm else None
        # the stream entry points
        want_qkv = (gpu.gemv_rmsnorm(W["qkv"], k, resid, norm, 1e-5) if with_norm
                    else gpu.gemv_q4_0_f32(W["qkv"], k, resid))
        want_o = gpu.gemv_q4_0_f32(W["o"], k, attn)
        want_act = gpu.gemv_gate_up_silu(W["gu"], k, resid, nw, 1e-5)
        want_down = gpu.gemv_q4_0_f32(W["down"], n_ff, want_act)
        ws0 = gpu.argmax_workspace()
        want_lm, want_pick = (gpu.gemv_rmsnorm_argmax(W["lm"], k, resid, norm, 1e-5, ws0) if with_norm
                              else gpu.gemv_q4_0_f32_argmax(W["lm"], k, resid, ws0))
        torch.cuda.synchronize()
        # the plan
        ys = {"qkv": poisoned_f32(3072), "o": poisoned_f32(k), "act": poisoned_f32(n_ff), "down": poisoned_f32(k),
              "lm": poisoned_f32(vocab)}
        pick = torch.full((1,), -1, dtype=torch.int32, device="cuda")
        ws = gpu.argmax_workspace()
        nptr = norm.data_ptr() if with_norm else None
        S = gpu.PlanStep
        steps = [S(gpu.PLAN_GEMV, W["qkv"].data_ptr(), resid.data_ptr(), ys["qkv"].data_ptr(), 3072, k, nptr, 1e-5),
                 S(gpu.PLAN_GEMV, W["o"].data_ptr(), attn.data_ptr(), ys["o"].data_ptr(), k, k, None, 0.0),
                 S(gpu.PLAN_GATE_UP_SILU, W["gu"].data_ptr(), resid.data_ptr(), ys["act"].data_ptr(), 2 * n_ff, k,
                   nptr, 1e-5),
                 S(gpu.PLAN_GEMV, W["down"].data_ptr(), ys["act"].data_ptr(), ys["down"].data_ptr(), k, n_ff,
                   None, 0.0),
                 S(gpu.PLAN_ARGMAX, W["lm"].data_ptr(), resid.data_ptr(), ys["lm"].data_ptr(), vocab, k, nptr, 1e-5,
                   pick.data_ptr(), ws.data_ptr())]
        _run_steps(gpu, steps, 2)
        tag = "rmsnorm" if with_norm else "plain"
        for name, want in (("qkv", want_qkv), ("o", want_o), ("act", want_act), ("down", want_down),
                           ("lm", want_lm)):
            assert_bytes_equal(host(ys[name]), host(want), f"{tag}: {name}")
        assert int(pick.item()) == int(want_pick.item()), f"{tag}: picked row"
        assert not ws.any().item(), "the argmax step leaves its workspace zero"


def test_plan_quantized_act_into_down(gpu):
    """gate|up quantizing its act in the epilogue (W4A8_PLAN_GATE_UP_SILU_Q8)
    and down on that engine-layout act (W4A8_PLAN_GEMV_ENGINE), in one pass
    and over three: both outputs against the stream entry points and the
    oracle."""
    import torch
    k, n_ff = 2048, 8192
    g = torch.Generator(device="cuda")
    g.manual_seed(9)
    resid = torch.randn(k, generator=g, device="cuda")
    norm = torch.randn(k, generator=g, device="cuda")
    gu, down = _blocks(2 * n_ff, k, 31), _blocks(k, n_ff, 32)
    for nw in (norm, None):
        want_act = gpu.gemv_gate_up_silu(gu, k, resid, nw, 1e-5, q8=True)
        want_down = gpu.gemv_engine(down, n_ff, want_act)
        want_down_f32 = gpu.gemv_q4_0_f32(down, n_ff, gpu.gemv_gate_up_silu(gu, k, resid, nw, 1e-5))
        torch.cuda.synchronize()
        assert_bytes_equal(host(want_down), host(want_down_f32), "down on the quantized act = down on the fp32 act")
        act = torch.full((gpu.engine_x_bytes(n_ff),), 0xAA, dtype=torch.uint8, device="cuda")
        y = poisoned_f32(k)
        S = gpu.PlanStep
        steps = [S(gpu.PLAN_GATE_UP_SILU_Q8, gu.data_ptr(), resid.data_ptr(), act.data_ptr(), 2 * n_ff, k,
                   None if nw is None else nw.data_ptr(), 1e-5),
                 S(gpu.PLAN_GEMV_ENGINE, down.data_ptr(), act.data_ptr(), y.data_ptr(), k, n_ff, None, 0.0)]
        for passes in (1, 3):
            act.fill_(0xAA)
            y.fill_(float("nan"))
            _run_steps(gpu, steps, passes)
            tag = f"{'rmsnorm' if nw is not None else 'plain'}, {passes} passes"
            assert torch.equal(act, want_act), f"{tag}: act"
            assert_bytes_equal(host(y), host(want_down), f"{tag}: down")


def test_plan_steps_argument_checks(gpu):
    import torch
    L = gpu.lib()
    S = gpu.PlanStep
    w = _blocks(64, 2048, 21)
    x = torch.zeros(2048, device="cuda")
    y = torch.zeros(64, device="cuda")
    p = ctypes.c_void_p()

    def create(step):
        arr = (S * 1)(step)
        return L.w4a8_chain_plan_create_steps(ctypes.cast(arr, ctypes.c_void_p), 1, ctypes.byref(p))
    assert create(S(7, w.data_ptr(), x.data_ptr(), y.data_ptr(), 64, 2048, None, 0.0)) == -2       # kind
    assert create(S(gpu.PLAN_ARGMAX, w.data_ptr(), x.data_ptr(), y.data_ptr(), 64, 2048, None, 0.0)) == -1
    assert create(S(gpu.PLAN_GATE_UP_SILU, w.data_ptr(), x.data_ptr(), y.data_ptr(), 6, 2048, None, 0.0)) == -2
    assert create(S(gpu.PLAN_GATE_UP_SILU_Q8, w.data_ptr(), x.data_ptr(), y.data_ptr(), 16, 2048, None, 0.0)) == -2
    assert create(S(gpu.PLAN_GEMV_ENGINE, w.data_ptr(), x.data_ptr(), y.data_ptr(), 64, 2048, x.data_ptr(),
                    1e-5)) == -2                                                                  # no rmsnorm on engine x
    assert create(S(5, w.data_ptr(), x.data_ptr(), y.data_ptr(), 64, 2048, None, 0.0)) == -2        # kind
    w16 = _blocks(64, 16384, 22)
    x16 = torch.zeros(16384, device="cuda")
    assert create(S(gpu.PLAN_GEMV, w16.data_ptr(), x16.data_ptr(), y.data_ptr(), 64, 16384, x16.data_ptr(),
                    1e-5)) == -2                                                                  # rmsnorm k > 8192
