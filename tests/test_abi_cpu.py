"""The C-ABI library without a GPU: it loads, exports every symbol the headers
declare, checks arguments before touching the device, and the host-only parts
of the board ABI (bump allocator, v2 layout formula) behave as the
reference's do (board/kv260gemv/udmabuf.c:47-52, gemv2_dev.h:66-72)."""

from __future__ import annotations

import ctypes
import os
import re
import subprocess
import sys

import numpy as np
import pytest

import kv260gemv

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INCLUDE = os.path.join(ROOT, "include")


def _declared_functions() -> set[str]:
    names = set()
    for h in os.listdir(INCLUDE):
        if not h.endswith(".h"):
            continue
        with open(os.path.join(INCLUDE, h)) as f:
            text = f.read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        text = re.sub(r"//[^\n]*", "", text)
        for m in re.finditer(r"^\s*(?!static|typedef|#)[A-Za-z_][\w\s\*]*?\b([a-z_][a-z0-9_]*)\s*\(", text, flags=re.M):
            names.add(m.group(1))
    return names


def test_library_loads_and_reports_contract():
    L = kv260gemv.lib()
    assert L.w4a8_contract_version().decode() == "llm-kv260/w4a8-q4_0-v2"
    assert kv260gemv.strerror(-2).startswith("shape")


def test_every_declared_symbol_is_exported():
    declared = _declared_functions()
    assert {"w4a8_gemv", "gemv_dev_start4", "gemv2_mac_start", "udmabuf_clean", "w4a8_chain_gemv"} <= declared
    L = kv260gemv.lib()
    missing = [n for n in sorted(declared) if not hasattr(L, n)]
    assert not missing, missing
    assert declared == set(kv260gemv.EXPORTS), declared ^ set(kv260gemv.EXPORTS)
    out = subprocess.run(["nm", "-D", "--defined-only", kv260gemv.LIB_PATH], capture_output=True, text=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    assert declared <= exported


def test_topk_no_alloc_checks_come_before_the_device():
    """The no-allocation top-k refuses sizes beyond its array, and bad pointers,
    without any HIP call (no GPU here)."""
    L = kv260gemv.lib()
    fake = 0x10000
    assert L.w4a8_topk_no_alloc(fake, 262145, 40, fake, fake, None) == -2
    assert L.w4a8_topk_no_alloc(fake, 0, 40, fake, fake, None) == -2
    assert L.w4a8_topk_no_alloc(fake, 1000, 0, fake, fake, None) == -2
    assert L.w4a8_topk_no_alloc(fake, 1000, 65, fake, fake, None) == -2
    assert L.w4a8_topk_no_alloc(None, 1000, 40, fake, fake, None) == -1
    assert L.w4a8_topk_no_alloc(fake + 2, 1000, 40, fake, fake, None) == -3


def test_size_helpers():
    L = kv260gemv.lib()
    assert L.w4a8_q4_0_row_bytes(2048) == 1152
    assert L.w4a8_engine_x_bytes(2048) == 2304
    assert L.w4a8_engine_x_bytes(8192) == 9216
    assert L.w4a8_q8_0_row_bytes(2048) == 2176


def test_argument_checks_come_before_the_device():
    """Invalid calls return their status without any HIP call (no GPU here)."""
    L = kv260gemv.lib()
    fake = 0x10000    # never dereferenced: every call below fails its checks first
    assert L.w4a8_gemv(None, fake, fake, 16, 2048, None) == -1
    assert L.w4a8_gemv(fake, fake, fake, 16, 2000, None) == -2          # k % 256
    assert L.w4a8_gemv(fake, fake, fake, 16, 128, None) == -2           # k < 256
    assert L.w4a8_gemv(fake, fake, fake, 16, 32768, None) == -2         # k > max
    assert L.w4a8_gemv(fake, fake, fake, 0, 2048, None) == -2
    assert L.w4a8_gemv(fake + 8, fake, fake, 16, 2048, None) == -3
    assert L.w4a8_gemv(fake, fake + 4, fake, 16, 2048, None) == -3
    assert L.w4a8_gemv(fake, fake, fake + 2, 16, 2048, None) == -3
    assert L.w4a8_gemv_q8_0(fake, fake + 1, fake, 16, 2048, None) == -3
    assert L.w4a8_gemm(fake, fake, fake, 0, 16, 2048, None) == -2
    assert L.w4a8_quantize_q8_0(fake, fake, 100, 1, None) == -2
    assert L.w4a8_quantize_q4_0(fake, fake, 1, 33, None) == -2
    assert L.w4a8_chain_gemv(None, 1, None) == -1
    quarters = (ctypes.c_void_p * 4)(fake, fake, None, fake)
    assert L.w4a8_gemv_quarters(quarters, fake, fake, 16, 2048, None) == -1
    plan = ctypes.c_void_p()
    assert L.w4a8_chain_plan_create(None, 1, ctypes.byref(plan)) == -1
    steps = (ctypes.c_void_p * 3)(fake, fake, fake)
    raw = (ctypes.c_int * 2)(16, 1024)                 # one step, k = 1024 < 2048
    buf = ctypes.create_string_buffer(bytes(steps) + bytes(raw))
    assert L.w4a8_chain_plan_create(buf, 1, ctypes.byref(plan)) == -2
    assert L.w4a8_chain_plan_create(buf, 0, ctypes.byref(plan)) == -2
    assert L.w4a8_chain_plan_create(buf, 1, None) == -1
    assert L.w4a8_chain_plan_launch(None, 1) == -1
    assert L.w4a8_chain_plan_wait(None, 0) == -1
    assert L.w4a8_chain_plan_destroy(None) == 0
    assert kv260gemv.strerror(-7).startswith("a bounded wait")
    # gate|up quantizing its act: k = 2048 only, whole Q8_0 blocks per workgroup, act 16-byte aligned
    assert L.w4a8_gemv_gate_up_silu_q8_0(fake, fake, None, 1e-5, fake, 64, 4096, None) == -2
    assert L.w4a8_gemv_gate_up_silu_q8_0(fake, fake, None, 1e-5, fake, 16, 2048, None) == -2
    assert L.w4a8_gemv_gate_up_silu_q8_0(fake, fake, None, 1e-5, fake + 4, 64, 2048, None) == -3
    assert L.w4a8_gemv_gate_up_silu_q8_0(fake, fake, None, 1e-5, None, 64, 2048, None) == -1
    # plan steps: an engine-layout x takes no rmsnorm; kinds past the last are refused
    S = kv260gemv.PlanStep
    one = (S * 1)(S(kv260gemv.PLAN_GEMV_ENGINE, fake, fake, fake, 64, 2048, fake, 1e-5))
    assert L.w4a8_chain_plan_create_steps(ctypes.cast(one, ctypes.c_void_p), 1, ctypes.byref(plan)) == -2
    one = (S * 1)(S(5, fake, fake, fake, 64, 2048, None, 0.0))
    assert L.w4a8_chain_plan_create_steps(ctypes.cast(one, ctypes.c_void_p), 1, ctypes.byref(plan)) == -2
    one = (S * 1)(S(kv260gemv.PLAN_GATE_UP_SILU_Q8, fake, fake, fake, 64, 4096, None, 0.0))
    assert L.w4a8_chain_plan_create_steps(ctypes.cast(one, ctypes.c_void_p), 1, ctypes.byref(plan)) == -2
    assert L.w4a8_chain_plan_launch_timed(None, 1, fake) == -1
    assert L.w4a8_chain_plan_workgroups(None, 0) == -1
    assert L.w4a8_wall_clock_hz(None) == -1


def test_plan_and_chain_range_checks_come_before_the_device():
    """What a plan step may not write over, refused (-2) before any HIP call:
    its own x; any step's weights, norm_w, argmax row or workspace. The same
    steps with the ranges apart pass the checks and only then fail for want
    of a device (-5). The stream chain refuses a step in place, and the batch
    any output over an input or another output."""
    L = kv260gemv.lib()
    S = kv260gemv.PlanStep
    k, rows = 2048, 64
    wb = rows * k // 32 * 18
    W, X, Y, N, A, WS, Y2 = (0x100000 * (i + 1) for i in range(7))
    plan = ctypes.c_void_p()

    def create(*steps):
        arr = (S * len(steps))(*steps)
        return L.w4a8_chain_plan_create_steps(ctypes.cast(arr, ctypes.c_void_p), len(steps), ctypes.byref(plan))

    gemv = lambda w, x, y, norm=None: S(kv260gemv.PLAN_GEMV, w, x, y, rows, k, norm, 1e-5)
    lm = lambda y, a, ws: S(kv260gemv.PLAN_ARGMAX, W, X, y, rows, k, None, 0.0, a, ws)
    assert create(gemv(W, X, Y), gemv(W, Y, Y2)) == -5            # y feeds x: allowed
    assert create(gemv(W, X, Y), gemv(W, X, Y + 64)) == -5        # outputs sharing bytes: allowed
    assert create(gemv(W, X, X + 16)) == -2                       # x over its own y
    assert create(gemv(W, X, Y), gemv(Y - wb + 16, X, Y2)) == -2  # weights over another step's y
    assert create(gemv(W, X, W + 64)) == -2                       # weights over its own y
    assert create(gemv(W, X, Y), gemv(W, X, Y2, Y + 128)) == -2   # norm_w over a y
    assert create(gemv(W, X, Y, N), gemv(W, X, Y2, N)) == -5
    assert create(gemv(W, X, Y), lm(Y2, Y + 8, WS)) == -2         # argmax row in a y
    assert create(gemv(W, X, Y), lm(Y2, A, Y + 16)) == -2         # workspace over a y
    assert create(gemv(W, X, Y), lm(Y2, A, WS)) == -5

    class Step(ctypes.Structure):   # include/w4a8.h's w4a8_chain_step
        _fields_ = [("w", ctypes.c_void_p), ("x", ctypes.c_void_p), ("y", ctypes.c_void_p),
                    ("rows", ctypes.c_int), ("k", ctypes.c_int)]

    in_place = (Step * 2)(Step(W, X, Y, rows, k), Step(W, Y, Y + 8, rows, k))
    assert L.w4a8_chain_gemv(ctypes.cast(in_place, ctypes.c_void_p), 2, None) == -2
    batch = (Step * 2)(Step(W, X, Y, rows, k), Step(W, Y2, Y + 128, rows, k))
    assert L.w4a8_gemv_batch(ctypes.cast(batch, ctypes.c_void_p), 2, None) == -2       # outputs overlap
    batch = (Step * 2)(Step(W, X, Y, rows, k), Step(W, Y, Y2, rows, k))
    assert L.w4a8_gemv_batch(ctypes.cast(batch, ctypes.c_void_p), 2, None) == -2       # y is another's x


class Udmabuf(ctypes.Structure):
    _fields_ = [("fd", ctypes.c_int), ("base", ctypes.c_void_p), ("phys", ctypes.c_uint64),
                ("size", ctypes.c_size_t), ("used", ctypes.c_size_t)]


def test_udmabuf_bump_allocator_host_logic():
    L = kv260gemv.lib()
    L.udmabuf_alloc.restype = ctypes.c_void_p
    L.udmabuf_alloc.argtypes = [ctypes.POINTER(Udmabuf), ctypes.c_size_t, ctypes.c_size_t]
    backing = (ctypes.c_uint8 * (1 << 20))()
    base = ctypes.addressof(backing)
    b = Udmabuf(fd=0, base=base, phys=0x7000_0000, size=1 << 20, used=0)
    p1 = L.udmabuf_alloc(ctypes.byref(b), 100, 64)
    p2 = L.udmabuf_alloc(ctypes.byref(b), 10, 4096)
    p3 = L.udmabuf_alloc(ctypes.byref(b), 1 << 20, 16)      # does not fit
    assert p1 == base and p2 == base + 4096 and p3 is None
    assert b.used == 4096 + 10


def _compile_layout_probe(tmp_path) -> str:
    src = tmp_path / "probe.c"
    src.write_text(
        '#include <stdio.h>\n#include "gemv2_dev.h"\n'
        "int main(int c, char **v) { int rows, k; sscanf(v[1], \"%d\", &rows); sscanf(v[2], \"%d\", &k);\n"
        " for (int r = 0; r < rows; ++r) for (int ch = 0; ch < k / 256; ++ch) { int p;\n"
        "   size_t o = gemv2_chunk_offset(r, ch, rows, k, &p); printf(\"%d %zu\\n\", p, o); } return 0; }\n")
    exe = tmp_path / "probe"
    subprocess.run(["gcc", "-std=c11", "-Wall", "-I", INCLUDE, "-o", str(exe), str(src)], check=True)
    return str(exe)


@pytest.mark.parametrize("rows,k", [(32, 256), (64, 2048), (96, 512)])
def test_gemv2_chunk_layout_is_a_permutation(tmp_path, rows, k):
    """Each port region holds exactly rows/4 rows of chunks, each 144-byte slot once,
    and the pairing puts row i and i + rows/8 of a port side by side
    (board/kv260gemv/gemv2_dev.h:46-49)."""
    exe = _compile_layout_probe(tmp_path)
    out = subprocess.run([exe, str(rows), str(k)], capture_output=True, text=True, check=True).stdout.split()
    port = np.array(out[0::2], dtype=int).reshape(rows, k // 256)
    off = np.array(out[1::2], dtype=np.int64).reshape(rows, k // 256)
    nch, per_port = k // 256, rows // 4
    for p in range(4):
        slots = np.sort(off[port == p])
        assert np.array_equal(slots, np.arange(per_port * nch) * 144)
    r = per_port // 2                    # row 0 and row rows/8 share chunk pairs
    assert off[r, 0] == off[0, 0] + 144 and port[r, 0] == port[0, 0]
    if nch > 1:
        assert off[0, 1] == off[0, 0] + 288


def test_shim_open_without_gpu_fails_cleanly():
    """No device: the engine open calls return -1 (quietly for gemv2), as the
    reference's do when no overlay is loaded (tp_llama.cpp:303-312 then falls back)."""
    code = (
        "import ctypes, sys; sys.path.insert(0, %r); import kv260gemv as k; L = k.lib()\n"
        "class D(ctypes.Structure): _fields_ = [('fd', ctypes.c_int), ('regs', ctypes.c_void_p)]\n"
        "class D2(ctypes.Structure): _fields_ = [('fetch', D), ('mac', D)]\n"
        "d = D(); d2 = D2()\n"
        "print(L.gemv_dev_open(ctypes.byref(d)), L.gemv2_dev_open(ctypes.byref(d2)))\n"
    ) % os.path.join(ROOT, "llm-kv260_amd")
    env = dict(os.environ, HIP_VISIBLE_DEVICES="-1", ROCR_VISIBLE_DEVICES="-1")
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, env=env, timeout=120)
    assert r.stdout.split() == ["-1", "-1"], (r.stdout, r.stderr)


# ------------------------------------------------- output tensors (Python)

def test_out_tensor_checks_before_any_launch():
    """The wrappers' check of a caller's out= tensor (kv260gemv._out): type,
    dtype, contiguity and size are refused before anything is launched, and a
    tensor off the weights' device too (here: any CPU tensor)."""
    import torch
    like = torch.empty(4, dtype=torch.uint8)
    with pytest.raises(TypeError, match="torch tensor"):
        kv260gemv._out(np.zeros(8, np.float32), (8,), torch.float32, like)
    with pytest.raises(TypeError, match="float32"):
        kv260gemv._out(torch.empty(8, dtype=torch.float16), (8,), torch.float32, like)
    with pytest.raises(ValueError, match="contiguous"):
        kv260gemv._out(torch.empty(16, dtype=torch.float32)[::2], (8,), torch.float32, like)
    with pytest.raises(ValueError, match="holds 7 elements, the call writes 8"):
        kv260gemv._out(torch.empty(7, dtype=torch.float32), (8,), torch.float32, like)
    with pytest.raises(ValueError, match="holds 11 elements, the call writes 12"):
        kv260gemv._out(torch.empty((3, 4), dtype=torch.float32)[:, :4].reshape(-1)[:11], (3, 4), torch.float32, like)
    with pytest.raises(ValueError, match="must be on"):
        kv260gemv._out(torch.empty(8, dtype=torch.float32), (8,), torch.float32, like)


def test_wrappers_refuse_host_tensors():
    """Every wrapper refuses CPU tensors with a TypeError / ValueError before it
    calls the library (no GPU here: a call would fail with a HIP error)."""
    import torch
    k = 256
    blocks = torch.zeros((16, k // 32 * 18), dtype=torch.uint8)
    x = torch.zeros(k, dtype=torch.float32)
    calls = [
        lambda: kv260gemv.gemv_q4_0_f32(blocks, k, x),
        lambda: kv260gemv.gemv_engine(blocks, k, torch.zeros(k + k // 8, dtype=torch.uint8)),
        lambda: kv260gemv.gemv_rmsnorm(blocks, k, x, x, 1e-5),
        lambda: kv260gemv.gemv_silu_mul(blocks, k, torch.zeros(2 * k)),
        lambda: kv260gemv.gemv_q8_0_blocks(blocks, k, torch.zeros(k // 32 * 34, dtype=torch.uint8)),
        lambda: kv260gemv.gemm_engine(blocks, k, torch.zeros((2, k + k // 8), dtype=torch.uint8)),
        lambda: kv260gemv.quantize_q8_0_engine(x),
        lambda: kv260gemv.rmsnorm_q8_0_engine(x, x, 1e-5),
        lambda: kv260gemv.silu_mul_q8_0_engine(torch.zeros(2 * k)),
        lambda: kv260gemv.gemv_quarters([blocks] * 4, k, torch.zeros(k + k // 8, dtype=torch.uint8), 64),
        lambda: kv260gemv.topk(x, 4),
    ]
    for c in calls:
        with pytest.raises((TypeError, ValueError)):
            c()
