"""The reference driver's ABI on the GPU, called exactly as board/tp and
bench_gemv2.c call it: udmabuf pools with clean / invalidate around each call,
the v1 engine's four quarters (gemv_dev_start4) and the v2 engine's
fetch + MAC pair on the chunk-interleaved port layout (gemv2_dev.h), each
compared byte for byte with the oracle. Outputs are poisoned with 0xAA in the
pool first (board/kv260gemv/bench_gemv2.c:63)."""

from __future__ import annotations

import ctypes
import hashlib
import json
import os
import sys

import numpy as np
import pytest

import c_oracle as C
import q4_0_oracle as O
from gpu_helpers import assert_bytes_equal

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))

import make_gen_vectors as GV  # noqa: E402

pytestmark = pytest.mark.gpu


class Udmabuf(ctypes.Structure):
    _fields_ = [("fd", ctypes.c_int), ("base", ctypes.c_void_p), ("phys", ctypes.c_uint64),
                ("size", ctypes.c_size_t), ("used", ctypes.c_size_t)]


class Dev(ctypes.Structure):
    _fields_ = [("fd", ctypes.c_int), ("regs", ctypes.c_void_p)]


class Dev2(ctypes.Structure):
    _fields_ = [("fetch", Dev), ("mac", Dev)]


u64, i32, vp = ctypes.c_uint64, ctypes.c_int, ctypes.c_void_p


@pytest.fixture(scope="module")
def board(gpu):
    before = os.environ.get("KV260GEMV_UDMABUF_SIZES")
    os.environ["KV260GEMV_UDMABUF_SIZES"] = "udmabuf0=96M"
    L = gpu.lib()
    L.udmabuf_open.argtypes = [ctypes.POINTER(Udmabuf), ctypes.c_char_p]
    L.udmabuf_alloc.argtypes = [ctypes.POINTER(Udmabuf), ctypes.c_size_t, ctypes.c_size_t]
    L.udmabuf_alloc.restype = vp
    L.udmabuf_clean.argtypes = [vp, ctypes.c_size_t]
    L.udmabuf_invalidate.argtypes = [vp, ctypes.c_size_t]
    L.udmabuf_close.argtypes = [ctypes.POINTER(Udmabuf)]
    L.gemv_dev_open.argtypes = [ctypes.POINTER(Dev)]
    L.gemv_dev_close.argtypes = [ctypes.POINTER(Dev)]
    L.gemv_dev_run.argtypes = [ctypes.POINTER(Dev), u64, u64, u64, i32, i32]
    L.gemv_dev_start4.argtypes = [ctypes.POINTER(Dev), ctypes.POINTER(u64), u64, u64, i32, i32]
    L.gemv_dev_wait.argtypes = [ctypes.POINTER(Dev)]
    for f in ("gemv2_dev_open", "gemv2_dev_close", "gemv2_fetch_wait", "gemv2_mac_wait", "gemv2_mac_idle",
              "gemv2_drain"):
        getattr(L, f).argtypes = [ctypes.POINTER(Dev2)]
    L.gemv2_fetch_start.argtypes = [ctypes.POINTER(Dev2), ctypes.POINTER(u64), i32, i32]
    L.gemv2_mac_start.argtypes = [ctypes.POINTER(Dev2), u64, u64, i32, i32]
    pool = Udmabuf()
    assert L.udmabuf_open(ctypes.byref(pool), b"udmabuf0") == 0
    yield L, pool
    L.udmabuf_close(ctypes.byref(pool))
    if before is None:
        os.environ.pop("KV260GEMV_UDMABUF_SIZES", None)
    else:
        os.environ["KV260GEMV_UDMABUF_SIZES"] = before


def _alloc(L, pool, data_or_size, align=4096):
    n = data_or_size if isinstance(data_or_size, int) else len(data_or_size)
    p = L.udmabuf_alloc(ctypes.byref(pool), n, align)
    assert p, "pool full"
    if not isinstance(data_or_size, int):
        ctypes.memmove(p, np.ascontiguousarray(data_or_size).ctypes.data, n)
    L.udmabuf_clean(p, n)
    return p, pool.phys + (p - pool.base)


def _poisoned_y(L, pool, rows):
    return _alloc(L, pool, np.full(4 * rows, 0xAA, np.uint8))


def _read_y(L, p, rows):
    L.udmabuf_invalidate(p, 4 * rows)
    return np.ctypeslib.as_array((ctypes.c_float * rows).from_address(p)).copy()


def _case(rows, k, seed):
    w = O.normal_f32((rows, k), seed, 0.02)
    x = O.normal_f32((1, k), seed + 1)[0]
    blocks = C.quantize_q4_0(w)
    xq, xd = C.quantize_q8_0(x)
    return blocks, C.pack_x_for_engine(xq, xd), C.gemv_q4_0(blocks, k, xq, xd)


@pytest.mark.parametrize("rows,k", [(512, 2048), (64, 8192), (2048, 2048),
                                    # rows per tile that do not divide a quarter (k = 768: 21 rows per
                                    # tile; k = 1280: 12; k = 6144: 2), quarters shorter than a tile
                                    (48, 768), (208, 1280), (1040, 6144), (16, 256)])
def test_v1_quarters_and_run(board, rows, k):
    """gemv_dev_start4 over quarters at staggered pool addresses (tp_llama.cpp:105-119),
    then gemv_dev_run over the same rows contiguous."""
    L, pool = board
    blocks, x_eng, want = _case(rows, k, 300 + rows)
    q = rows // 4
    d = Dev()
    assert L.gemv_dev_open(ctypes.byref(d)) == 0
    phys = []
    for i in range(4):
        L.udmabuf_alloc(ctypes.byref(pool), (16 << 10) * (i % 2), 16)    # ports 1 and 3 at +16 KB
        phys.append(_alloc(L, pool, blocks[i * q:(i + 1) * q].reshape(-1), 64 << 10)[1])
    _, xp = _alloc(L, pool, x_eng)
    yp_host, yp = _poisoned_y(L, pool, rows)
    L.gemv_dev_start4(ctypes.byref(d), (u64 * 4)(*phys), xp, yp, k, rows)
    L.gemv_dev_wait(ctypes.byref(d))
    assert_bytes_equal(_read_y(L, yp_host, rows), want, "gemv_dev_start4")

    _, wp = _alloc(L, pool, blocks.reshape(-1), 64 << 10)
    y2_host, y2 = _poisoned_y(L, pool, rows)
    L.gemv_dev_run(ctypes.byref(d), wp, xp, y2, k, rows)
    assert_bytes_equal(_read_y(L, y2_host, rows), want, "gemv_dev_run")
    L.gemv_dev_close(ctypes.byref(d))
    pool.used = 0


def _chunk_offset(r, c, rows, k):
    """The v2 layout formula of gemv2_dev.h (port-relative byte offset, port)."""
    per_port = rows // 4
    half = per_port // 2
    chunks = k // 256
    local = r % per_port
    pair, second = local % half, local // half
    return ((pair * chunks + c) * 2 + second) * 144, r // per_port


@pytest.mark.parametrize("rows,k", [(768, 2048), (32, 256), (2048, 8192), (4096, 2048),
                                    # odd chunks per row: tiles of 10 (k = 768), 6 (k = 1280) and 1
                                    # (k = 6144) row pairs, port regions that end inside a tile
                                    (96, 768), (160, 1280), (544, 6144), (352, 3840)])
def test_v2_fetch_then_mac(board, rows, k):
    """gemv2_fetch_start + gemv2_mac_start + gemv2_mac_wait on the chunk-interleaved
    layout, as engine_t::gemv issues them (tp_llama.cpp:364-368)."""
    L, pool = board
    blocks, x_eng, want = _case(rows, k, 400 + rows)
    chunks = k // 256
    raw = blocks.reshape(rows, chunks, 144)
    regions = [np.zeros(rows // 4 * chunks * 144, np.uint8) for _ in range(4)]
    for r in range(rows):
        for c in range(chunks):
            off, port = _chunk_offset(r, c, rows, k)
            regions[port][off:off + 144] = raw[r, c]
    d2 = Dev2()
    assert L.gemv2_dev_open(ctypes.byref(d2)) == 0
    assert L.gemv2_mac_idle(ctypes.byref(d2)) == 1
    L.gemv2_drain(ctypes.byref(d2))
    phys = [_alloc(L, pool, reg, 64 << 10)[1] for reg in regions]
    _, xp = _alloc(L, pool, x_eng)
    y_host, yp = _poisoned_y(L, pool, rows)
    L.gemv2_fetch_start(ctypes.byref(d2), (u64 * 4)(*phys), k, rows)
    L.gemv2_fetch_wait(ctypes.byref(d2))
    L.gemv2_mac_start(ctypes.byref(d2), xp, yp, k, rows)
    L.gemv2_mac_wait(ctypes.byref(d2))
    assert L.gemv2_mac_idle(ctypes.byref(d2)) == 1
    assert_bytes_equal(_read_y(L, y_host, rows), want, "gemv2 fetch + mac")
    L.gemv2_dev_close(ctypes.byref(d2))
    pool.used = 0


def _v2_check_case(L, pool, blocks, x_eng, rows, k):
    """bench_gemv2.c:47-79 (check_case): x and a 0xAA-poisoned y in the pool,
    the matrix in four 64 KB-aligned port regions with ports 1 and 3 offset by
    16 KB (new_mat, :29-40), rows placed by the chunk formula (put_row, :41-43),
    one fetch + MAC, the outputs read back after invalidate."""
    x_host, xp = _alloc(L, pool, np.concatenate([x_eng, np.zeros(64, np.uint8)]))
    y_host, yp = _poisoned_y(L, pool, rows)
    quarter = rows // 4 * k // 32 * 18
    ports, phys = [], []
    for p in range(4):
        off = (p & 1) * (16 << 10)
        host = L.udmabuf_alloc(ctypes.byref(pool), quarter + off, 64 << 10)
        assert host, "pool full"
        ports.append(np.ctypeslib.as_array((ctypes.c_uint8 * quarter).from_address(host + off)))
        phys.append(pool.phys + (host - pool.base) + off)
    raw = blocks.reshape(rows, k // 256, 144)
    for r in range(rows):
        for c in range(k // 256):
            o, port = _chunk_offset(r, c, rows, k)
            ports[port][o:o + 144] = raw[r, c]
    for p in range(4):
        L.udmabuf_clean(ports[p].ctypes.data, quarter)
    d2 = Dev2()
    assert L.gemv2_dev_open(ctypes.byref(d2)) == 0
    assert L.gemv2_mac_idle(ctypes.byref(d2)) == 1
    L.gemv2_fetch_start(ctypes.byref(d2), (u64 * 4)(*phys), k, rows)
    L.gemv2_mac_start(ctypes.byref(d2), xp, yp, k, rows)
    L.gemv2_mac_wait(ctypes.byref(d2))
    y = _read_y(L, y_host, rows)
    L.gemv2_dev_close(ctypes.byref(d2))
    return y


@pytest.fixture(scope="module")
def gen_vectors():
    """The reference's exactness cases (gen_vectors.py), regenerated by the
    oracle and checked against the committed digests before any GPU call."""
    with open(os.path.join(HERE, "golden", "gen_vectors.json")) as f:
        pinned = json.load(f)
    out = {}
    for group, cases in (("cases", GV.CASES), ("shard_cases", GV.SHARD_CASES)):
        for want, (k, rows, blocks, x_eng, y, _, _) in zip(pinned[group], GV.draw(cases)):
            sha = lambda a: hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()
            assert (want["k"], want["rows"]) == (k, rows)
            assert (sha(blocks), sha(x_eng), sha(y)) == (want["w"], want["x"], want["y"]), want["name"]
            out[want["name"]] = (k, rows, blocks, x_eng, y)
    return out


GEN_VECTOR_NAMES = ([f"k{k}_n{rows}" for k, rows in GV.CASES] +
                    [f"k{k}_n{rows}" for k, rows in GV.SHARD_CASES])


def _v1_run(L, pool, blocks, x_eng, rows, k):
    """The v1 engine's exactness run (evidence 0006-bench-gemv-kv260-01.txt:2-5):
    the rows contiguous at a 64 KB-aligned address, x, a poisoned y, one
    gemv_dev_run."""
    _, wp = _alloc(L, pool, blocks.reshape(-1), 64 << 10)
    _, xp = _alloc(L, pool, x_eng)
    y_host, yp = _poisoned_y(L, pool, rows)
    d = Dev()
    assert L.gemv_dev_open(ctypes.byref(d)) == 0
    L.gemv_dev_run(ctypes.byref(d), wp, xp, yp, k, rows)
    y = _read_y(L, y_host, rows)
    L.gemv_dev_close(ctypes.byref(d))
    return y


@pytest.mark.parametrize("name", GEN_VECTOR_NAMES)
def test_gen_vectors_exactness(board, gen_vectors, name):
    """Every case of gen_vectors.py, plus the shard shapes the board run names
    (0013-bench-gemv2.txt:1): through the v1 engine's gemv_dev_run (rows % 16,
    as the v1 bench ran the first three), and through gemv2_fetch_start /
    gemv2_mac_start as check_case issues them wherever gemv2's rows % 32
    holds (gemv2_dev.h:14). Bit-exact, every row written."""
    L, pool = board
    k, rows, blocks, x_eng, want = gen_vectors[name]
    assert rows % 16 == 0 and k % 256 == 0
    got = _v1_run(L, pool, blocks, x_eng, rows, k)
    pool.used = 0
    assert_bytes_equal(got, want, f"gen_vectors {name}, v1")
    if rows % 32 == 0:
        got = _v2_check_case(L, pool, blocks, x_eng, rows, k)
        pool.used = 0
        assert_bytes_equal(got, want, f"gen_vectors {name}, gemv2")


class _DeviceBytes:
    """A pool's device bytes at `phys`, for torch.as_tensor (CUDA array interface)."""

    def __init__(self, phys, n):
        self.__cuda_array_interface__ = {"shape": (n,), "typestr": "|u1", "data": (phys, False), "version": 3}


def test_pool_copies_follow_the_current_copy(board):
    """Which copy of a pool range is current: bytes written into the device copy
    from outside the engine calls reach the host through invalidate (in a range
    that is not host-current: a clean of 1 MiB or more copies at once and
    leaves none); a range the host cleaned is not overwritten by invalidate (its
    host bytes are the current ones); an engine call's y lands in the host
    copy, and a later clean of new bytes in that range reaches the next call
    that reads it."""
    import torch
    L, pool = board
    span = 1 << 20
    p = L.udmabuf_alloc(ctypes.byref(pool), span, 4096)
    L.udmabuf_clean(p, span)                          # copied at once: no part host-current
    n = 4096 + 20                                     # whole 16-byte pieces plus a ragged tail
    phys = pool.phys + (p - pool.base)
    host = np.ctypeslib.as_array((ctypes.c_uint8 * n).from_address(p))
    host[:] = 0x11
    dev_view = torch.as_tensor(_DeviceBytes(phys, n), device="cuda")
    dev_view.fill_(0x5A)                              # a write the engine calls know nothing of
    torch.cuda.synchronize()
    L.udmabuf_invalidate(p, n)
    assert (host == 0x5A).all()
    host[:] = 0x33
    L.udmabuf_clean(p, n)                             # host-current now: nothing copied yet
    L.udmabuf_invalidate(p, n)
    assert (host == 0x33).all(), "invalidate overwrote bytes the host had cleaned"
    # An engine call writes its y into the host copy; that range then takes,
    # cleaned, the second call's x (576 rows of y = the 2,304 bytes of an
    # engine-layout x at k = 2048), which the second call must read.
    k = 2048
    rows1 = (k + k // 8) // 4
    blocks, x_eng, want = _case(rows1, k, 77)
    _, wp = _alloc(L, pool, blocks.reshape(-1), 64 << 10)
    _, xp = _alloc(L, pool, x_eng)
    y_host, yp = _poisoned_y(L, pool, rows1)
    d = Dev()
    assert L.gemv_dev_open(ctypes.byref(d)) == 0
    L.gemv_dev_run(ctypes.byref(d), wp, xp, yp, k, rows1)
    assert_bytes_equal(_read_y(L, y_host, rows1), want, "first call")
    rows2 = 64
    blocks2, x2, want2 = _case(rows2, k, 78)
    assert len(x2) == 4 * rows1
    _, wp2 = _alloc(L, pool, blocks2.reshape(-1), 64 << 10)
    y2_host, yp2 = _poisoned_y(L, pool, rows2)
    ctypes.memmove(y_host, np.ascontiguousarray(x2).ctypes.data, len(x2))
    L.udmabuf_clean(y_host, len(x2))
    L.gemv_dev_run(ctypes.byref(d), wp2, yp, yp2, k, rows2)
    assert_bytes_equal(_read_y(L, y2_host, rows2), want2, "second call, x where the first call's y was")
    L.gemv_dev_close(ctypes.byref(d))
    pool.used = 0
