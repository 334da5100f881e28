"""ctypes front end of the scalar C oracle (`q4_0_oracle.c`).

TEST INFRASTRUCTURE ONLY (tests/, __graft_entry__.smoke(), bench.py's
cpu_baseline leg). Same functions and argument meaning as `q4_0_oracle.py`,
but fast enough for the full-size configurations (the 128256 x 2048 LM head,
the 65-matrix decode chain), parallel over rows with OpenMP.
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle_q4_0.so")
_lib = None

QK = 32
Q4_0_BYTES = 18


def build() -> str:
    """Compile the oracle library in place (gcc; a second or so)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        p, i64, c_int = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
        L.oracle_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.oracle_f16_to_f32.restype = ctypes.c_float
        L.oracle_f32_to_f16.argtypes = [ctypes.c_float]
        L.oracle_f32_to_f16.restype = ctypes.c_uint16
        L.oracle_quantize_q8_0.argtypes = [p, p, p, i64]
        L.oracle_quantize_q4_0.argtypes = [p, p, i64, i64, c_int]
        L.oracle_gemv_q4_0.argtypes = [p, p, p, p, i64, i64, c_int]
        L.oracle_gemm_q4_0.argtypes = [p, p, p, p, i64, i64, i64, c_int]
        L.oracle_pack_x_for_engine.argtypes = [p, p, p, i64]
        L.oracle_contract_version.restype = ctypes.c_char_p
        L.oracle_rmsnorm.argtypes = [p, p, i64, ctypes.c_float, p]
        L.oracle_ggml_expf.argtypes = [ctypes.c_float]
        L.oracle_ggml_expf.restype = ctypes.c_float
        L.oracle_silu_mul.argtypes = [p, p, i64, p]
        L.oracle_topk.argtypes = [p, i64, ctypes.c_int, p, p]
        _lib = L
    return _lib


def _ptr(a: np.ndarray) -> int:
    assert a.flags.c_contiguous
    return a.ctypes.data


def default_threads() -> int:
    return len(os.sched_getaffinity(0))


def f16_to_f32(h: int) -> float:
    return lib().oracle_f16_to_f32(h)


def f32_to_f16_bits(f: float) -> int:
    return lib().oracle_f32_to_f16(f)


def quantize_q8_0(x: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    x = np.ascontiguousarray(x, dtype=np.float32)
    k = x.shape[0]
    q = np.empty(k, np.int8)
    d = np.empty(k // QK, np.uint16)
    lib().oracle_quantize_q8_0(_ptr(x), _ptr(q), _ptr(d), k)
    return q, d.view(np.float16)


def quantize_q8_0_rows(x: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    out = [quantize_q8_0(r) for r in x]
    return np.stack([q for q, _ in out]), np.stack([d for _, d in out])


def quantize_q4_0(w: np.ndarray, threads: int | None = None) -> np.ndarray:
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows, k = w.shape
    out = np.empty((rows, k // QK * Q4_0_BYTES), np.uint8)
    lib().oracle_quantize_q4_0(_ptr(w), _ptr(out), rows, k, threads or default_threads())
    return out


def gemv_q4_0(blocks: np.ndarray, k: int, xq: np.ndarray, xd: np.ndarray,
              threads: int | None = None) -> np.ndarray:
    blocks = np.ascontiguousarray(blocks)
    rows = blocks.shape[0]
    xq = np.ascontiguousarray(xq, dtype=np.int8)
    xd16 = np.ascontiguousarray(xd, dtype=np.float16).view(np.uint16)
    y = np.empty(rows, np.float32)
    lib().oracle_gemv_q4_0(_ptr(blocks), _ptr(xq), _ptr(xd16), _ptr(y), rows, k,
                           threads or default_threads())
    return y


def gemm_q4_0_rows(blocks: np.ndarray, k: int, xq: np.ndarray, xd: np.ndarray,
                   threads: int | None = None) -> np.ndarray:
    blocks = np.ascontiguousarray(blocks)
    rows = blocks.shape[0]
    m = xq.shape[0]
    xq = np.ascontiguousarray(xq, dtype=np.int8)
    xd16 = np.ascontiguousarray(xd, dtype=np.float16).view(np.uint16)
    y = np.empty((m, rows), np.float32)
    lib().oracle_gemm_q4_0(_ptr(blocks), _ptr(xq), _ptr(xd16), _ptr(y), m, rows, k,
                           threads or default_threads())
    return y


def pack_x_for_engine(xq: np.ndarray, xd: np.ndarray) -> np.ndarray:
    k = xq.shape[0]
    out = np.empty(k + 4 * (k // QK), np.uint8)
    xq = np.ascontiguousarray(xq, dtype=np.int8)
    xd16 = np.ascontiguousarray(xd, dtype=np.float16).view(np.uint16)
    lib().oracle_pack_x_for_engine(_ptr(xq), _ptr(xd16), _ptr(out), k)
    return out


def contract_version() -> str:
    return lib().oracle_contract_version().decode()


# ------------------------------------------------ producers of the activation

def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    """board/tp/tp_llama.cpp:557-569 on float32 [n] (n % 4 == 0)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    out = np.empty_like(x)
    lib().oracle_rmsnorm(x.ctypes.data, w.ctypes.data, x.size, float(eps), out.ctypes.data)
    return out


def ggml_expf(x) -> np.float32:
    return np.float32(lib().oracle_ggml_expf(float(x)))


def silu_mul(g: np.ndarray, u: np.ndarray) -> np.ndarray:
    """board/tp/tp_llama.cpp:612-619 on float32 [n]."""
    g = np.ascontiguousarray(g, dtype=np.float32)
    u = np.ascontiguousarray(u, dtype=np.float32)
    out = np.empty_like(g)
    lib().oracle_silu_mul(g.ctypes.data, u.ctypes.data, g.size, out.ctypes.data)
    return out


def topk(y: np.ndarray, k: int):
    """board/tp/tp_llama.cpp:894-909's candidate selection on float32 [n]:
    (vals float32 [k], idx int32 [k])."""
    y = np.ascontiguousarray(y, dtype=np.float32)
    vals = np.empty(k, dtype=np.float32)
    idx = np.empty(k, dtype=np.int32)
    lib().oracle_topk(y.ctypes.data, y.size, int(k), vals.ctypes.data, idx.ctypes.data)
    return vals, idx
