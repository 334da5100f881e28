"""Python front end of the MI355X W4A8 engine (libkv260gemv.so, C ABI in include/w4a8.h).

Mirrors the contract module's interface, src/llm_kv260/q4_0.py (same function
names, argument meaning and TypeError / ValueError behaviour), but every
array is a torch tensor on the GPU and every computation runs in the HIP
library. There is no CPU fallback: a missing library or device raises.

    blocks = quantize_q4_0(w)                 # float32 [N, K]  -> uint8 [N, K/32*18]
    xq, xd = quantize_q8_0(x)                 # float32 [K]     -> int8 [K], float16 [K/32]
    y = gemv_q4_0(blocks, k, xq, xd)          # float32 [N]
    y = gemv_q4_0_f32(blocks, k, x)           # quantize fused into the GEMV kernel
    Y = gemm_q4_0(blocks, k, xq_rows, xd_rows)  # M > 1, int8 MFMA, [M, N]

PyTorch is used for device memory and streams only; calls go on torch's
current stream of the tensors' device.
"""

from __future__ import annotations

import ctypes
import os

QK = 32
Q4_0_BYTES = 18
Q8_0_BYTES = 34
LANES = 8
MAX_K = 16384
CHAIN_ONE_LAUNCH = 0
CHAIN_PER_STEP = 1
CONTRACT_VERSION = "llm-kv260/w4a8-q4_0-v2"

_PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(_PKG_DIR, "libkv260gemv.so")

# Every symbol include/*.h declares (checked by the tests without a GPU).
EXPORTS = (
    # w4a8.h
    "w4a8_contract_version", "w4a8_strerror", "w4a8_last_hip_error",
    "w4a8_q4_0_row_bytes", "w4a8_engine_x_bytes", "w4a8_q8_0_row_bytes",
    "w4a8_gemv", "w4a8_gemv_q8_0", "w4a8_gemv_f32", "w4a8_gemv_quarters",
    "w4a8_quantize_q8_0", "w4a8_quantize_q8_0_blocks", "w4a8_quantize_q4_0", "w4a8_gemm",
    "w4a8_chain_gemv", "w4a8_gemv_batch", "w4a8_argmax_workspace_bytes", "w4a8_gemv_f32_argmax",
    "w4a8_gemv_rmsnorm", "w4a8_gemv_rmsnorm_argmax", "w4a8_gemv_silu_mul", "w4a8_rmsnorm_q8_0",
    "w4a8_silu_mul_q8_0", "w4a8_topk_workspace_bytes", "w4a8_topk", "w4a8_topk_no_alloc", "w4a8_gemv_gate_up_silu",
    "w4a8_gemv_gate_up_silu_q8_0",
    "w4a8_chain_set_mode", "w4a8_chain_set_spin_limit", "w4a8_chain_timeouts",
    "w4a8_chain_plan_create", "w4a8_chain_plan_create_steps", "w4a8_chain_plan_launch", "w4a8_chain_plan_wait",
    "w4a8_chain_plan_destroy", "w4a8_chain_plan_create_overlapped", "w4a8_chain_plan_launch_timed", "w4a8_chain_plan_workgroups",
    "w4a8_wall_clock_hz",
    # w4a8_gguf.h
    "w4a8_gguf_open", "w4a8_gguf_close", "w4a8_gguf_version", "w4a8_gguf_n_tensors", "w4a8_gguf_n_kv",
    "w4a8_gguf_data_offset", "w4a8_gguf_find_key", "w4a8_gguf_find_tensor", "w4a8_gguf_key",
    "w4a8_gguf_kv_type", "w4a8_gguf_get_u32", "w4a8_gguf_get_i32", "w4a8_gguf_get_u64", "w4a8_gguf_get_f32",
    "w4a8_gguf_get_str", "w4a8_gguf_tensor_info", "w4a8_gguf_tensor_data", "w4a8_gguf_upload",
    # gemv_dev.h
    "gemv_dev_open", "gemv_dev_open_named", "gemv_dev_close", "gemv_dev_run",
    "gemv_dev_start", "gemv_dev_wait", "gemv_dev_start4",
    # gemv2_dev.h
    "gemv2_dev_open", "gemv2_dev_close", "gemv2_fetch_start", "gemv2_fetch_wait",
    "gemv2_mac_start", "gemv2_mac_wait", "gemv2_mac_idle", "gemv2_drain",
    # udmabuf.h
    "udmabuf_open", "udmabuf_close", "udmabuf_alloc", "udmabuf_clean", "udmabuf_invalidate",
)

_lib = None


class W4A8Error(RuntimeError):
    """A non-zero status from the C ABI."""

    def __init__(self, fn: str, status: int, hip_error: int = 0):
        msg = f"{fn}: {strerror(status)} (status {status}"
        if hip_error:
            msg += f", hipError {hip_error}"
        super().__init__(msg + ")")
        self.status = status


def lib() -> ctypes.CDLL:
    """Load libkv260gemv.so (built in-tree by `make -C llm-kv260_amd`)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is not built; run `make -C llm-kv260_amd` (or __graft_entry__.build())")
    try:  # share torch's HIP runtime (same soname) when torch is importable
        import torch  # noqa: F401
    except ImportError:
        pass
    L = ctypes.CDLL(LIB_PATH)
    p, i = ctypes.c_void_p, ctypes.c_int
    L.w4a8_contract_version.restype = ctypes.c_char_p
    L.w4a8_strerror.argtypes = [i]
    L.w4a8_strerror.restype = ctypes.c_char_p
    L.w4a8_last_hip_error.restype = i
    for f in ("w4a8_q4_0_row_bytes", "w4a8_engine_x_bytes", "w4a8_q8_0_row_bytes"):
        getattr(L, f).argtypes = [i]
        getattr(L, f).restype = ctypes.c_size_t
    for f in ("w4a8_gemv", "w4a8_gemv_q8_0", "w4a8_gemv_f32"):
        getattr(L, f).argtypes = [p, p, p, i, i, p]
        getattr(L, f).restype = i
    L.w4a8_gemv_quarters.argtypes = [ctypes.POINTER(p), p, p, i, i, p]
    L.w4a8_gemv_quarters.restype = i
    for f in ("w4a8_quantize_q8_0", "w4a8_quantize_q8_0_blocks", "w4a8_quantize_q4_0"):
        getattr(L, f).argtypes = [p, p, i, i, p]
        getattr(L, f).restype = i
    L.w4a8_gemm.argtypes = [p, p, p, i, i, i, p]
    L.w4a8_gemm.restype = i
    L.w4a8_argmax_workspace_bytes.argtypes = []
    L.w4a8_argmax_workspace_bytes.restype = ctypes.c_size_t
    L.w4a8_gemv_f32_argmax.argtypes = [p, p, p, i, i, p, p, ctypes.c_size_t, p]
    L.w4a8_gemv_f32_argmax.restype = i
    f32 = ctypes.c_float
    L.w4a8_gemv_rmsnorm.argtypes = [p, p, p, f32, p, i, i, p]
    L.w4a8_gemv_rmsnorm.restype = i
    L.w4a8_gemv_rmsnorm_argmax.argtypes = [p, p, p, f32, p, i, i, p, p, ctypes.c_size_t, p]
    L.w4a8_gemv_rmsnorm_argmax.restype = i
    L.w4a8_gemv_silu_mul.argtypes = [p, p, p, i, i, p]
    L.w4a8_gemv_silu_mul.restype = i
    L.w4a8_rmsnorm_q8_0.argtypes = [p, p, f32, p, i, i, p]
    L.w4a8_rmsnorm_q8_0.restype = i
    L.w4a8_silu_mul_q8_0.argtypes = [p, p, i, i, p]
    L.w4a8_silu_mul_q8_0.restype = i
    L.w4a8_topk_workspace_bytes.argtypes = [i]
    L.w4a8_topk_workspace_bytes.restype = ctypes.c_size_t
    L.w4a8_topk.argtypes = [p, i, i, p, p, p, ctypes.c_size_t, p]
    L.w4a8_topk.restype = i
    L.w4a8_topk_no_alloc.argtypes = [p, i, i, p, p, p]
    L.w4a8_topk_no_alloc.restype = i
    L.w4a8_gemv_gate_up_silu.argtypes = [p, p, p, f32, p, i, i, p]
    L.w4a8_gemv_gate_up_silu.restype = i
    L.w4a8_gemv_gate_up_silu_q8_0.argtypes = [p, p, p, f32, p, i, i, p]
    L.w4a8_gemv_gate_up_silu_q8_0.restype = i
    for f in ("w4a8_chain_gemv", "w4a8_gemv_batch"):
        getattr(L, f).argtypes = [p, i, p]
        getattr(L, f).restype = i
    for f in ("w4a8_chain_set_mode", "w4a8_chain_set_spin_limit"):
        getattr(L, f).argtypes = [i]
        getattr(L, f).restype = i
    L.w4a8_chain_timeouts.argtypes = []
    L.w4a8_chain_timeouts.restype = i
    for f in ("w4a8_chain_plan_create", "w4a8_chain_plan_create_steps", "w4a8_chain_plan_create_overlapped"):
        getattr(L, f).argtypes = [p, i, ctypes.POINTER(p)]
        getattr(L, f).restype = i
    for f in ("w4a8_chain_plan_launch", "w4a8_chain_plan_wait"):
        getattr(L, f).argtypes = [p, i]
        getattr(L, f).restype = i
    L.w4a8_chain_plan_destroy.argtypes = [p]
    L.w4a8_chain_plan_destroy.restype = i
    L.w4a8_chain_plan_launch_timed.argtypes = [p, i, p]
    L.w4a8_chain_plan_launch_timed.restype = i
    L.w4a8_chain_plan_workgroups.argtypes = [p, i]
    L.w4a8_chain_plan_workgroups.restype = ctypes.c_long
    L.w4a8_wall_clock_hz.argtypes = [ctypes.POINTER(ctypes.c_int64)]
    L.w4a8_wall_clock_hz.restype = i
    _lib = L
    return L


PLAN_GEMV, PLAN_GATE_UP_SILU, PLAN_ARGMAX, PLAN_GATE_UP_SILU_Q8, PLAN_GEMV_ENGINE = 0, 1, 2, 3, 4
CHAIN_MAX_STEPS = 96           # W4A8_CHAIN_MAX_STEPS: steps per chain, batch or plan


class PlanStep(ctypes.Structure):
    """include/w4a8.h's w4a8_plan_step."""
    _fields_ = [("kind", ctypes.c_int), ("w", ctypes.c_void_p), ("x", ctypes.c_void_p), ("y", ctypes.c_void_p),
                ("rows", ctypes.c_int), ("k", ctypes.c_int), ("norm_w", ctypes.c_void_p), ("eps", ctypes.c_float),
                ("argmax", ctypes.c_void_p), ("workspace", ctypes.c_void_p)]


def strerror(status: int) -> str:
    return lib().w4a8_strerror(status).decode()


def check(fn: str, status: int) -> None:
    if status != 0:
        raise W4A8Error(fn, status, lib().w4a8_last_hip_error())


def require_device(index: int = 0) -> None:
    """Raise unless a gfx950 GPU is usable and the library is loaded."""
    import torch
    lib()
    if not torch.cuda.is_available():
        raise RuntimeError("no GPU visible to torch")
    arch = torch.cuda.get_device_properties(index).gcnArchName
    if not arch.startswith("gfx950"):
        raise RuntimeError(f"device {index} is {arch}, the engine is built for gfx950")


def _stream(t) -> int:
    import torch
    return torch.cuda.current_stream(t.device).cuda_stream


def _need(t, dtype, name):
    import torch
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch tensor, got {type(t).__name__}")
    if t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")
    if not t.is_cuda:
        raise ValueError(f"{name} must be on the GPU")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def _out(out, shape, dtype, like, name="out"):
    """The caller's output tensor, checked before anything is launched (dtype,
    device, contiguity and at least the elements the call writes), or a new
    one. The C ABI sees only its address, so a short tensor would be written
    past its end."""
    import torch
    numel = 1
    for s in shape:
        numel *= s
    if out is None:
        return torch.empty(shape, dtype=dtype, device=like.device)
    if not isinstance(out, torch.Tensor):
        raise TypeError(f"{name} must be a torch tensor, got {type(out).__name__}")
    if out.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {out.dtype}")
    if not out.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if out.numel() < numel:
        raise ValueError(f"{name} holds {out.numel()} elements, the call writes {numel}")
    if not out.is_cuda or out.device != like.device:
        raise ValueError(f"{name} must be on {like.device}, got {out.device}")
    return out


def _same_device(t, like, name):
    if t.device != like.device:
        raise ValueError(f"{name} is on {t.device}, the weights on {like.device}")


def _check_k(k: int) -> None:
    if k % 256 or not 256 <= k <= MAX_K:
        raise ValueError(f"K={k}: the engine needs K % 256 == 0 and 256 <= K <= {MAX_K}")


# ------------------------------------------------------------------ sizes

def q4_0_row_bytes(k: int) -> int:
    return k // QK * Q4_0_BYTES


def engine_x_bytes(k: int) -> int:
    return k + k // QK * 4


# ------------------------------------------------------------- quantizers

def quantize_q8_0_engine(x, out=None):
    """float32 [K] or [M, K] -> engine layout uint8 [K + K/8] (or [M, K + K/8]), on the GPU."""
    import torch
    _need(x, torch.float32, "x")
    if x.dim() not in (1, 2) or x.shape[-1] % QK:
        raise ValueError(f"x must be [K] or [M, K] with K a multiple of {QK}, got {tuple(x.shape)}")
    k = x.shape[-1]
    _check_k(k)
    m = 1 if x.dim() == 1 else x.shape[0]
    shape = (engine_x_bytes(k),) if x.dim() == 1 else (m, engine_x_bytes(k))
    out = _out(out, shape, torch.uint8, x)
    check("w4a8_quantize_q8_0", lib().w4a8_quantize_q8_0(x.data_ptr(), out.data_ptr(), k, m, _stream(x)))
    return out


def quantize_q8_0(x):
    """Contract interface (q4_0.py:83-97): float32 [K] -> (int8 [K], float16 [K/32])."""
    import torch
    _need(x, torch.float32, "x")
    if x.dim() != 1 or x.shape[0] % QK:
        raise ValueError(f"x must be 1-D with a multiple of {QK} elements, got {tuple(x.shape)}")
    k = x.shape[0]
    if k % 256 or not 256 <= k <= MAX_K:
        raise ValueError(f"K={k}: the engine quantizer needs K % 256 == 0 and 256 <= K <= {MAX_K}")
    blocks = torch.empty((k // QK, Q8_0_BYTES), dtype=torch.uint8, device=x.device)
    check("w4a8_quantize_q8_0_blocks",
          lib().w4a8_quantize_q8_0_blocks(x.data_ptr(), blocks.data_ptr(), k, 1, _stream(x)))
    xd = blocks[:, :2].contiguous().view(torch.float16).reshape(-1)
    xq = blocks[:, 2:].contiguous().view(torch.int8).reshape(-1)
    return xq, xd


def quantize_q4_0(w):
    """Contract interface (q4_0.py:100-121): float32 [N, K] -> uint8 [N, K/32*18]."""
    import torch
    _need(w, torch.float32, "weights")
    if w.dim() != 2:
        raise ValueError(f"weights must be [N, K], got {tuple(w.shape)}")
    n, k = w.shape
    if k % QK:
        raise ValueError(f"in_features must be a multiple of {QK}, got {k}")
    out = torch.empty((n, k // QK * Q4_0_BYTES), dtype=torch.uint8, device=w.device)
    check("w4a8_quantize_q4_0", lib().w4a8_quantize_q4_0(w.data_ptr(), out.data_ptr(), n, k, _stream(w)))
    return out


def pack_x_for_engine(xq, xd):
    """Engine layout int8[K] then float32[K/32] (q4_0.py:193-200), on the GPU."""
    import torch
    _need(xq, torch.int8, "xq")
    _need(xd, torch.float16, "xd")
    return torch.cat([xq.view(torch.uint8), xd.float().view(torch.uint8)])


# ------------------------------------------------------------------- gemv

def _check_blocks(blocks, k):
    import torch
    _need(blocks, torch.uint8, "blocks")
    if blocks.dim() != 2 or blocks.shape[1] != k // QK * Q4_0_BYTES:
        raise ValueError(f"{tuple(blocks.shape)} is not [N, {k // QK} blocks of {Q4_0_BYTES}]")
    if (k // QK) % LANES:
        raise ValueError(f"{k // QK} blocks is not a multiple of {LANES} lanes")
    _check_k(k)


def gemv_engine(blocks, k: int, x_engine, out=None):
    """y = W x with x already in the engine layout (uint8 [K + K/8])."""
    import torch
    _check_blocks(blocks, k)
    _need(x_engine, torch.uint8, "x")
    if x_engine.numel() != engine_x_bytes(k):
        raise ValueError(f"engine x must be {engine_x_bytes(k)} bytes, got {x_engine.numel()}")
    _same_device(x_engine, blocks, "x")
    n = blocks.shape[0]
    y = _out(out, (n,), torch.float32, blocks)
    check("w4a8_gemv", lib().w4a8_gemv(blocks.data_ptr(), x_engine.data_ptr(), y.data_ptr(), n, k,
                                       _stream(blocks)))
    return y


def gemv_q4_0(blocks, k: int, xq, xd):
    """Contract interface (q4_0.py:151-182): y float32 [N], on the GPU."""
    import torch
    if xq.dtype != torch.int8 or xd.dtype != torch.float16:
        raise TypeError(f"x must be (int8, float16), got ({xq.dtype}, {xd.dtype})")
    _check_blocks(blocks, k)
    if tuple(xq.shape) != (k,) or tuple(xd.shape) != (k // QK,):
        raise ValueError(f"x shapes {tuple(xq.shape)}, {tuple(xd.shape)} do not match K={k}")
    return gemv_engine(blocks, k, pack_x_for_engine(xq, xd))


def gemv_q4_0_f32(blocks, k: int, x, out=None):
    """Contract interface (q4_0.py:185-188); the Q8_0 quantize runs inside the GEMV kernel."""
    import torch
    _need(x, torch.float32, "x")
    _check_blocks(blocks, k)
    if tuple(x.shape) != (k,):
        raise ValueError(f"x must be [{k}], got {tuple(x.shape)}")
    _same_device(x, blocks, "x")
    n = blocks.shape[0]
    y = _out(out, (n,), torch.float32, blocks)
    check("w4a8_gemv_f32", lib().w4a8_gemv_f32(blocks.data_ptr(), x.data_ptr(), y.data_ptr(), n, k,
                                               _stream(blocks)))
    return y


def argmax_workspace():
    """A zero-filled workspace for gemv_q4_0_f32_argmax on the current device."""
    import torch
    return torch.zeros(lib().w4a8_argmax_workspace_bytes(), dtype=torch.uint8, device="cuda")


def gemv_gate_up_silu(blocks, k: int, x, norm_w=None, eps: float = 1e-5, out=None, q8: bool = False):
    """act = silu(gate) * up of the gate|up GEMV y = W Q8_0(rmsnorm(x) * norm_w)
    (or of x itself when norm_w is None), rows = 2n gate rows then up rows:
    float32 [n], in one kernel (board/tp/tp_llama.cpp:557-569, 612-619).
    q8: act quantized in the same kernel, returned in the engine layout
    (uint8 [n + n/8], the input of gemv_engine; k = 2048 only)."""
    import torch
    _need(x, torch.float32, "x")
    _check_blocks(blocks, k)
    if tuple(x.shape) != (k,):
        raise ValueError(f"x must be [{k}], got {tuple(x.shape)}")
    _same_device(x, blocks, "x")
    rows = blocks.shape[0]
    if rows % 2:
        raise ValueError(f"gate|up needs an even number of rows (gate rows, then up rows), got {rows}")
    if norm_w is not None:
        _need(norm_w, torch.float32, "norm_w")
        if tuple(norm_w.shape) != (k,):
            raise ValueError(f"norm_w must be [{k}], got {tuple(norm_w.shape)}")
        _same_device(norm_w, blocks, "norm_w")
    if q8:
        act = _out(out, (engine_x_bytes(rows // 2),), torch.uint8, blocks)
        fn = "w4a8_gemv_gate_up_silu_q8_0"
    else:
        act = _out(out, (rows // 2,), torch.float32, blocks)
        fn = "w4a8_gemv_gate_up_silu"
    check(fn, getattr(lib(), fn)(
        blocks.data_ptr(), x.data_ptr(), None if norm_w is None else norm_w.data_ptr(), float(eps), act.data_ptr(),
        rows, k, _stream(blocks)))
    return act


def topk(y, k: int, workspace=None):
    """The sampler's k candidates of the logits y (board/tp/tp_llama.cpp:894-909):
    (vals float32 [k], idx int32 [k]) on the GPU, values descending, the smaller
    index first among equals, never a value at or below -1e30 (left-over slots
    hold -1e30 and index 0). 1 <= k <= 64."""
    import torch
    _need(y, torch.float32, "y")
    if y.dim() != 1:
        raise ValueError(f"y must be 1-D, got {tuple(y.shape)}")
    n = y.shape[0]
    if workspace is None:
        workspace = torch.empty(max(lib().w4a8_topk_workspace_bytes(n), 8), dtype=torch.uint8, device=y.device)
    vals = torch.empty(k, dtype=torch.float32, device=y.device)
    idx = torch.empty(k, dtype=torch.int32, device=y.device)
    check("w4a8_topk", lib().w4a8_topk(y.data_ptr(), n, k, vals.data_ptr(), idx.data_ptr(), workspace.data_ptr(),
                                       workspace.numel() * workspace.element_size(), _stream(y)))
    return vals, idx


def gemv_q4_0_f32_argmax(blocks, k: int, x, workspace, out=None):
    """The LM head and its greedy pick in one launch: (y, argmax) with argmax an
    int32 [1] GPU tensor holding the first row of the largest y
    (board/tp/tp_llama.cpp:879-880). `workspace` comes from argmax_workspace()."""
    import torch
    _need(x, torch.float32, "x")
    _check_blocks(blocks, k)
    if tuple(x.shape) != (k,):
        raise ValueError(f"x must be [{k}], got {tuple(x.shape)}")
    _same_device(x, blocks, "x")
    _need(workspace, torch.uint8, "workspace")
    _same_device(workspace, blocks, "workspace")
    n = blocks.shape[0]
    y = _out(out, (n,), torch.float32, blocks)
    best = torch.empty(1, dtype=torch.int32, device=blocks.device)
    check("w4a8_gemv_f32_argmax", lib().w4a8_gemv_f32_argmax(
        blocks.data_ptr(), x.data_ptr(), y.data_ptr(), n, k, best.data_ptr(), workspace.data_ptr(),
        workspace.numel() * workspace.element_size(), _stream(blocks)))
    return y, best


def gemv_rmsnorm(blocks, k: int, x, norm_w, eps: float, out=None):
    """y = W Q8_0(rmsnorm(x) * norm_w), rmsnorm as board/tp/tp_llama.cpp:557-569, in one kernel."""
    import torch
    _need(x, torch.float32, "x")
    _need(norm_w, torch.float32, "norm_w")
    _check_blocks(blocks, k)
    if tuple(x.shape) != (k,) or tuple(norm_w.shape) != (k,):
        raise ValueError(f"x and norm_w must be [{k}]")
    _same_device(x, blocks, "x")
    _same_device(norm_w, blocks, "norm_w")
    n = blocks.shape[0]
    y = _out(out, (n,), torch.float32, blocks)
    check("w4a8_gemv_rmsnorm", lib().w4a8_gemv_rmsnorm(blocks.data_ptr(), x.data_ptr(), norm_w.data_ptr(), eps,
                                                       y.data_ptr(), n, k, _stream(blocks)))
    return y


def gemv_rmsnorm_argmax(blocks, k: int, x, norm_w, eps: float, workspace, out=None):
    """The LM head step: rmsnorm, Q8_0, GEMV and the greedy pick in one kernel -> (y, argmax)."""
    import torch
    _need(x, torch.float32, "x")
    _need(norm_w, torch.float32, "norm_w")
    _check_blocks(blocks, k)
    if tuple(x.shape) != (k,) or tuple(norm_w.shape) != (k,):
        raise ValueError(f"x and norm_w must be [{k}]")
    _same_device(x, blocks, "x")
    _same_device(norm_w, blocks, "norm_w")
    _need(workspace, torch.uint8, "workspace")
    _same_device(workspace, blocks, "workspace")
    n = blocks.shape[0]
    y = _out(out, (n,), torch.float32, blocks)
    best = torch.empty(1, dtype=torch.int32, device=blocks.device)
    check("w4a8_gemv_rmsnorm_argmax", lib().w4a8_gemv_rmsnorm_argmax(
        blocks.data_ptr(), x.data_ptr(), norm_w.data_ptr(), eps, y.data_ptr(), n, k, best.data_ptr(),
        workspace.data_ptr(), workspace.numel() * workspace.element_size(), _stream(blocks)))
    return y, best


def gemv_silu_mul(blocks, k: int, gate_up, out=None):
    """y = W Q8_0(silu(gate) * up) with gate_up = gate | up, float32 [2k], in one kernel."""
    import torch
    _need(gate_up, torch.float32, "gate_up")
    _check_blocks(blocks, k)
    if tuple(gate_up.shape) != (2 * k,):
        raise ValueError(f"gate_up must be [{2 * k}]")
    _same_device(gate_up, blocks, "gate_up")
    n = blocks.shape[0]
    y = _out(out, (n,), torch.float32, blocks)
    check("w4a8_gemv_silu_mul", lib().w4a8_gemv_silu_mul(blocks.data_ptr(), gate_up.data_ptr(), y.data_ptr(), n, k,
                                                         _stream(blocks)))
    return y


def rmsnorm_q8_0_engine(x, norm_w, eps: float):
    """Engine-layout rows of Q8_0(rmsnorm(x) * norm_w) for x float32 [k] or [m, k]."""
    import torch
    _need(x, torch.float32, "x")
    _need(norm_w, torch.float32, "norm_w")
    if x.dim() not in (1, 2):
        raise ValueError(f"x must be [k] or [m, k], got {tuple(x.shape)}")
    k = x.shape[-1]
    _check_k(k)
    if tuple(norm_w.shape) != (k,):
        raise ValueError(f"norm_w must be [{k}], got {tuple(norm_w.shape)}")
    _same_device(norm_w, x, "norm_w")
    m = 1 if x.dim() == 1 else x.shape[0]
    out = torch.empty((m, k + k // 8), dtype=torch.uint8, device=x.device)
    check("w4a8_rmsnorm_q8_0", lib().w4a8_rmsnorm_q8_0(x.data_ptr(), norm_w.data_ptr(), eps, out.data_ptr(), k, m,
                                                       _stream(x)))
    return out if x.dim() == 2 else out[0]


def silu_mul_q8_0_engine(gate_up):
    """Engine-layout rows of Q8_0(silu(gate) * up) for gate_up float32 [2k] or [m, 2k]."""
    import torch
    _need(gate_up, torch.float32, "gate_up")
    if gate_up.dim() not in (1, 2) or gate_up.shape[-1] % 2:
        raise ValueError(f"gate_up must be [2k] or [m, 2k], got {tuple(gate_up.shape)}")
    k = gate_up.shape[-1] // 2
    _check_k(k)
    m = 1 if gate_up.dim() == 1 else gate_up.shape[0]
    out = torch.empty((m, k + k // 8), dtype=torch.uint8, device=gate_up.device)
    check("w4a8_silu_mul_q8_0", lib().w4a8_silu_mul_q8_0(gate_up.data_ptr(), out.data_ptr(), k, m, _stream(gate_up)))
    return out if gate_up.dim() == 2 else out[0]


def gemv_q8_0_blocks(blocks, k: int, x_blocks, out=None):
    """y = W x with x as ggml Q8_0 blocks (uint8 [K/32*34])."""
    import torch
    _check_blocks(blocks, k)
    _need(x_blocks, torch.uint8, "x_blocks")
    if x_blocks.numel() != k // QK * Q8_0_BYTES:
        raise ValueError(f"Q8_0 x must be {k // QK * Q8_0_BYTES} bytes")
    _same_device(x_blocks, blocks, "x_blocks")
    n = blocks.shape[0]
    y = _out(out, (n,), torch.float32, blocks)
    check("w4a8_gemv_q8_0", lib().w4a8_gemv_q8_0(blocks.data_ptr(), x_blocks.data_ptr(), y.data_ptr(), n, k,
                                                 _stream(blocks)))
    return y


def gemv_quarters(quarters, k: int, x_engine, rows: int, out=None):
    """The v1 engine's four-quarter layout: quarter m = rows/4 rows at its own tensor."""
    import torch
    if len(quarters) != 4:
        raise ValueError("need four quarters")
    _check_k(k)
    if rows < 4 or rows % 4:
        raise ValueError(f"rows must be a positive multiple of 4, got {rows}")
    _need(x_engine, torch.uint8, "x")
    if x_engine.numel() != engine_x_bytes(k):
        raise ValueError(f"engine x must be {engine_x_bytes(k)} bytes, got {x_engine.numel()}")
    quarter_bytes = rows // 4 * q4_0_row_bytes(k)
    for q in quarters:
        _need(q, torch.uint8, "quarter")
        _same_device(q, x_engine, "quarter")
        if q.numel() < quarter_bytes:
            raise ValueError(f"a quarter holds {q.numel()} bytes, {rows // 4} rows need {quarter_bytes}")
    y = _out(out, (rows,), torch.float32, x_engine)
    arr = (ctypes.c_void_p * 4)(*[q.data_ptr() for q in quarters])
    check("w4a8_gemv_quarters", lib().w4a8_gemv_quarters(arr, x_engine.data_ptr(), y.data_ptr(), rows, k,
                                                         _stream(x_engine)))
    return y


def gemm_engine(blocks, k: int, x_rows, out=None):
    """Y[M, N] for M activation rows already in the engine layout (uint8 [M, K + K/8])."""
    import torch
    _check_blocks(blocks, k)
    _need(x_rows, torch.uint8, "x_rows")
    if x_rows.dim() != 2 or x_rows.shape[1] != engine_x_bytes(k):
        raise ValueError(f"x_rows must be [M, {engine_x_bytes(k)}], got {tuple(x_rows.shape)}")
    _same_device(x_rows, blocks, "x_rows")
    m, n = x_rows.shape[0], blocks.shape[0]
    y = _out(out, (m, n), torch.float32, blocks)
    check("w4a8_gemm", lib().w4a8_gemm(blocks.data_ptr(), x_rows.data_ptr(), y.data_ptr(), m, n, k,
                                       _stream(blocks)))
    return y


def gemm_q4_0(blocks, k: int, xq, xd):
    """M > 1: each row of (xq int8 [M, K], xd float16 [M, K/32]) through the contract, [M, N]."""
    import torch
    if xq.dtype != torch.int8 or xd.dtype != torch.float16:
        raise TypeError(f"x must be (int8, float16), got ({xq.dtype}, {xd.dtype})")
    m = xq.shape[0]
    x_rows = torch.cat([xq.view(torch.uint8), xd.float().contiguous().view(torch.uint8).reshape(m, -1)], dim=1)
    return gemm_engine(blocks, k, x_rows.contiguous())
