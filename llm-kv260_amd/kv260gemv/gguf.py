"""GGUF model files through the library's reader (include/w4a8_gguf.h).

The reference loads weights from GGUF with llama.cpp's gguf API and copies
each Q4_0 tensor's rows into engine memory as they lie (board/tp/
tp_llama.cpp:149-208). Here the same file is parsed by the C library over a
read-only mmap, and a tensor's bytes are copied unchanged into a torch device
tensor: for a Q4_0 tensor of ne = [k, rows] that is the uint8 [rows, k/32*18]
weight matrix the GEMV entry points read in place.

    with GGUFFile(path) as f:
        n_layer = f.u32("llama.block_count")
        w = f.upload("blk.0.attn_q.weight")     # uint8 [rows, k/32*18] on the GPU
        y = kv260gemv.gemv_q4_0_f32(w, f.tensor("blk.0.attn_q.weight").ne[0], x)
"""

from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass

from . import W4A8Error, lib

GGML_TYPE_F32, GGML_TYPE_F16, GGML_TYPE_Q4_0, GGML_TYPE_Q8_0 = 0, 1, 2, 8
ERR_FORMAT = -6


def _text(b: bytes) -> str:
    """Key, name and string bytes as text. GGUF strings are UTF-8; bytes that are
    not decode to lone surrogates, so every name still round-trips through _raw."""
    return b.decode("utf-8", "surrogateescape")


def _raw(s: str) -> bytes:
    return s.encode("utf-8", "surrogateescape")


class _Tensor(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("type", ctypes.c_uint32), ("n_dims", ctypes.c_uint32),
                ("ne", ctypes.c_uint64 * 4), ("offset", ctypes.c_uint64), ("nbytes", ctypes.c_uint64)]


@dataclass(frozen=True)
class TensorInfo:
    name: str
    type: int
    ne: tuple          # ne[0] = elements per row, n_dims entries
    offset: int        # from the start of the data section
    nbytes: int


_bound = False


def _bind():
    global _bound
    L = lib()
    if _bound:
        return L
    p, i, i64, u64, s = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_uint64, ctypes.c_char_p
    L.w4a8_gguf_open.argtypes = [s, ctypes.POINTER(p)]
    L.w4a8_gguf_open.restype = i
    L.w4a8_gguf_close.argtypes = [p]
    L.w4a8_gguf_close.restype = None
    L.w4a8_gguf_version.argtypes = [p]
    L.w4a8_gguf_version.restype = ctypes.c_uint32
    for f in ("w4a8_gguf_n_tensors", "w4a8_gguf_n_kv"):
        getattr(L, f).argtypes = [p]
        getattr(L, f).restype = i64
    L.w4a8_gguf_data_offset.argtypes = [p]
    L.w4a8_gguf_data_offset.restype = u64
    for f in ("w4a8_gguf_find_key", "w4a8_gguf_find_tensor"):
        getattr(L, f).argtypes = [p, s]
        getattr(L, f).restype = i64
    L.w4a8_gguf_key.argtypes = [p, i64]
    L.w4a8_gguf_key.restype = s
    L.w4a8_gguf_kv_type.argtypes = [p, i64, ctypes.POINTER(ctypes.c_uint32), ctypes.POINTER(ctypes.c_uint32),
                                    ctypes.POINTER(u64)]
    L.w4a8_gguf_kv_type.restype = i
    for f, t in (("w4a8_gguf_get_u32", ctypes.c_uint32), ("w4a8_gguf_get_i32", ctypes.c_int32),
                 ("w4a8_gguf_get_u64", ctypes.c_uint64), ("w4a8_gguf_get_f32", ctypes.c_float)):
        getattr(L, f).argtypes = [p, s, ctypes.POINTER(t)]
        getattr(L, f).restype = i
    L.w4a8_gguf_get_str.argtypes = [p, s, ctypes.POINTER(p), ctypes.POINTER(u64)]
    L.w4a8_gguf_get_str.restype = i
    L.w4a8_gguf_tensor_info.argtypes = [p, i64, ctypes.POINTER(_Tensor)]
    L.w4a8_gguf_tensor_info.restype = i
    L.w4a8_gguf_tensor_data.argtypes = [p, i64]
    L.w4a8_gguf_tensor_data.restype = p
    L.w4a8_gguf_upload.argtypes = [p, i64, p, ctypes.c_size_t, p]
    L.w4a8_gguf_upload.restype = i
    _bound = True
    return L


class GGUFFile:
    """A parsed GGUF file (mapped read-only until close())."""

    def __init__(self, path: str):
        self._L = _bind()
        h = ctypes.c_void_p()
        st = self._L.w4a8_gguf_open(os.fsencode(str(path)), ctypes.byref(h))
        if st != 0:
            raise W4A8Error("w4a8_gguf_open", st)
        self._h = h

    def close(self) -> None:
        if self._h:
            self._L.w4a8_gguf_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    @property
    def version(self) -> int:
        return self._L.w4a8_gguf_version(self._h)

    @property
    def data_offset(self) -> int:
        return self._L.w4a8_gguf_data_offset(self._h)

    def keys(self) -> list:
        return [_text(self._L.w4a8_gguf_key(self._h, i)) for i in range(self._L.w4a8_gguf_n_kv(self._h))]

    def _scalar(self, fn, ctype, key):
        v = ctype()
        st = getattr(self._L, fn)(self._h, _raw(key), ctypes.byref(v))
        if st != 0:
            raise KeyError(key) if st == -2 else W4A8Error(fn, st)
        return v.value

    def u32(self, key: str) -> int:
        return self._scalar("w4a8_gguf_get_u32", ctypes.c_uint32, key)

    def i32(self, key: str) -> int:
        return self._scalar("w4a8_gguf_get_i32", ctypes.c_int32, key)

    def u64(self, key: str) -> int:
        return self._scalar("w4a8_gguf_get_u64", ctypes.c_uint64, key)

    def f32(self, key: str, default=None) -> float:
        try:
            return self._scalar("w4a8_gguf_get_f32", ctypes.c_float, key)
        except KeyError:
            if default is None:
                raise
            return default

    def string(self, key: str) -> str:
        ptr, n = ctypes.c_void_p(), ctypes.c_uint64()
        st = self._L.w4a8_gguf_get_str(self._h, _raw(key), ctypes.byref(ptr), ctypes.byref(n))
        if st != 0:
            raise KeyError(key) if st == -2 else W4A8Error("w4a8_gguf_get_str", st)
        return _text(ctypes.string_at(ptr.value, n.value))

    def kv_type(self, key: str) -> tuple:
        i = self._L.w4a8_gguf_find_key(self._h, _raw(key))
        if i < 0:
            raise KeyError(key)
        t, et, n = ctypes.c_uint32(), ctypes.c_uint32(), ctypes.c_uint64()
        self._L.w4a8_gguf_kv_type(self._h, i, ctypes.byref(t), ctypes.byref(et), ctypes.byref(n))
        return t.value, et.value, n.value

    def tensors(self) -> list:
        return [self._info(i) for i in range(self._L.w4a8_gguf_n_tensors(self._h))]

    def _index(self, name: str) -> int:
        i = self._L.w4a8_gguf_find_tensor(self._h, _raw(name))
        if i < 0:
            raise KeyError(f"tensor {name} missing")
        return i

    def _info(self, i: int) -> TensorInfo:
        t = _Tensor()
        st = self._L.w4a8_gguf_tensor_info(self._h, i, ctypes.byref(t))
        if st != 0:
            raise W4A8Error("w4a8_gguf_tensor_info", st)
        return TensorInfo(_text(t.name), t.type, tuple(t.ne[d] for d in range(t.n_dims)), t.offset, t.nbytes)

    def tensor(self, name: str) -> TensorInfo:
        return self._info(self._index(name))

    def tensor_bytes(self, name: str) -> bytes:
        """The tensor's bytes as they lie in the file (host)."""
        i = self._index(name)
        return ctypes.string_at(self._L.w4a8_gguf_tensor_data(self._h, i), self._info(i).nbytes)

    def upload(self, name: str, out=None):
        """Copy the tensor's bytes unchanged to the GPU: uint8 [rows, k/32*18] for
        Q4_0 (ne = [k, rows]), else a flat uint8 tensor of its bytes."""
        import torch
        i = self._index(name)
        info = self._info(i)
        if not info.nbytes:
            raise ValueError(f"tensor {name}: ggml type {info.type} is not one the engine reads")
        shape = (int(info.nbytes),)
        if info.type == GGML_TYPE_Q4_0 and len(info.ne) == 2:
            shape = (int(info.ne[1]), int(info.ne[0]) // 32 * 18)
        if out is None:
            out = torch.empty(shape, dtype=torch.uint8, device="cuda")
        if out.numel() < info.nbytes or not out.is_contiguous() or not out.is_cuda:
            raise ValueError("out must be a contiguous GPU tensor of at least the tensor's bytes")
        stream = torch.cuda.current_stream(out.device).cuda_stream
        st = self._L.w4a8_gguf_upload(self._h, i, out.data_ptr(), out.numel() * out.element_size(), stream)
        if st != 0:
            raise W4A8Error("w4a8_gguf_upload", st)
        return out
