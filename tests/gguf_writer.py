"""A GGUF v2/v3 writer for the tests, from ggml's published GGUF format: magic
"GGUF", u32 version, u64 tensor count, u64 key/value count, key/value pairs
(u64-length string key, u32 type, value), tensor infos (name, u32 n_dims,
u64 ne[n_dims], u32 ggml type, u64 offset from the data section), then the
data section at the next multiple of general.alignment (default 32), each
tensor's data at an aligned offset. Test infrastructure only."""

from __future__ import annotations

import struct

UINT8, INT8, UINT16, INT16, UINT32, INT32, FLOAT32, BOOL, STRING, ARRAY, UINT64, INT64, FLOAT64 = range(13)
_FMT = {UINT8: "<B", INT8: "<b", UINT16: "<H", INT16: "<h", UINT32: "<I", INT32: "<i", FLOAT32: "<f",
        BOOL: "<?", UINT64: "<Q", INT64: "<q", FLOAT64: "<d"}


def _str(s) -> bytes:
    b = s.encode() if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def _value(t, v) -> bytes:
    if t in _FMT:
        return struct.pack(_FMT[t], v)
    if t == STRING:
        return _str(v)
    if t == ARRAY:
        et, items = v
        return struct.pack("<IQ", et, len(items)) + b"".join(_value(et, x) for x in items)
    raise ValueError(t)


def gguf_bytes(kvs, tensors, alignment=32, version=3) -> bytes:
    """kvs: [(key, type, value)], tensors: [(name, ggml_type, ne, data_bytes)]."""
    head = b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(kvs))
    for key, t, v in kvs:
        head += _str(key) + struct.pack("<I", t) + _value(t, v)
    offsets, off = [], 0
    for _, _, _, data in tensors:
        off = (off + alignment - 1) // alignment * alignment
        offsets.append(off)
        off += len(data)
    for (name, gt, ne, _), o in zip(tensors, offsets):
        head += _str(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", n) for n in ne)
        head += struct.pack("<IQ", gt, o)
    data_start = (len(head) + alignment - 1) // alignment * alignment
    out = bytearray(head + b"\0" * (data_start - len(head)))
    for (_, _, _, data), o in zip(tensors, offsets):
        out += b"\0" * (data_start + o - len(out))
        out += data
    return bytes(out), data_start, offsets


def llama_gguf(path, n_layer=2, n_embd=512, n_ff=1024, n_head=8, n_head_kv=2, n_vocab=1024, seed=0):
    """A Llama-shaped GGUF file with seeded N(0, 0.02) Q4_0 weights (quantized by
    the oracle) under llama.cpp's tensor names; returns {name: Q4_0 bytes}."""
    import c_oracle as C
    import numpy as np
    import q4_0_oracle as O

    kv_rows = n_head_kv * (n_embd // n_head)
    kvs = [("general.architecture", STRING, "llama"), ("general.alignment", UINT32, 32),
           ("llama.block_count", UINT32, n_layer), ("llama.embedding_length", UINT32, n_embd),
           ("llama.feed_forward_length", UINT32, n_ff), ("llama.attention.head_count", UINT32, n_head),
           ("llama.attention.head_count_kv", UINT32, n_head_kv), ("llama.vocab_size", UINT32, n_vocab),
           ("llama.rope.freq_base", FLOAT32, 500000.0),
           ("llama.attention.layer_norm_rms_epsilon", FLOAT32, 1e-5)]
    tensors, q4 = [], {}
    s = seed

    def q4_0(name, rows, k):
        nonlocal s
        b = C.quantize_q4_0(O.normal_f32((rows, k), 500 + s, 0.02))
        s += 1
        q4[name] = b.tobytes()
        tensors.append((name, 2, (k, rows), q4[name]))

    def f32(name, n):
        tensors.append((name, 0, (n,), np.ones(n, dtype=np.float32).tobytes()))

    q4_0("token_embd.weight", n_vocab, n_embd)
    for l in range(n_layer):
        f32(f"blk.{l}.attn_norm.weight", n_embd)
        q4_0(f"blk.{l}.attn_q.weight", n_embd, n_embd)
        q4_0(f"blk.{l}.attn_k.weight", kv_rows, n_embd)
        q4_0(f"blk.{l}.attn_v.weight", kv_rows, n_embd)
        q4_0(f"blk.{l}.attn_output.weight", n_embd, n_embd)
        f32(f"blk.{l}.ffn_norm.weight", n_embd)
        q4_0(f"blk.{l}.ffn_gate.weight", n_ff, n_embd)
        q4_0(f"blk.{l}.ffn_up.weight", n_ff, n_embd)
        q4_0(f"blk.{l}.ffn_down.weight", n_embd, n_ff)
    f32("output_norm.weight", n_embd)
    blob, _, _ = gguf_bytes(kvs, tensors)
    with open(path, "wb") as fh:
        fh.write(blob)
    return q4
