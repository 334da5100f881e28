"""The library's GGUF reader (include/w4a8_gguf.h) on the CPU: metadata of
every GGUF value type, tensor infos, data offsets and bytes, against files
written by the tests' own spec writer; malformed and truncated files are
refused with W4A8_ERR_FORMAT, never read past their end. The reference reads
the same surface through llama.cpp's gguf API (board/tp/tp_llama.cpp:149-188);
llama.cpp and gguf-py are not in this image, so agreement with them on
real model files is parity unpinned here, and the format is pinned by the
published specification the writer follows."""

from __future__ import annotations

import numpy as np
import pytest

import c_oracle as C
import q4_0_oracle as O
from gguf_writer import (ARRAY, BOOL, FLOAT32, FLOAT64, INT8, INT16, INT32, INT64, STRING, UINT8, UINT16,
                         UINT32, UINT64, gguf_bytes)
from kv260gemv import W4A8Error
from kv260gemv.gguf import GGML_TYPE_F16, GGML_TYPE_F32, GGML_TYPE_Q4_0, GGUFFile

KVS = [("general.architecture", STRING, "llama"),
       ("general.alignment", UINT32, 64),
       ("llama.block_count", UINT32, 2),
       ("llama.embedding_length", UINT32, 512),
       ("llama.rope.freq_base", FLOAT32, 500000.0),
       ("llama.attention.layer_norm_rms_epsilon", FLOAT32, 1e-5),
       ("test.u8", UINT8, 200), ("test.i8", INT8, -7), ("test.u16", UINT16, 65000), ("test.i16", INT16, -300),
       ("test.i32", INT32, -123456), ("test.bool", BOOL, True), ("test.u64", UINT64, 1 << 40),
       ("test.i64", INT64, -(1 << 40)), ("test.f64", FLOAT64, 0.25),
       ("tokenizer.ggml.tokens", ARRAY, (STRING, ["<s>", "</s>", "héllo"])),
       ("tokenizer.ggml.scores", ARRAY, (FLOAT32, [0.0, -1.5, 2.0])),
       ("test.nested", ARRAY, (ARRAY, [(INT32, [1, 2]), (INT32, [3])]))]


def _model(tmp_path, alignment=64, version=3):
    wq = C.quantize_q4_0(O.normal_f32((48, 512), 11, 0.02))
    emb = C.quantize_q4_0(O.normal_f32((100, 512), 12, 0.02))
    norm = O.normal_f32((512,), 13)
    f16 = np.arange(64, dtype=np.float16).reshape(4, 16)
    tensors = [("blk.0.attn_q.weight", GGML_TYPE_Q4_0, (512, 48), wq.tobytes()),
               ("blk.0.attn_norm.weight", GGML_TYPE_F32, (512,), norm.tobytes()),
               ("test.f16", GGML_TYPE_F16, (16, 4), f16.tobytes()),
               ("token_embd.weight", GGML_TYPE_Q4_0, (512, 100), emb.tobytes())]
    kvs = [kv for kv in KVS if kv[0] != "general.alignment" or alignment != 32]
    if alignment != 64:
        kvs = [(k, t, alignment if k == "general.alignment" else v) for k, t, v in kvs]
    blob, data_start, offsets = gguf_bytes(kvs, tensors, alignment=alignment, version=version)
    path = tmp_path / "model.gguf"
    path.write_bytes(blob)
    return path, blob, tensors, data_start, offsets, kvs


@pytest.mark.parametrize("alignment,version", [(64, 3), (32, 3), (256, 2)])
def test_metadata_and_tensors(tmp_path, alignment, version):
    path, blob, tensors, data_start, offsets, kvs = _model(tmp_path, alignment, version)
    with GGUFFile(path) as f:
        assert f.version == version
        assert f.data_offset == data_start
        assert f.keys() == [k for k, _, _ in kvs]
        assert f.string("general.architecture") == "llama"
        assert f.u32("llama.block_count") == 2
        assert f.f32("llama.rope.freq_base") == 500000.0
        assert f.f32("llama.attention.layer_norm_rms_epsilon") == np.float32(1e-5)
        assert f.f32("llama.missing", 10000.0) == 10000.0    # the reference's f32(key, default)
        assert f.i32("test.i32") == -123456
        assert f.u64("test.u64") == 1 << 40
        assert f.kv_type("tokenizer.ggml.tokens") == (ARRAY, STRING, 3)
        assert f.kv_type("test.nested") == (ARRAY, ARRAY, 2)
        assert f.kv_type("test.bool")[0] == BOOL
        with pytest.raises(KeyError):
            f.u32("llama.nope")
        with pytest.raises(W4A8Error):
            f.u32("llama.rope.freq_base")                      # a key of another type
        infos = f.tensors()
        assert [t.name for t in infos] == [t[0] for t in tensors]
        for info, (name, gt, ne, data), off in zip(infos, tensors, offsets):
            assert (info.type, info.ne, info.offset, info.nbytes) == (gt, ne, off, len(data))
            assert off % alignment == 0
            assert f.tensor_bytes(name) == data == blob[data_start + off:data_start + off + len(data)]
        with pytest.raises(KeyError):
            f.tensor("blk.9.attn_q.weight")


def test_malformed_files_are_refused(tmp_path):
    path, blob, *_ = _model(tmp_path)
    bad = tmp_path / "bad.gguf"

    def refused(data):
        bad.write_bytes(data)
        with pytest.raises(W4A8Error) as e:
            GGUFFile(bad)
        assert e.value.status == -6

    refused(b"GGUX" + blob[4:])                               # magic
    refused(blob[:4] + (1).to_bytes(4, "little") + blob[8:])  # GGUF v1 (u32 counts) is not read
    # every cut before the end of the last tensor's data
    for n in list(range(0, 200, 7)) + list(range(len(blob) - 300, len(blob), 13)):
        refused(blob[:n])
    # a tensor whose data would run past the end of the file
    kvs = [("general.alignment", UINT32, 32)]
    blob2, _, _ = gguf_bytes(kvs, [("t", GGML_TYPE_F32, (8,), b"\0" * 32)])
    refused(blob2[:-4])
    # alignment that is not a power of two
    blob3, _, _ = gguf_bytes([("general.alignment", UINT32, 48)], [], alignment=32)
    refused(blob3)
    # counts the file cannot hold: refused before anything is reserved for them
    huge = (1 << 62).to_bytes(8, "little")
    refused(blob[:8] + huge + blob[16:])                      # tensor count
    refused(blob[:16] + huge + blob[24:])                     # key/value count
    refused(blob[:8] + (len(blob) // 32 + 1).to_bytes(8, "little") + blob[16:])
    # a key or a tensor name twice (llama.cpp refuses both), a NUL inside a name
    t8 = ("t", GGML_TYPE_F32, (8,), b"\0" * 32)
    refused(gguf_bytes([("a.b", UINT32, 1), ("a.b", UINT32, 2)], [t8])[0])
    refused(gguf_bytes([("a.b", UINT32, 1)], [t8, t8])[0])
    refused(gguf_bytes([("a\0b", UINT32, 1)], [t8])[0])
    refused(gguf_bytes([("a.b", UINT32, 1)], [("t\0u", GGML_TYPE_F32, (8,), b"\0" * 32)])[0])


def test_mutated_files_open_or_are_refused(tmp_path):
    """Random byte flips, overwritten counts and lengths, and truncations of a valid
    file: every one either opens (and then reads within the file) or is refused with
    the format status; none crashes. (The same mutations, 20,000 of them, were also
    run through the reader built with AddressSanitizer: no invalid access.)"""
    path, blob, *_ = _model(tmp_path, 32, 3)
    rng = np.random.default_rng(2024)
    bad = tmp_path / "mutated.gguf"
    opened = refused = 0
    for _ in range(400):
        b = bytearray(blob)
        for _ in range(int(rng.integers(1, 8))):
            pos = int(rng.integers(0, len(b)))
            kind = int(rng.integers(0, 4))
            if kind == 0:
                b[pos] = int(rng.integers(0, 256))
            elif kind == 1:
                b[pos] ^= 1 << int(rng.integers(0, 8))
            elif kind == 2 and pos + 8 <= len(b):
                v = (1 << 64) - 1 if rng.integers(0, 4) == 0 else int(rng.integers(0, 1_000_000))
                b[pos:pos + 8] = v.to_bytes(8, "little")
            elif kind == 3:
                del b[max(pos, 24):]
        bad.write_bytes(bytes(b))
        try:
            with GGUFFile(bad) as f:
                f.keys()
                for info in f.tensors():
                    assert len(f.tensor_bytes(info.name)) == info.nbytes
                opened += 1
        except W4A8Error as e:
            assert e.status == -6
            refused += 1
    assert opened and refused


@pytest.mark.parametrize("gtype,ne0", [(GGML_TYPE_F32, (1 << 62) + 32), (GGML_TYPE_F16, (1 << 63) + 32),
                                       (GGML_TYPE_Q4_0, 1 << 63), (GGML_TYPE_F32, (1 << 61) + 64)])
def test_byte_count_overflow_is_refused(tmp_path, gtype, ne0):
    """A tensor whose element count fits 64 bits but whose byte count does not
    (2^62 + 32 float32 values are 2^64 + 128 bytes, 128 modulo 2^64) must not
    pass the range check with a wrapped-around size: the file is refused."""
    data = b"\0" * 256
    blob, *_ = gguf_bytes([("general.architecture", STRING, "llama")], [("big", gtype, (ne0,), data)])
    path = tmp_path / "big.gguf"
    path.write_bytes(blob)
    with pytest.raises(W4A8Error) as e:
        GGUFFile(path)
    assert e.value.status == -6
