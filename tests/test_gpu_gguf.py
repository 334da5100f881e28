"""GGUF weights on the GPU: a Q4_0 tensor uploaded from the file unchanged is
the weight matrix the GEMV reads in place (checked byte for byte against the
oracle on the same blocks), and the reference's caller loads a Llama-shaped
GGUF file the way load_model does (board/tp/tp_llama.cpp:226-287: q|k|v and
gate|up fused by row copies, token_embd as the LM head) and computes with it
through the reference ABI."""

from __future__ import annotations

import numpy as np
import pytest

import c_oracle as C
import q4_0_oracle as O
from gguf_writer import llama_gguf
from gpu_helpers import assert_bytes_equal, dev, host
from kv260gemv.gguf import GGUFFile
from test_gpu_caller import _check_call, _run

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def model(tmp_path_factory):
    path = tmp_path_factory.mktemp("gguf") / "llama-tiny.gguf"
    return path, llama_gguf(path)


def test_uploaded_tensor_is_the_gemv_weight(gpu, model):
    path, q4 = model
    with GGUFFile(path) as f:
        for name in ("blk.0.attn_q.weight", "blk.1.ffn_down.weight", "token_embd.weight"):
            info = f.tensor(name)
            k, rows = info.ne
            w = f.upload(name)
            assert tuple(w.shape) == (rows, k // 32 * 18)
            assert host(w).tobytes() == q4[name]
            x = O.normal_f32((1, k), 77)[0]
            y = host(gpu.gemv_q4_0_f32(w, k, dev(x)))
            xq, xd = C.quantize_q8_0(x)
            blocks = np.frombuffer(q4[name], dtype=np.uint8).reshape(rows, -1)
            assert_bytes_equal(y, C.gemv_q4_0(blocks, k, xq, xd), name)
        small = dev(np.zeros(10, dtype=np.uint8))
        with pytest.raises(ValueError):
            f.upload("blk.0.attn_q.weight", out=small)


@pytest.mark.parametrize("engine", ["gemv2", "v1"])
def test_caller_loads_gguf(gpu, model, tmp_path, engine):
    path, q4 = model
    out, dump = _run(tmp_path, "--gguf", str(path), "--tokens", "2", *(["--v1"] if engine == "v1" else []))
    assert out["layers"] == 2 and out["calls_per_token"] == 9
    qkv = b"".join(q4[f"blk.0.attn_{t}.weight"] for t in "qkv")
    assert (dump / "qkv.w.q4_0").read_bytes() == qkv
    assert (dump / "o.w.q4_0").read_bytes() == q4["blk.0.attn_output.weight"]
    assert (dump / "down.w.q4_0").read_bytes() == q4["blk.0.ffn_down.weight"]
    assert (dump / "lm_head.w.q4_0").read_bytes() == q4["token_embd.weight"]
    for name in ("qkv", "o", "down"):
        _check_call(dump, name)
    y = _check_call(dump, "lm_head")
    assert out["first_token_argmax"] == int(np.argmax(y))
