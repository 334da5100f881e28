"""The reference's decode-side caller (board/tp/tp_llama.cpp engine_t and the
forward() call order), rebuilt against the reference driver headers only and
linked against the library (llm-kv260_amd/caller/engine_caller.cpp), run on
the GPU with both engines: gemv2 (chunk-interleaved port layout, fetch of the
next matrix after each MAC) and the v1 four quarters. The first token's calls
of layer 0 and the LM head are dumped and checked byte for byte against the
oracle applied to the same weights and activations: the caller quantizes on
the host with the contract's Q8_0, cleans x, invalidates y, starts, waits and
invalidates again, exactly as engine_t::gemv does (tp_llama.cpp:355-374)."""

from __future__ import annotations

import json
import os
import subprocess

import numpy as np
import pytest

import c_oracle as C
from gpu_helpers import assert_bytes_equal

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CALLER = os.path.join(ROOT, "llm-kv260_amd", "caller", "engine_caller")


def _run(tmp_path, *args):
    if not os.path.exists(CALLER):
        pytest.fail(f"{CALLER} is not built (make -C llm-kv260_amd)")
    dump = tmp_path / "dump"
    dump.mkdir()
    print(f"engine_caller {' '.join(args)}", flush=True)
    env = dict(os.environ, KV260GEMV_UDMABUF_SIZES="udmabuf0=1G")    # the caller's own pool, whatever ran before
    p = subprocess.run([CALLER, *args, "--dump", str(dump)], capture_output=True, text=True, timeout=180, env=env)
    assert p.returncode == 0, p.stderr[-2000:]
    return json.loads(p.stdout.strip().splitlines()[-1]), dump


def _check_call(dump, name):
    rows, k = (int(v) for v in (dump / f"{name}.shape").read_text().split())
    w = np.fromfile(dump / f"{name}.w.q4_0", dtype=np.uint8).reshape(rows, k // 32 * 18)
    x = np.fromfile(dump / f"{name}.x.f32", dtype=np.float32)
    y = np.fromfile(dump / f"{name}.y.f32", dtype=np.float32)
    xq, xd = C.quantize_q8_0(x)
    assert_bytes_equal(y, C.gemv_q4_0(w, k, xq, xd), f"caller {name}")
    return y


@pytest.mark.parametrize("engine", ["gemv2", "v1"])
def test_reference_caller_runs_unchanged(gpu, tmp_path, engine):
    args = ["--tokens", "2", "--layers", "2"] + (["--v1"] if engine == "v1" else [])
    out, dump = _run(tmp_path, *args)
    assert out["engine"] == ("gemv2" if engine == "gemv2" else "gemv_q4_0")
    assert out["calls_per_token"] == 9
    for name in ("qkv", "o", "down"):
        _check_call(dump, name)
    y = _check_call(dump, "lm_head")
    assert out["first_token_argmax"] == int(np.argmax(y))
