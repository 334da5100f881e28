"""Writes tests/golden/configs.json: SHA-256 digests of the five workload
configurations' inputs and outputs, computed by the CPU oracle.

    python tests/golden/make_fixtures.py            # rewrites configs.json

The oracle is pinned before it is trusted here (tests/test_oracle.py: the
reference-held golden digest, known answers, brute force). The two
restatements (NumPy and scalar C) must agree where both are affordable
(configurations 0, 1 and the M sweep). The C one alone covers the LM head and
the 65-matrix chain.

Inputs follow the reference tests' idiom (tests/test_q4_0_contract.py:29-30):
float64 standard normals from numpy.random.default_rng(seed), times 0.02 for
weights, then float32. Seeds:
  config 0  o 2048x2048: weights 0, activation 1
  config 1  q|k|v 3072x2048, o 2048x2048, gate|up 16384x2048, down 2048x8192:
            weights 10 + j, activations 20 + j
  config 2  LM head 128256x2048: weights 30, activation 31
  config 3  16 layers x (q|k|v, o, gate|up, down) + LM head: weights
            1000 + 4 l + j (LM head 1064), activations 2000 + 4 l + j (2064)
  config 4  gate|up and down of config 1 at M = 1, 2, 4, 8, 16, 24, 64
            activation rows: default_rng(40 + M).standard_normal((M, K))
  config3_prefill24
            config 3's weights, a 24-token prompt per matrix: activation rows
            default_rng(3000 + j).standard_normal((24, K)) for matrix j
"""

from __future__ import annotations

import hashlib
import json
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, os.path.join(ROOT, "llm-kv260_amd"))

import c_oracle as C          # noqa: E402
import q4_0_oracle as O       # noqa: E402
from kv260gemv import configs as cf   # noqa: E402  (shapes and seeds only; pure Python)

OUT = os.path.join(HERE, "configs.json")


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def head_hex(y: np.ndarray, n: int = 4) -> list[str]:
    return [f"{int(v):08x}" for v in np.ascontiguousarray(y).reshape(-1)[:n].view(np.uint32)]


def quantized_weights(m: cf.Matrix) -> np.ndarray:
    blocks = np.empty((m.rows, m.k // 32 * 18), np.uint8)
    for r0, w in cf.weight_chunks(m):
        blocks[r0:r0 + w.shape[0]] = C.quantize_q4_0(w)
    return blocks


def matrix_record(m: cf.Matrix, cross_check: bool, blocks: np.ndarray | None = None) -> dict:
    x = cf.activation(m)
    if blocks is None:
        blocks = quantized_weights(m)
    xq, xd = C.quantize_q8_0(x)
    y = C.gemv_q4_0(blocks, m.k, xq, xd)
    if cross_check:
        assert np.array_equal(O.quantize_q4_0(cf.weights(m)), blocks), m
        q2, d2 = O.quantize_q8_0(x)
        assert np.array_equal(q2, xq) and np.array_equal(d2.view(np.uint16), xd.view(np.uint16)), m
        assert np.array_equal(O.gemv_q4_0(blocks, m.k, xq, xd).view(np.uint32), y.view(np.uint32)), m
    return {"name": m.name, "rows": m.rows, "k": m.k, "w_seed": m.w_seed, "x_seed": m.x_seed,
            "q4_0": sha(blocks), "xq": sha(xq), "xd": sha(xd.view(np.uint16)),
            "y": sha(y), "y_head": head_hex(y), "argmax": int(np.argmax(y))}


def gemm_record(m: cf.Matrix, mrows: int, blocks: np.ndarray, cross_check: bool) -> dict:
    x = cf.gemm_activation(mrows, m.k)
    xq, xd = C.quantize_q8_0_rows(x)
    y = C.gemm_q4_0_rows(blocks, m.k, xq, xd)
    if cross_check:
        want = O.gemm_q4_0_rows(blocks, m.k, *O.quantize_q8_0_rows(x))
        assert np.array_equal(want.view(np.uint32), y.view(np.uint32)), (m, mrows)
    return {"name": m.name, "m": mrows, "rows": m.rows, "k": m.k, "x_seed": 40 + mrows,
            "xq": sha(xq), "y": sha(y), "y_head": head_hex(y)}


def prefill_record(index: int, m: cf.Matrix, blocks: np.ndarray, mrows: int) -> dict:
    x = cf.prefill_activation(index, mrows, m.k)
    xq, xd = C.quantize_q8_0_rows(x)
    y = C.gemm_q4_0_rows(blocks, m.k, xq, xd)
    return {"name": m.name, "m": mrows, "rows": m.rows, "k": m.k, "x_seed": 3000 + index,
            "xq": sha(xq), "y": sha(y), "y_head": head_hex(y)}


def build() -> dict:
    t0 = time.time()
    out = {"contract": O.CONTRACT_VERSION,
           "hash": "sha256 of the little-endian bytes: Q4_0 rows, int8 xq, fp16 xd bits, fp32 y"}
    out["config0"] = [matrix_record(cf.O_PROJ, True)]
    out["config1"] = [matrix_record(m, True) for m in cf.LAYER_SHAPES]
    print(f"configs 0-1 done ({time.time() - t0:.1f} s)", flush=True)
    out["config2"] = [matrix_record(cf.LM_HEAD, False)]
    print(f"config 2 done ({time.time() - t0:.1f} s)", flush=True)
    c3, p24 = [], []
    for j, m in enumerate(cf.decode_chain()):
        blocks = quantized_weights(m)
        c3.append(matrix_record(m, False, blocks))
        p24.append(prefill_record(j, m, blocks, cf.PREFILL_M))
    out["config3"] = c3
    out["config3_prefill24"] = p24
    print(f"config 3 done ({time.time() - t0:.1f} s)", flush=True)
    g4 = []
    for m in cf.GEMM_SHAPES:
        blocks = quantized_weights(m)
        for mrows in cf.GEMM_M:
            g4.append(gemm_record(m, mrows, blocks, cross_check=mrows <= 8))
    out["config4"] = g4
    print(f"config 4 done ({time.time() - t0:.1f} s)", flush=True)
    return out


if __name__ == "__main__":
    data = build()
    with open(OUT, "w") as f:
        json.dump(data, f, indent=1)
        f.write("\n")
    print(f"wrote {OUT}")
