"""Writes tests/golden/gen_vectors.json: the reference's own exactness cases,
hls/int4_core/gen_vectors.py:23-50, computed by the CPU oracle.

    python tests/golden/make_gen_vectors.py       # rewrites gen_vectors.json

The reference draws every case from ONE numpy.random.default_rng(4) stream, in
the order of its CASES list (gen_vectors.py:24-32): per case the weights
rng.standard_normal((rows, k)).astype(float32) -- unit scale, not the 0.02 of
the workload configurations -- then the activation
rng.standard_normal(k).astype(float32); quantize_q4_0, quantize_q8_0,
pack_x_for_engine, gemv_q4_0. Its board run (docs/buildlog/evidence/
0013-bench-gemv2.txt:1, bench_gemv2.c:47-90) adds one rank's shard shapes
given on the command line, which gen_vectors.py draws from a fresh
default_rng(4) stream of their own (gen_vectors.py:53-55). The vectors
directory is not committed in the reference (hls/int4_core/.gitignore:1), so
the cases are regenerated here and stored as SHA-256 digests of the bytes
w.bin, x.bin and y.bin would hold, with the first outputs' bits.
"""

from __future__ import annotations

import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))

import c_oracle as C          # noqa: E402
import q4_0_oracle as O       # noqa: E402

OUT = os.path.join(HERE, "gen_vectors.json")

# gen_vectors.py:24-32, in order.
CASES = [(256, 16), (2048, 64), (8192, 16), (256, 32), (8192, 32), (512, 64), (1024, 32)]
# The shard shapes of the board run (0013-bench-gemv2.txt:1), a stream of their own.
SHARD_CASES = [(512, 2048), (2048, 768), (2048, 2048), (2048, 4096)]


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def draw(cases):
    """(k, rows, Q4_0 rows, engine-layout x, y) per case, one default_rng(4) stream."""
    rng = np.random.default_rng(4)
    out = []
    for k, rows in cases:
        w = rng.standard_normal((rows, k)).astype(np.float32)
        x = rng.standard_normal(k).astype(np.float32)
        blocks = C.quantize_q4_0(w)
        xq, xd = C.quantize_q8_0(x)
        y = C.gemv_q4_0(blocks, k, xq, xd)
        out.append((k, rows, blocks, C.pack_x_for_engine(xq, xd), y, w, x))
    return out


def record(k, rows, blocks, x_eng, y, w, x, cross_check):
    if cross_check:
        assert np.array_equal(O.quantize_q4_0(w), blocks), (k, rows)
        q, d = O.quantize_q8_0(x)
        assert np.array_equal(O.pack_x_for_engine(q, d), x_eng), (k, rows)
        assert np.array_equal(O.gemv_q4_0(blocks, k, q, d).view(np.uint32), y.view(np.uint32)), (k, rows)
    return {"name": f"k{k}_n{rows}", "k": k, "rows": rows, "w": sha(blocks), "x": sha(x_eng), "y": sha(y),
            "y_head": [f"{int(v):08x}" for v in y[:4].view(np.uint32)]}


def build() -> dict:
    return {"source": "hls/int4_core/gen_vectors.py:23-50 (default_rng(4), unit-scale weights)",
            "hash": "sha256 of w.bin (Q4_0 rows), x.bin (int8[k] then float32[k/32]), y.bin (float32[rows])",
            "cases": [record(*c, cross_check=True) for c in draw(CASES)],
            "shard_cases": [record(*c, cross_check=c[1] <= 2048) for c in draw(SHARD_CASES)]}


if __name__ == "__main__":
    data = build()
    with open(OUT, "w") as f:
        json.dump(data, f, indent=1)
        f.write("\n")
    print(f"wrote {OUT}")
