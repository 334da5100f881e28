"""The engine's workloads: Llama-3.2-1B GEMV shapes and their seeded inputs.

Every matrix is fp32 N(0, 0.02) weights quantized to Q4_0 per 32-element
block, every activation fp32 N(0, 1) quantized to Q8_0. Inputs are drawn as
the reference's tests draw them (tests/test_q4_0_contract.py:29-30): float64
standard normals from numpy's default_rng(seed), scaled in float64, then cast
to float32. The shapes are the ones board/tp/tp_llama.cpp:226-287 builds for
one board holding the whole model (nranks = 1): fused q|k|v (32 query heads +
8 key/value heads of 64), o, fused gate|up, down, and the LM head tied to the
token embedding.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

HIDDEN = 2048
FFN = 8192
N_LAYERS = 16
VOCAB = 128256
QKV_ROWS = HIDDEN + 2 * 8 * 64          # 3072
W_SCALE = 0.02


@dataclass(frozen=True)
class Matrix:
    name: str
    rows: int
    k: int
    w_seed: int
    x_seed: int

    @property
    def weight_bytes(self) -> int:
        return self.rows * self.k // 32 * 18

    @property
    def algorithmic_bytes(self) -> int:
        """Weights + engine-layout activation (int8[K] + f32[K/32]) + f32 output."""
        return self.weight_bytes + self.k + self.k // 8 + 4 * self.rows


def normal_f32(shape, seed: int, scale: float | None = None) -> np.ndarray:
    z = np.random.default_rng(seed).standard_normal(shape)
    if scale is not None:
        z *= scale          # in place: the same float64 products as z * scale
    return z.astype(np.float32)


def weights(m: Matrix) -> np.ndarray:
    return normal_f32((m.rows, m.k), m.w_seed, W_SCALE)


def weight_chunks(m: Matrix, rows_per_chunk: int = 4096):
    """The rows of weights(m) in consecutive chunks: (first_row, float32 [r, K]).

    The generator's stream continues across calls, so the chunks concatenate
    to exactly weights(m); one float64 buffer is reused, so large matrices
    (the 128256-row LM head) never hold more than a chunk in memory."""
    rng = np.random.default_rng(m.w_seed)
    buf = np.empty((rows_per_chunk, m.k), np.float64)
    for r0 in range(0, m.rows, rows_per_chunk):
        r = min(rows_per_chunk, m.rows - r0)
        z = buf[:r]
        rng.standard_normal(out=z)
        z *= W_SCALE
        yield r0, z.astype(np.float32)


def activation(m: Matrix) -> np.ndarray:
    return normal_f32(m.k, m.x_seed)


# Single GEMV, o_proj shape, seeds 0 / 1.
O_PROJ = Matrix("o", HIDDEN, HIDDEN, 0, 1)

# The per-layer shapes, weight seed 10 + j, activation seed 20 + j.
LAYER_SHAPES = (
    Matrix("qkv", QKV_ROWS, HIDDEN, 10, 20),
    Matrix("o", HIDDEN, HIDDEN, 11, 21),
    Matrix("gate_up", 2 * FFN, HIDDEN, 12, 22),
    Matrix("down", HIDDEN, FFN, 13, 23),
)

# LM head, seeds 30 / 31 (147,750,912 bytes of Q4_0).
LM_HEAD = Matrix("lm_head", VOCAB, HIDDEN, 30, 31)
LM_HEAD_COPIES = 3   # 3 x 148 MB rotate past the 256 MB Infinity Cache


def decode_chain() -> list[Matrix]:
    """One token's 65 GEMVs: 16 x (q|k|v, o, gate|up, down) + LM head.

    Weight seed 1000 + 4l + j, activation seed 2000 + 4l + j; LM head 1064 / 2064.
    """
    chain = []
    for layer in range(N_LAYERS):
        for j, base in enumerate(LAYER_SHAPES):
            chain.append(Matrix(f"l{layer}.{base.name}", base.rows, base.k, 1000 + 4 * layer + j,
                                2000 + 4 * layer + j))
    chain.append(Matrix("lm_head", VOCAB, HIDDEN, 1064, 2064))
    return chain


CHAIN_STEPS = 400
GEMM_M = (1, 2, 4, 8, 16, 24, 64)
GEMM_SHAPES = (LAYER_SHAPES[2], LAYER_SHAPES[3])   # gate+up 16384x2048, down 2048x8192


def gemm_activation(m_rows: int, k: int) -> np.ndarray:
    """M rows of fp32 N(0, 1), seed 40 + M."""
    return normal_f32((m_rows, k), 40 + m_rows)


# A prompt through the decode chain's matrices at once (the M > 1 path).
PREFILL_M = 24


def prefill_activation(index: int, m_rows: int, k: int) -> np.ndarray:
    """m_rows prompt rows for matrix `index` of decode_chain(): fp32 N(0, 1), seed 3000 + index."""
    return normal_f32((m_rows, k), 3000 + index)


def chain_weight_bytes() -> int:
    return sum(m.weight_bytes for m in decode_chain())


def chain_algorithmic_bytes() -> int:
    return sum(m.algorithmic_bytes for m in decode_chain())
