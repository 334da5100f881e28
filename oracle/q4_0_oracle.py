"""CPU oracle for the W4A8 (Q4_0 weights x Q8_0 activation) GEMV contract.

TEST INFRASTRUCTURE ONLY. This module is what the library is compared against, never the thing that is
measured or shipped: only `tests/`, `__graft_entry__.smoke()` and the
`cpu_baseline` leg of `bench.py` may import it. The product path (the HIP
library under `llm-kv260_amd/`) never calls into it and fails loudly when its
own extension is missing.

It restates, clean-room and in NumPy fixed-width arithmetic, the contract the
reference engine is held to (`src/llm_kv260/q4_0.py`). Each function cites the
reference lines whose behaviour it follows. Pinning (see `tests/test_oracle.py`):

* `quantize_q4_0 -> quantize_q8_0 -> gemv_q4_0` end to end: the reference-held
  golden SHA-256 `efa9eda8...29cc` (`tests/test_q4_0_contract.py:181-191`).
* `quantize_q8_0` rounding: known answers `tests/test_q4_0_contract.py:51-59`
  plus a brute-force scalar check against exact rational rounding around every
  tie, including the 0.49999997f case where `floor(|s| + 0.5f)` differs from a
  round-to-nearest of the exact quotient.
* `unpack_q4_0` nibble layout: known answer `tests/test_q4_0_contract.py:69-78`.
* `pack_x_for_engine`: known answer `tests/test_q4_0_contract.py:171-176`.
* `gemv_q4_0` order: closed form at nb == 8 (`tests/...:118-132`), the
  "sequential order gives different bits" negative test (`:135-158`), and a
  float64 dequantized-matmul tolerance check (`:102-115`).
* `tree_sum`: brute force against an explicit pairwise tree on 1..64 lanes.
* fp16 <-> fp32: exhaustive over all 65,536 half patterns (exact widening)
  and RNE narrowing checked against exact rational rounding.

The second restatement, `q4_0_oracle.c`, must agree with this one byte for
byte; the two were written independently of each other from the closed forms.
"""

from __future__ import annotations

import numpy as np

QK = 32              # weights per block (Q4_0 and Q8_0); q4_0.py:59
Q4_0_BYTES = 18      # f16 d + 16 nibble bytes; q4_0.py:60
Q8_0_BYTES = 34      # f16 d + 32 int8; q4_0.py:61
LANES = 8            # fp32 accumulation lanes; q4_0.py:62
CONTRACT_VERSION = "llm-kv260/w4a8-q4_0-v2"   # q4_0.py:64

_F32 = np.float32


def tree_sum(values: np.ndarray) -> np.ndarray:
    """Adjacent-pair binary tree over the last axis, no widening.

    Follows `src/llm_kv260/q4_0.py:67-78` (and `tree8`, hls/int4_core/gemv_core.h:85-89).
    """
    n = values.shape[-1]
    if n == 0 or n & (n - 1):
        raise ValueError(f"reduction length must be a power of two, got {n}")
    level = values
    while level.shape[-1] != 1:
        pairs = level.reshape(level.shape[:-1] + (level.shape[-1] // 2, 2))
        level = pairs[..., 0] + pairs[..., 1]
    return level[..., 0]


def quantize_q8_0(x: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Q8_0 activation quantizer, `src/llm_kv260/q4_0.py:83-97`.

    Per 32-block: amax = max|x|; d = amax / 127 (fp32); inv = 0 if d == 0 else
    1 / d (fp32); s = x * inv; q = sign(s) * floor(|s| + 0.5) -> int8; d stored
    as fp16 with round-to-nearest-even. Returns (q int8[K], d float16[K/32]).
    """
    if x.dtype != np.float32:
        raise TypeError(f"activations must be float32, got {x.dtype}")
    if x.ndim != 1 or x.shape[0] % QK:
        raise ValueError(f"x must be 1-D with a multiple of {QK} elements, got {x.shape}")
    blk = x.reshape(-1, QK)
    amax = np.max(np.abs(blk), axis=1)
    d = amax / _F32(127.0)
    with np.errstate(divide="ignore"):
        inv = np.where(d == _F32(0.0), _F32(0.0), _F32(1.0) / d).astype(_F32)
    s = blk * inv[:, None]
    mag = np.floor(np.abs(s) + _F32(0.5))
    q = np.where(s < _F32(0.0), -mag, mag)
    return q.astype(np.int8).reshape(-1), d.astype(np.float16)


def quantize_q8_0_rows(x: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Row-by-row `quantize_q8_0` for an [M, K] activation batch."""
    if x.ndim != 2:
        raise ValueError(f"expected [M, K], got {x.shape}")
    out = [quantize_q8_0(row) for row in x]
    return np.stack([q for q, _ in out]), np.stack([d for _, d in out])


def quantize_q4_0(w: np.ndarray) -> np.ndarray:
    """Q4_0 weight quantizer, `src/llm_kv260/q4_0.py:100-121`.

    Per 32-block: the signed element of largest magnitude (first on ties) is the
    extreme; d = extreme / -8 (fp32); inv = 0 if d == 0 else 1 / d; nibble
    n = min(trunc(w * inv + 8.5), 15); byte j = n[j] | n[j + 16] << 4; the
    block is fp16(d) little-endian then the 16 bytes. Returns uint8[N, K/32*18].
    """
    if w.dtype != np.float32:
        raise TypeError(f"weights must be float32, got {w.dtype}")
    rows, k = w.shape
    if k % QK:
        raise ValueError(f"in_features must be a multiple of {QK}, got {k}")
    nb = k // QK
    blk = w.reshape(rows, nb, QK)
    pick = np.argmax(np.abs(blk), axis=2)
    extreme = np.take_along_axis(blk, pick[..., None], axis=2)[..., 0]
    d = (extreme / _F32(-8.0)).astype(_F32)
    with np.errstate(divide="ignore"):
        inv = np.where(d == _F32(0.0), _F32(0.0), _F32(1.0) / d).astype(_F32)
    v = blk * inv[..., None] + _F32(8.5)
    nib = np.minimum(np.trunc(v).astype(np.uint8), np.uint8(15))
    out = np.empty((rows, nb, Q4_0_BYTES), dtype=np.uint8)
    out[..., :2] = d.astype(np.float16)[..., None].view(np.uint8)
    out[..., 2:] = nib[..., :16] | (nib[..., 16:] << np.uint8(4))
    return out.reshape(rows, nb * Q4_0_BYTES)


def unpack_q4_0(blocks: np.ndarray, k: int) -> tuple[np.ndarray, np.ndarray]:
    """Block bytes -> (int8[N, K] in [-8, 7], float16 d[N, K/32]).

    Follows `src/llm_kv260/q4_0.py:126-140`: byte j holds weight j in its low
    nibble and weight j + 16 in its high nibble; nibble n means n - 8.
    """
    if blocks.dtype != np.uint8:
        raise TypeError(f"expected uint8 block bytes, got {blocks.dtype}")
    nb = k // QK
    rows = blocks.shape[0]
    if blocks.ndim != 2 or blocks.shape[1] != nb * Q4_0_BYTES:
        raise ValueError(f"{blocks.shape[1:]} bytes per row is not {nb} blocks of {Q4_0_BYTES}")
    b3 = blocks.reshape(rows, nb, Q4_0_BYTES)
    d = np.ascontiguousarray(b3[..., :2]).view(np.float16)[..., 0]
    qs = b3[..., 2:].astype(np.int16)
    ints = np.concatenate([(qs & 15) - 8, (qs >> 4) - 8], axis=2).astype(np.int8)
    return ints.reshape(rows, k), d


def dequantize_q4_0(blocks: np.ndarray, k: int) -> np.ndarray:
    """(n - 8) * fp32(d) expansion, `src/llm_kv260/q4_0.py:143-146`."""
    ints, d = unpack_q4_0(blocks, k)
    return ints.astype(_F32) * np.repeat(d.astype(_F32), QK, axis=1)


def block_dots(blocks: np.ndarray, k: int, xq: np.ndarray) -> np.ndarray:
    """Exact int32 in-block dot products sumi[N, nb] (step 1 of q4_0.py:170-171)."""
    ints, _ = unpack_q4_0(blocks, k)
    nb = k // QK
    w3 = ints.reshape(-1, nb, QK).astype(np.int32)
    x2 = xq.reshape(nb, QK).astype(np.int32)
    return np.einsum("nbj,bj->nb", w3, x2, dtype=np.int32)


def gemv_q4_0(blocks: np.ndarray, k: int, xq: np.ndarray, xd: np.ndarray) -> np.ndarray:
    """y = W x in the engine's order, `src/llm_kv260/q4_0.py:151-182`.

    t[n, b] = (fp32(sumi) * fp32(dw)) * fp32(dx); lane l accumulates t[n, 8c+l]
    for c = 0, 1, ... starting from +0.0; y = tree_sum(lanes). float32 [N].
    """
    if xq.dtype != np.int8 or xd.dtype != np.float16:
        raise TypeError(f"x must be (int8, float16), got ({xq.dtype}, {xd.dtype})")
    _, dw = unpack_q4_0(blocks, k)
    rows, nb = dw.shape
    if xq.shape != (k,) or xd.shape != (nb,):
        raise ValueError(f"x shapes {xq.shape}, {xd.shape} do not match K={k}")
    if nb % LANES:
        raise ValueError(f"{nb} blocks is not a multiple of {LANES} lanes")
    sumi = block_dots(blocks, k, xq)
    t = (sumi.astype(_F32) * dw.astype(_F32)) * xd.astype(_F32)[None, :]
    t = t.reshape(rows, nb // LANES, LANES)
    acc = np.zeros((rows, LANES), dtype=_F32)
    for c in range(nb // LANES):
        acc = acc + t[:, c, :]
    return tree_sum(acc)


def gemv_q4_0_f32(blocks: np.ndarray, k: int, x: np.ndarray) -> np.ndarray:
    """`quantize_q8_0` then `gemv_q4_0`, `src/llm_kv260/q4_0.py:185-188`."""
    xq, xd = quantize_q8_0(x)
    return gemv_q4_0(blocks, k, xq, xd)


def gemm_q4_0_rows(blocks: np.ndarray, k: int, xq: np.ndarray, xd: np.ndarray) -> np.ndarray:
    """M > 1: the contract applied row by row (q4_0.py's gemv takes 1-D x). float32 [M, N]."""
    return np.stack([gemv_q4_0(blocks, k, xq[m], xd[m]) for m in range(xq.shape[0])])


def pack_x_for_engine(xq: np.ndarray, xd: np.ndarray) -> np.ndarray:
    """Engine activation layout int8[K] then float32[K/32], `src/llm_kv260/q4_0.py:193-200`."""
    return np.concatenate([xq.view(np.uint8), xd.astype(_F32).view(np.uint8)])


def pack_q8_0_blocks(xq: np.ndarray, xd: np.ndarray) -> np.ndarray:
    """ggml's native Q8_0 blocks: fp16 d then 32 int8, 34 bytes per block."""
    nb = xd.shape[0]
    out = np.empty((nb, Q8_0_BYTES), dtype=np.uint8)
    out[:, :2] = xd.astype(np.float16)[:, None].view(np.uint8)
    out[:, 2:] = xq.reshape(nb, QK).view(np.uint8)
    return out.reshape(-1)


def normal_f32(shape, seed: int, scale: float | None = None) -> np.ndarray:
    """Seeded inputs: float64 standard normals (times `scale` in float64), then float32.

    The idiom of `tests/test_q4_0_contract.py:29-30` for scale None.
    """
    z = np.random.default_rng(seed).standard_normal(shape)
    if scale is not None:
        z *= scale
    return z.astype(_F32)
