"""Pins the CPU oracle before anything is checked against it.

Every check here is independent of the oracle's own formulas: the
reference-held golden digest, the reference's known answers, values fixed by
the arithmetic of the contract (worked out by hand below), NumPy's own fp16
conversion, brute force in Python integers, and agreement between the two
independently written restatements (NumPy and C).
"""

from __future__ import annotations

import hashlib
import struct

import numpy as np
import pytest

import c_oracle as C
import q4_0_oracle as O

GOLDEN_SHA256 = "efa9eda8cef689d6392ddf2e1b3e945d19797aff1cbd55398c87ffffec7c29cc"  # tests/test_q4_0_contract.py:181


def _golden_inputs():
    # tests/test_q4_0_contract.py:184-189: w = _weights(96, 2048, 2024), x = _weights(1, 2048, 2025)[0]
    return O.normal_f32((96, 2048), 2024), O.normal_f32((1, 2048), 2025)[0]


# ------------------------------------------------------------------ golden

def test_golden_numpy_oracle():
    w, x = _golden_inputs()
    y = O.gemv_q4_0_f32(O.quantize_q4_0(w), 2048, x)
    assert hashlib.sha256(y.tobytes()).hexdigest() == GOLDEN_SHA256


def test_golden_c_oracle():
    w, x = _golden_inputs()
    xq, xd = C.quantize_q8_0(x)
    y = C.gemv_q4_0(C.quantize_q4_0(w), 2048, xq, xd)
    assert hashlib.sha256(y.tobytes()).hexdigest() == GOLDEN_SHA256


def test_golden_is_sensitive_to_a_planted_mistake():
    """A sequential (one-accumulator) order must not reproduce the digest."""
    w, x = _golden_inputs()
    blocks = O.quantize_q4_0(w)
    xq, xd = O.quantize_q8_0(x)
    _, dw = O.unpack_q4_0(blocks, 2048)
    t = (O.block_dots(blocks, 2048, xq).astype(np.float32) * dw.astype(np.float32)) * xd.astype(np.float32)
    seq = np.zeros(96, np.float32)
    for b in range(64):
        seq = seq + t[:, b]
    assert hashlib.sha256(seq.tobytes()).hexdigest() != GOLDEN_SHA256


# ------------------------------------------------------------ known answers

@pytest.mark.parametrize("impl", [O, C], ids=["numpy", "c"])
def test_q8_0_rounds_half_away_from_zero(impl):
    # tests/test_q4_0_contract.py:51-59
    x = np.zeros(32, np.float32)
    x[:4] = [127.0, 2.5, -2.5, 0.5]
    q, d = impl.quantize_q8_0(x)
    assert q[:4].tolist() == [127, 3, -3, 1]
    assert d[0] == np.float16(1.0)


@pytest.mark.parametrize("impl", [O, C], ids=["numpy", "c"])
def test_q8_0_floor_of_half_plus_fp32_sum(impl):
    """0.49999997f = 0.5 - 2^-25. In fp32, |s| + 0.5 = 1 - 2^-25 is a tie between
    1 - 2^-24 and 1.0 and rounds to even (1.0), so floor gives 1. A roundf of the
    quotient (the reference runtime's NEON vcvta) would give 0. The contract
    (q4_0.py:96) is the fp32 floor form."""
    x = np.zeros(32, np.float32)
    x[0] = 127.0
    x[1] = np.float32(0.49999997)
    x[2] = -np.float32(0.49999997)
    x[3] = np.float32(0.49999994)   # 0.5 - 2^-24: |s| + 0.5 = 1 - 2^-24 exactly, floor 0
    assert struct.pack("<f", x[1]) == struct.pack("<I", 0x3EFFFFFF)
    q, _ = impl.quantize_q8_0(x)
    assert q[1:4].tolist() == [1, -1, 0]


@pytest.mark.parametrize("impl", [O, C], ids=["numpy", "c"])
def test_q8_0_scale_uses_fp32_reciprocal(impl):
    """With amax = 1: d = fp32(1/127), inv = fp32(1/d), s = fp32(x * inv),
    q = floor(fp32(|s| + 0.5)). Expected values come from exact rational
    arithmetic with one fp32 rounding per operation (a product or sum of two
    fp32 values is exact in a double, so float32(float(exact)) rounds once)."""
    from fractions import Fraction as F
    x = np.zeros(32, np.float32)
    x[0] = 1.0
    x[1:] = (np.arange(1, 32) / 127.0 + 0.5 / 127.0).astype(np.float32)   # near the .5 boundaries
    q, d = impl.quantize_q8_0(x)
    d32 = np.float32(F(1, 127))
    inv = np.float32(F(1) / F(float(d32)))
    for j in range(1, 32):
        s32 = np.float32(float(F(float(x[j])) * F(float(inv))))
        t32 = np.float32(float(F(float(s32)) + F(1, 2)))
        assert q[j] == int(np.floor(t32))
    assert d[0] == np.float16(d32)


@pytest.mark.parametrize("impl", [O, C], ids=["numpy", "c"])
def test_q4_0_first_index_extreme_and_clip(impl):
    """w[3] = +1 and w[7] = -1 tie for largest magnitude; the first (index 3)
    is the extreme, so d = 1 / -8 = -0.125 and inv = -8: w[3] -> trunc(-8 + 8.5) = 0,
    w[7] -> trunc(8 + 8.5) = 16 -> clipped to 15, zeros -> trunc(8.5) = 8,
    w[5] = 0.3 -> trunc(-2.4 + 8.5) = 6."""
    w = np.zeros((1, 32), np.float32)
    w[0, 3], w[0, 7], w[0, 5] = 1.0, -1.0, 0.3
    blk = impl.quantize_q4_0(w)[0]
    assert blk[:2].view(np.float16)[0] == np.float16(-0.125)
    nib = np.concatenate([blk[2:] & 15, blk[2:] >> 4])
    assert nib[3] == 0 and nib[7] == 15 and nib[5] == 6 and nib[0] == 8 and nib[31] == 8


@pytest.mark.parametrize("impl", [O, C], ids=["numpy", "c"])
def test_q4_0_round_trips_grid_values(impl):
    """Weights already on the grid (n - 8) * d with some element at -8 * d come back exactly."""
    rng = np.random.default_rng(3)
    n = rng.integers(0, 16, size=(4, 64))
    n[:, ::32] = 0                                   # the extreme of each block sits at nibble 0
    d = np.float32(0.0625)
    w = ((n - 8) * d).astype(np.float32)
    blk = impl.quantize_q4_0(w)
    back = O.dequantize_q4_0(blk, 64)
    assert np.array_equal(back, w)


def test_q4_0_all_zero_block_sign_of_scale():
    """All zeros: the extreme is +0, d = +0 / -8 = -0 (fp16 0x8000), every nibble 8."""
    for impl in (O, C):
        blk = impl.quantize_q4_0(np.zeros((1, 32), np.float32))[0]
        assert blk[0] == 0x00 and blk[1] == 0x80
        assert np.all(blk[2:] == 0x88)


def test_nibble_layout_is_low_then_high_half_block():
    # tests/test_q4_0_contract.py:69-78
    row = np.zeros((1, 18), np.uint8)
    row[0, :2] = np.array([1.0], np.float16).view(np.uint8)
    row[0, 2] = 0x0F
    row[0, 3] = 0x08 | (0x09 << 4)
    ints, d = O.unpack_q4_0(row, 32)
    assert d[0, 0] == np.float16(1.0)
    assert ints[0, 0] == 7 and ints[0, 16] == -8 and ints[0, 1] == 0 and ints[0, 17] == 1


def test_engine_x_layout():
    # tests/test_q4_0_contract.py:171-176
    xq, xd = O.quantize_q8_0(O.normal_f32((1, 64), 15)[0])
    packed = O.pack_x_for_engine(xq, xd)
    assert packed.dtype == np.uint8 and packed.shape == (64 + 2 * 4,)
    assert np.array_equal(packed[:64].view(np.int8), xq)
    assert np.array_equal(packed[64:].view(np.float32), xd.astype(np.float32))
    assert np.array_equal(C.pack_x_for_engine(xq, xd), packed)


def test_codec_rejects_wrong_inputs():
    # tests/test_q4_0_contract.py:89-97, 161-168
    with pytest.raises(TypeError):
        O.quantize_q4_0(np.zeros((2, 32), np.float64))
    with pytest.raises(TypeError):
        O.quantize_q8_0(np.zeros(32, np.float64))
    with pytest.raises(ValueError):
        O.quantize_q8_0(np.zeros(33, np.float32))
    with pytest.raises(ValueError):
        O.unpack_q4_0(np.zeros((1, 17), np.uint8), 32)
    blocks = O.quantize_q4_0(O.normal_f32((2, 256), 11))
    xq, xd = O.quantize_q8_0(O.normal_f32((1, 256), 12)[0])
    assert O.gemv_q4_0(blocks, 256, xq, xd).dtype == np.float32
    with pytest.raises(TypeError):
        O.gemv_q4_0(blocks, 256, xq.astype(np.int32), xd)
    with pytest.raises(ValueError):   # nb = 4 is not a multiple of 8 lanes
        O.gemv_q4_0(O.quantize_q4_0(O.normal_f32((2, 128), 13)), 128,
                    *O.quantize_q8_0(O.normal_f32((1, 128), 14)[0]))


# -------------------------------------------------------------------- gemv

def test_gemv_exact_when_each_lane_holds_one_block():
    # tests/test_q4_0_contract.py:118-132: nb == 8, so the tree is the whole reduction
    k = 256
    w, x = O.normal_f32((4, k), 7), O.normal_f32((1, k), 8)[0]
    blocks = O.quantize_q4_0(w)
    xq, xd = O.quantize_q8_0(x)
    ints, dw = O.unpack_q4_0(blocks, k)
    sumi = np.array([[sum(int(a) * int(b) for a, b in zip(ints[n, 32 * j:32 * j + 32], xq[32 * j:32 * j + 32]))
                      for j in range(8)] for n in range(4)], dtype=np.int64)
    t = (sumi.astype(np.float32) * dw.astype(np.float32)) * xd.astype(np.float32)
    want = ((t[:, 0] + t[:, 1]) + (t[:, 2] + t[:, 3])) + ((t[:, 4] + t[:, 5]) + (t[:, 6] + t[:, 7]))
    assert np.array_equal(O.gemv_q4_0(blocks, k, xq, xd), want)
    assert np.array_equal(C.gemv_q4_0(blocks, k, xq, xd), want)


def test_lane_accumulation_order_by_construction():
    """nb = 16, so lane 0 accumulates blocks 0 then 8 and lane 1 holds block 1.
    Blocks chosen so t0 = 2^24, t1 = -2^24, t8 = 1, every other t = 0:
    lane0 = (0 + 2^24) + 1 = 2^24 (the tie rounds to even), lane1 = -2^24, y = 0.
    One accumulator over all blocks in order would give (2^24 - 2^24) + 1 = 1."""
    k, nb = 512, 16
    nib = np.full((nb, 32), 8, np.int64)             # weight 0 everywhere ...
    nib[0, 0], nib[1, 0], nib[8, 0] = 8 + 4, 8 - 4, 8 + 1
    dw = np.ones(nb, np.float16)
    dw[0] = dw[1] = 2048.0
    blocks = np.empty((nb, 18), np.uint8)
    blocks[:, :2] = dw[:, None].view(np.uint8).reshape(nb, 2)
    blocks[:, 2:] = (nib[:, :16] | (nib[:, 16:] << 4)).astype(np.uint8)
    blocks = blocks.reshape(1, -1)
    xq = np.zeros(k, np.int8)
    xq[::32] = 1                                     # ... times x = 1 at each block's first element
    xd = np.ones(nb, np.float16)
    xd[0] = xd[1] = 2048.0                           # t0 = 4 * 2048 * 2048 = 2^24
    for impl in (O, C):
        y = impl.gemv_q4_0(blocks, k, xq, xd)
        assert y[0] == np.float32(0.0)
    seq = np.float32(0)
    for t in [2.0 ** 24, -(2.0 ** 24)] + [0.0] * 6 + [1.0]:
        seq = seq + np.float32(t)
    assert seq == np.float32(1.0)


def test_lane_order_is_observable():
    # tests/test_q4_0_contract.py:135-158
    k = 2048
    w, x = O.normal_f32((256, k), 9), O.normal_f32((1, k), 10)[0]
    blocks = O.quantize_q4_0(w)
    xq, xd = O.quantize_q8_0(x)
    ours = O.gemv_q4_0(blocks, k, xq, xd)
    _, dw = O.unpack_q4_0(blocks, k)
    t = (O.block_dots(blocks, k, xq).astype(np.float32) * dw.astype(np.float32)) * xd.astype(np.float32)
    seq = np.zeros(256, np.float32)
    for b in range(64):
        seq = seq + t[:, b]
    assert np.count_nonzero(ours.view(np.uint32) != seq.view(np.uint32)) > 0
    np.testing.assert_allclose(ours, seq, rtol=1e-4, atol=1e-3)


def test_gemv_agrees_with_dequantized_matmul():
    # tests/test_q4_0_contract.py:102-115
    w, x = O.normal_f32((64, 2048), 5), O.normal_f32((1, 2048), 6)[0]
    blocks = O.quantize_q4_0(w)
    xq, xd = O.quantize_q8_0(x)
    y = O.gemv_q4_0(blocks, 2048, xq, xd)
    x_deq = xq.astype(np.float32) * np.repeat(xd.astype(np.float32), 32)
    ref = O.dequantize_q4_0(blocks, 2048).astype(np.float64) @ x_deq.astype(np.float64)
    np.testing.assert_allclose(y, ref, rtol=1e-4, atol=1e-3)


def test_block_dots_brute_force():
    w, x = O.normal_f32((3, 256), 21, 0.02), O.normal_f32((1, 256), 22)[0]
    blocks = O.quantize_q4_0(w)
    xq, _ = O.quantize_q8_0(x)
    got = O.block_dots(blocks, 256, xq)
    raw = blocks.reshape(3, 8, 18)
    for n in range(3):
        for b in range(8):
            s = 0
            for j in range(16):
                byte = int(raw[n, b, 2 + j])
                s += ((byte & 15) - 8) * int(xq[32 * b + j]) + ((byte >> 4) - 8) * int(xq[32 * b + j + 16])
            assert got[n, b] == s


def test_tree_sum_brute_force():
    rng = np.random.default_rng(0)

    def pairwise(v):
        if len(v) == 1:
            return v[0]
        h = len(v) // 2
        # adjacent pairs first: recursion over the pair sums
        return pairwise([np.float32(v[2 * i] + v[2 * i + 1]) for i in range(h)])

    for n in (1, 2, 4, 8, 16, 64):
        v = (rng.standard_normal(n) * 10.0 ** rng.integers(-8, 8, n)).astype(np.float32)
        assert O.tree_sum(v) == pairwise(list(v))
    with pytest.raises(ValueError):
        O.tree_sum(np.zeros(6, np.float32))


# ------------------------------------------------------------------- fp16

def test_f16_to_f32_exhaustive():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = bits.view(np.float16).astype(np.float32)
    got = np.array([C.f16_to_f32(int(b)) for b in bits], np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_f32_to_f16_rne_sweep():
    rng = np.random.default_rng(5)
    cases = []
    for e in range(-30, 18):                          # every binade that maps into or near fp16
        base = np.float32(2.0 ** e).view(np.uint32)
        low = np.array([0, 1, 0xFFF, 0x1000, 0x1001, 0x1FFF, 0x2000, 0x3000, 0x7FFFFF,
                        0x400000, 0x7FF000, 0x7FE000], np.uint32)
        cases.append(base + low)
        cases.append(base + rng.integers(0, 1 << 23, 256, dtype=np.uint32))
    cases.append(np.array([0x477FE000, 0x477FEFFF, 0x477FF000, 0x47800000, 0x7F800000,
                           0x33000000, 0x33000001, 0x32FFFFFF, 0x387FC000, 0x387FE000], np.uint32))
    u = np.concatenate(cases)
    u = np.concatenate([u, u | np.uint32(0x80000000)])
    f = u.view(np.float32)
    want = f.astype(np.float16).view(np.uint16)
    got = np.array([C.f32_to_f16_bits(float(v)) for v in f], np.uint16)
    assert np.array_equal(got, want)


# --------------------------------------------------- the two restatements

@pytest.mark.parametrize("rows,k,seed", [(16, 256, 0), (64, 2048, 1), (16, 8192, 2), (33, 512, 3),
                                         (7, 1024, 4), (100, 4096, 5)])
def test_numpy_and_c_oracles_agree(rows, k, seed):
    w = O.normal_f32((rows, k), seed, 0.02)
    x = O.normal_f32((1, k), seed + 100)[0]
    b_np = O.quantize_q4_0(w)
    b_c = C.quantize_q4_0(w)
    assert np.array_equal(b_np, b_c)
    q_np, d_np = O.quantize_q8_0(x)
    q_c, d_c = C.quantize_q8_0(x)
    assert np.array_equal(q_np, q_c) and np.array_equal(d_np.view(np.uint16), d_c.view(np.uint16))
    y_np = O.gemv_q4_0(b_np, k, q_np, d_np)
    y_c = C.gemv_q4_0(b_np, k, q_np, d_np)
    assert np.array_equal(y_np.view(np.uint32), y_c.view(np.uint32))


def test_gemm_rows_is_gemv_per_row():
    k, rows, m = 512, 48, 5
    blocks = O.quantize_q4_0(O.normal_f32((rows, k), 8, 0.02))
    xq, xd = O.quantize_q8_0_rows(O.normal_f32((m, k), 9))
    y = C.gemm_q4_0_rows(blocks, k, xq, xd)
    for i in range(m):
        assert np.array_equal(y[i], O.gemv_q4_0(blocks, k, xq[i], xd[i]))


def test_contract_version():
    assert O.CONTRACT_VERSION == C.contract_version() == "llm-kv260/w4a8-q4_0-v2"
