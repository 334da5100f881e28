"""The two identities the M > 1 MFMA kernels rest on, checked exhaustively on the CPU
(the GPU parity tests run the kernels themselves against the oracle).

- The weight operand (csrc/gemm_rows.hip block_weights, csrc/gemm_mfma.hip): each nibble
  n moved to its byte's high half and its top bit flipped, (n << 4) ^ 0x80, read as a
  signed byte, is 16 (n - 8) -- for the low nibbles (shifted up) and the high ones (in
  place), in every byte of a dword, with no carry between bytes.
- The scale: with MFMA sums 16 sumi, the term's first product f32(16 sumi) * (d_w / 16)
  equals the contract's f32(sumi) * d_w bit for bit, for every fp16 scale (subnormal,
  infinite and NaN included) and every block sum a block can have (|sumi| <= 32 * 8 *
  128). The same check with a factor that is not a power of two fails.
"""
import numpy as np


def _operand(raw: np.ndarray, high: bool) -> np.ndarray:
    """The kernels' operand bytes of a dword of nibble pairs: the high nibbles in place,
    or the low ones shifted up by 4, masked to the high halves, top bits flipped."""
    up = 0 if high else 4
    return (((raw << np.uint32(up)) & np.uint32(0xF0F0F0F0)) ^ np.uint32(0x80808080)).astype(np.uint32)


def test_weight_operand_is_16_times_signed_nibble():
    # Every byte value in every byte position (the other bytes random), both halves.
    rng = np.random.default_rng(5)
    for pos in range(4):
        b = np.arange(256, dtype=np.uint32)
        other = rng.integers(0, 1 << 32, size=256, dtype=np.uint64).astype(np.uint32)
        raw = (other & ~np.uint32(0xFF << (8 * pos))) | (b << np.uint32(8 * pos))
        for high in (False, True):
            got = ((_operand(raw, high) >> np.uint32(8 * pos)) & np.uint32(0xFF)).astype(np.uint8).view(np.int8)
            n = (b >> np.uint32(4)) if high else (b & np.uint32(0xF))
            assert np.array_equal(got.astype(np.int32), 16 * (n.astype(np.int32) - 8)), (pos, high)
            # The other three bytes are their own nibbles' operands: no carry across bytes.
            for q in range(4):
                if q == pos:
                    continue
                oq = (raw >> np.uint32(8 * q)) & np.uint32(0xFF)
                nq = (oq >> np.uint32(4)) if high else (oq & np.uint32(0xF))
                gq = ((_operand(raw, high) >> np.uint32(8 * q)) & np.uint32(0xFF)).astype(np.uint8).view(np.int8)
                assert np.array_equal(gq.astype(np.int32), 16 * (nq.astype(np.int32) - 8)), (pos, q, high)


def test_signed_operand_dot_is_16_times_contract_sum():
    # The block sum through the operand equals 16 x the contract's sum((n - 8) x), for
    # random blocks and extreme ones (all nibbles 0 or 15, x = -128 .. 127 bounds).
    rng = np.random.default_rng(6)
    for case in range(200):
        if case == 0:
            nib, x = np.zeros(32, np.int32), np.full(32, -128, np.int32)
        elif case == 1:
            nib, x = np.full(32, 15, np.int32), np.full(32, 127, np.int32)
        else:
            nib = rng.integers(0, 16, 32).astype(np.int32)
            x = rng.integers(-128, 128, 32).astype(np.int32)
        op = ((nib << 4) ^ 0x80).astype(np.uint8).view(np.int8).astype(np.int64)
        assert int(np.dot(op, x)) == 16 * int(np.dot(nib - 8, x))


@np.errstate(invalid="ignore", over="ignore")
def test_scaled_product_equals_contract_product_for_every_fp16_scale():
    d16 = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16).view(np.float16)
    d = d16.astype(np.float32)                       # exact widening
    d_over_16 = d * np.float32(0.0625)               # the kernels' scale
    # Exact: no fp16 value divided by 16 is subnormal in fp32, and inf / NaN stay so.
    fin = np.isfinite(d)
    assert np.array_equal((d_over_16[fin] * np.float32(16)).view(np.uint32), d[fin].view(np.uint32))
    sums = np.concatenate([np.arange(-300, 301), [32768, -32768, 32767, -32767, 4095, -4097, 12345, -23456]])
    for s in sums.astype(np.int64):
        want = np.float32(s) * d                                       # the contract: f32(sumi) * d_w
        got = np.float32(16 * s) * d_over_16                           # the kernels: f32(16 sumi) * (d_w / 16)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), int(s)


@np.errstate(invalid="ignore", over="ignore")
def test_scaled_product_check_catches_a_wrong_scaling():
    # The same check with a factor that is not a power of two (sums 3 sumi, scale d_w / 3,
    # which fp32 rounds) fails: the identity rests on d_w / 16 being exact.
    d = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16).view(np.float16).astype(np.float32)
    fin = np.isfinite(d)
    s = np.int64(12345)
    want = (np.float32(s) * d)[fin]
    wrong = (np.float32(3 * s) * (d / np.float32(3)))[fin]
    assert not np.array_equal(wrong.view(np.uint32), want.view(np.uint32))
