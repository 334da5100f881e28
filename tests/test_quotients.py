"""The two division-free quotients the kernels use, checked exhaustively over the
ranges they are used in (CPU only; the GPU parity tests run the kernels
themselves at odd divisors, k = 2304 among them).

- small_div / div_mul (csrc/gemv_mt.hip): n / d = high 32 bits of n * m with
  m = floor(2^32 / d) + 1, for 0 <= n < 2^16 and 2 <= d <= 256 (staging index
  over blocks per row, lane over chunks per row or lanes per token).
- lane_quot (csrc/gemv_tile.h): n / d = trunc((n + 0.5) * rcp(d)) in fp32, for
  0 <= n < 64 and 1 <= d <= 64, with rcp any value within one ulp of 1 / d
  (v_rcp_f32's error bound).
"""
import numpy as np


def test_multiply_high_quotient_exact():
    n = np.arange(1 << 16, dtype=np.uint64)
    for d in range(2, 257):
        m = np.uint64((1 << 32) // d + 1)
        assert m < (1 << 32)
        q = (n * m) >> np.uint64(32)
        assert np.array_equal(q, n // np.uint64(d)), d


def test_reciprocal_quotient_exact_within_one_ulp():
    n = np.arange(64, dtype=np.float32)
    want_n = np.arange(64)
    for d in range(1, 65):
        r = np.float32(1.0) / np.float32(d)
        for rc in (np.nextafter(r, np.float32(0.0)), r, np.nextafter(r, np.float32(2.0))):
            p = (n + np.float32(0.5)) * np.float32(rc)          # fp32 add and multiply, each rounded
            assert p.dtype == np.float32
            assert np.array_equal(p.astype(np.int64), want_n // d), (d, rc)


def test_reciprocal_quotient_fails_without_the_half():
    """The + 0.5 is what makes it exact: without it a rounded-down reciprocal
    puts exact multiples one below (9 * rcp(9) < 1)."""
    bad = 0
    for d in range(1, 65):
        r = np.nextafter(np.float32(1.0) / np.float32(d), np.float32(0.0))
        n = np.arange(64, dtype=np.float32)
        bad += int(np.count_nonzero((n * r).astype(np.int64) != np.arange(64) // d))
    assert bad > 0
