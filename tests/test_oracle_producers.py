"""Pinning the oracle's restatement of the reference's activation producers
(board/tp/tp_llama.cpp): rmsnorm (:557-569) and silu_mul with ggml's vector
expf (:530-553, :612-619). The reference holds no test vectors for them and
its NEON code does not build here, so they are pinned by what the
mathematics fixes and by a second restatement:

rmsnorm: a NumPy restatement (sequential float64 accumulation per lane) must
agree bit for bit; closed forms; and three constructed inputs around a
float32 rounding midpoint, each of which a plausible mistake in the order of
the float64 sum gets wrong (one lane instead of four; an exact or pairwise
sum; the lanes met as ((l0+l1)+l2)+l3 instead of (l0+l2)+(l1+l3)).

expf / silu: a pure-Python restatement of the same algorithm with exact fused
multiply-adds (fractions) must agree bit for bit, including the |n| > 126
and |n| > 192 scaling branches; the result stays within the routine's
published bound (1.45 + 0.5 ulp) of exp in float64 over the float32 range;
exp(0) = 1 and the overflow / underflow ends."""

from __future__ import annotations

import math
from fractions import Fraction

import numpy as np
import pytest

import c_oracle as C

F32 = np.float32


# ---------------------------------------------------------------- rmsnorm

def rmsnorm_numpy(x, w, eps):
    x = np.asarray(x, dtype=np.float32)
    sq = x.astype(np.float64) ** 2                    # exact: float32 products fit float64
    lanes = [np.add.accumulate(sq[r::4])[-1] for r in range(4)]   # sequential, left to right
    ss = (lanes[0] + lanes[2]) + (lanes[1] + lanes[3])
    scale = F32(1.0) / np.sqrt(F32(ss / x.size) + F32(eps))
    return (x * scale) * np.asarray(w, dtype=np.float32)


def _scale(ss, n, eps=0.0):
    return F32(1.0) / np.sqrt(F32(ss / n) + F32(eps))


@pytest.mark.parametrize("n,seed", [(256, 0), (2048, 1), (8192, 2), (16384, 3)])
def test_rmsnorm_numpy_and_c_agree(n, seed):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal(n) * 3).astype(np.float32)
    w = rng.standard_normal(n).astype(np.float32)
    got, want = C.rmsnorm(x, w, 1e-5), rmsnorm_numpy(x, w, 1e-5)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    exact = x.astype(np.float64) / np.sqrt((x.astype(np.float64) ** 2).mean() + 1e-5) * w
    assert np.allclose(got, exact, rtol=2e-6, atol=1e-7)


def test_rmsnorm_closed_forms():
    n = 2048
    x = np.full(n, 0.5, np.float32)                   # ss = n / 4 exactly
    out = C.rmsnorm(x, np.ones(n, np.float32), 1e-5)
    assert np.all(out == F32(0.5) * (F32(1.0) / np.sqrt(F32(0.25) + F32(1e-5))))
    z = C.rmsnorm(np.zeros(n, np.float32), np.ones(n, np.float32), 1e-5)
    assert np.all(z == 0.0)                           # 0 * (1 / sqrt(eps))
    big = C.rmsnorm(np.full(n, 2.0, np.float32), np.full(n, 3.0, np.float32), 0.0)
    assert np.all(big == F32(2.0) * F32(0.5) * F32(3.0))


# x[0]^2 = 1 + 2^-11 + 2^-24 is exactly a float32 midpoint after the exact
# division by n = 2048, so the float64 sum's last bits decide the rounding.
X0 = F32(1.0 + 2.0 ** -12)
TINY = F32(2.0 ** -27)                                # square 2^-54: absorbed next to x0^2, not alone


def _order_case(lane_counts):
    x = np.zeros(2048, np.float32)
    x[0] = X0
    for lane, count in lane_counts.items():
        idx = [i for i in range(lane, 2048, 4) if i != 0][:count]
        x[idx] = TINY
    return x


def test_rmsnorm_order_of_the_float64_sum():
    x0sq = float(X0) ** 2
    up = F32(1.0 + 2.0 ** -11 + 2.0 ** -23) * F32(2.0 ** -11)      # the midpoint rounded up
    down = F32(1.0 + 2.0 ** -11) * F32(2.0 ** -11)                 # ... and to even (down)
    ones = np.ones(2048, np.float32)

    def first_out(x):                                 # out[0] = (x0 * scale) * 1
        return C.rmsnorm(x, ones, 0.0)[0]

    # A: small squares in lanes 1-3 survive (4 lanes) but not behind x0 (1 lane).
    a = _order_case({1: 512, 2: 512, 3: 512})
    assert F32(x0sq / 2048) == down
    assert np.float32(((x0sq + 512 * 2.0 ** -54) + (512 * 2.0 ** -54 + 512 * 2.0 ** -54)) / 2048) == up
    assert first_out(a) == X0 * _scale(float(up) * 2048, 2048)
    # B: all small squares behind x0 in lane 0: absorbed one by one, though the
    # exact (or pairwise) sum would round up.
    b = _order_case({0: 511})
    assert np.float32(math.fsum([x0sq] + [2.0 ** -54] * 511) / 2048) == up
    assert first_out(b) == X0 * _scale(float(down) * 2048, 2048)
    # C: (l0 + l2) + (l1 + l3) adds l1 + l3 = 2^-52 to l0 whole; ((l0 + l1) + l2) + l3
    # would add each lane's 2^-53 (half an ulp, a tie to even) to l0 and lose both.
    c = _order_case({1: 2, 3: 2})
    l0, l1, l3 = x0sq, 2.0 ** -53, 2.0 ** -53
    assert np.float32(((l0 + l1) + 0.0 + l3) / 2048) == down
    assert np.float32(((l0 + 0.0) + (l1 + l3)) / 2048) == up
    assert first_out(c) == X0 * _scale(float(up) * 2048, 2048)
    assert first_out(a) != first_out(b)
    for x in (a, b, c):
        assert np.array_equal(C.rmsnorm(x, ones, 0.0).view(np.uint32), rmsnorm_numpy(x, ones, 0.0).view(np.uint32))


# ------------------------------------------------------------ expf / silu

def _f32_round(q: Fraction) -> float:
    """Round an exact rational to float32 (nearest, ties to even), with
    subnormals and overflow to infinity."""
    if q == 0:
        return 0.0
    sign = -1.0 if q < 0 else 1.0
    a = abs(q)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    e = max(e, -126)                                  # subnormal spacing below 2^-126
    ulp = Fraction(2) ** (e - 23)
    m = a / ulp
    f = math.floor(m)
    r = m - f
    if r > Fraction(1, 2) or (r == Fraction(1, 2) and f % 2 == 1):
        f += 1
    v = f * ulp
    if v >= Fraction(2) ** 128 - Fraction(2) ** 103:
        return sign * math.inf
    return sign * float(v)


def fmaf_exact(a, b, c) -> F32:
    vals = (float(a), float(b), float(c))
    if any(math.isinf(v) or math.isnan(v) for v in vals):
        return F32(np.float32(vals[0]) * np.float32(vals[1]) + np.float32(vals[2]))
    return F32(_f32_round(Fraction(vals[0]) * Fraction(vals[1]) + Fraction(vals[2])))


def bits(f) -> int:
    return int(np.array(f, dtype=np.float32).view(np.uint32))


def from_bits(u) -> F32:
    return np.array(u & 0xFFFFFFFF, dtype=np.uint32).view(np.float32)[()]


def expf_python(x) -> F32:
    """The same algorithm as the C oracle, written independently."""
    x = F32(x)
    shift = F32(float.fromhex("0x1.8p23"))
    z = fmaf_exact(x, F32(float.fromhex("0x1.715476p+0")), shift)
    n = F32(z - shift)
    b = fmaf_exact(-n, F32(float.fromhex("0x1.7f7d1cp-20")), fmaf_exact(-n, F32(float.fromhex("0x1.62e4p-1")), x))
    e = (bits(z) << 23) & 0xFFFFFFFF
    k = from_bits(e + 0x3F800000)
    u = F32(b * b)
    p1 = fmaf_exact(F32(float.fromhex("0x1.555e66p-3")), b, F32(float.fromhex("0x1.fffdb6p-2")))
    p2 = fmaf_exact(F32(float.fromhex("0x1.0e4020p-7")), b, F32(float.fromhex("0x1.573e2ep-5")))
    j = fmaf_exact(fmaf_exact(p2, u, p1), u, F32(F32(float.fromhex("0x1.ffffecp-1")) * b))
    if not abs(n) > 126:
        return fmaf_exact(k, j, k)
    d = 0x82000000 if n <= 0 else 0
    s1, s2 = from_bits(d + 0x7F000000), from_bits(e - d)
    if abs(n) > 192:
        return F32(s1 * s1)
    return F32(fmaf_exact(s2, j, s2) * s1)


def _expf_inputs():
    rng = np.random.default_rng(7)
    edges = [0.0, -0.0, 1e-30, -1e-30, 0.5, -0.5, 1.0, -1.0, 10.0, -10.0, 80.0, -80.0, 87.0, -87.0, 88.0, 88.7,
             88.72, 89.0, -88.0, -89.0, -90.0, -100.0, -103.0, -104.0, -120.0, 100.0, 130.0, -130.0, 140.0, -140.0,
             200.0, -200.0, 1e10, -1e10, 2.0 ** -149]
    return np.concatenate([np.array(edges, np.float32), rng.uniform(-95, 95, 1500).astype(np.float32),
                           (rng.standard_normal(500) * 4).astype(np.float32)])


def test_expf_restatements_agree():
    with np.errstate(over="ignore", under="ignore", invalid="ignore"):
        for x in _expf_inputs():
            got, want = C.ggml_expf(x), expf_python(x)
            assert bits(got) == bits(want), (x, got, want)


def test_expf_error_bound_and_ends():
    assert C.ggml_expf(0.0) == 1.0
    assert C.ggml_expf(89.0) == np.inf and C.ggml_expf(200.0) == np.inf
    assert C.ggml_expf(-110.0) == 0.0 and C.ggml_expf(-200.0) == 0.0
    assert 0.0 < C.ggml_expf(-100.0) < 2.0 ** -126                  # a subnormal through the |n| > 126 path
    xs = np.linspace(-87.3, 88.7, 200001).astype(np.float32)
    got = np.array([C.ggml_expf(v) for v in xs[::7]], dtype=np.float64)
    want = np.exp(xs[::7].astype(np.float64))
    ulp = np.spacing(want.astype(np.float32)).astype(np.float64)
    assert np.max(np.abs(got - want) / ulp) <= 1.96                 # 1.45358 + 0.5 ulp, published bound


def test_silu_mul_closed_forms_and_tolerance():
    g = np.array([0.0, -0.0, 1.0, -1.0, 20.0, -20.0, 100.0, -100.0, 3.5], np.float32)
    u = np.array([5.0, 5.0, 2.0, 2.0, 1.0, 1.0, 1.0, 1.0, -1.0], np.float32)
    a = C.silu_mul(g, u)
    assert a[0] == 0.0 and a[4] == F32(20.0) / (F32(1.0) + C.ggml_expf(-20.0))
    assert a[6] == 100.0 and a[7] == 0.0                            # exp(100) = inf: -100 / inf = -0 -> * 1
    rng = np.random.default_rng(8)
    g = (rng.standard_normal(4096) * 3).astype(np.float32)
    u = rng.standard_normal(4096).astype(np.float32)
    exact = g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64))) * u
    assert np.allclose(C.silu_mul(g, u), exact, rtol=1e-6, atol=1e-12)
