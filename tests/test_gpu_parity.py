"""GPU parity: the HIP library, called through its C ABI, byte for byte against
the oracle on the same seeded inputs.

Sizes here are the ones the oracle finishes in seconds; the full-size
configurations (LM head, decode chain, M sweep) are in test_gpu_configs.py.
Every output buffer is poisoned with 0xAA first, so a row the kernel never
writes cannot pass by accident.
"""

from __future__ import annotations

import numpy as np
import pytest

import c_oracle as C
import q4_0_oracle as O
from gpu_helpers import assert_bytes_equal, dev, host, poisoned_f32

pytestmark = pytest.mark.gpu


def _case(rows, k, w_seed, x_seed, w_scale=0.02):
    w = O.normal_f32((rows, k), w_seed, w_scale)
    x = O.normal_f32((1, k), x_seed)[0]
    blocks = C.quantize_q4_0(w)
    xq, xd = C.quantize_q8_0(x)
    return w, x, blocks, xq, xd


# ------------------------------------------------------------ quantizers

@pytest.mark.parametrize("rows,k,seed", [(16, 256, 0), (64, 2048, 1), (2048, 2048, 0), (3, 8192, 2), (5, 96, 3)])
def test_quantize_q4_0_matches_oracle(gpu, rows, k, seed):
    w = O.normal_f32((rows, k), seed, 0.02)
    got = host(gpu.quantize_q4_0(dev(w)))
    assert_bytes_equal(got, C.quantize_q4_0(w), "Q4_0 blocks")


@pytest.mark.parametrize("k,seed", [(256, 0), (2048, 1), (8192, 2), (16384, 3)])
def test_quantize_q8_0_matches_oracle(gpu, k, seed):
    x = O.normal_f32((1, k), seed)[0]
    xq, xd = gpu.quantize_q8_0(dev(x))
    q_ref, d_ref = C.quantize_q8_0(x)
    assert_bytes_equal(host(xq), q_ref, "q")
    assert_bytes_equal(host(xd).view(np.uint16), d_ref.view(np.uint16), "d")
    eng = host(gpu.quantize_q8_0_engine(dev(x)))
    assert_bytes_equal(eng, C.pack_x_for_engine(q_ref, d_ref), "engine x")


def test_quantize_q8_0_rounding_edges(gpu):
    """Ties and the 0.49999997f case (floor(|s| + 0.5f) in fp32), signed zeros,
    an all-zero block, subnormal and huge scales."""
    x = np.zeros(256, np.float32)
    x[0:6] = [127.0, 2.5, -2.5, 0.5, 0.49999997, -0.49999997]
    x[32] = -0.0
    x[64:96] = np.float32(1e-30) * np.arange(32, dtype=np.float32)     # tiny amax: fp16 scale underflows
    x[96:128] = np.float32(3e38) * np.linspace(-1, 1, 32, dtype=np.float32)
    x[128:160] = np.float32(6e-6) * np.arange(-16, 16, dtype=np.float32)  # fp16-subnormal scale
    x[160:192] = np.float32(0.3)
    rng = np.random.default_rng(7)
    x[192:] = rng.standard_normal(64).astype(np.float32) * np.float32(1e4)
    q_ref, d_ref = C.quantize_q8_0(x)
    q_np, d_np = O.quantize_q8_0(x)
    assert np.array_equal(q_ref, q_np) and np.array_equal(d_ref.view(np.uint16), d_np.view(np.uint16))
    xq, xd = gpu.quantize_q8_0(dev(x))
    assert_bytes_equal(host(xq), q_ref, "q")
    assert_bytes_equal(host(xd).view(np.uint16), d_ref.view(np.uint16), "d")
    assert host(xq)[1:6].tolist() == [3, -3, 1, 1, -1]


def test_quantize_q4_0_edges(gpu):
    w = np.zeros((4, 64), np.float32)
    w[0, 3], w[0, 7], w[0, 5] = 1.0, -1.0, 0.3           # first-index tie, clip to 15
    w[1, :32] = np.float32(1e-30) * np.arange(32)         # fp16 scale underflows to 0
    w[2, :32] = np.float32(2e-6) * np.arange(-16, 16)     # subnormal fp16 scale
    w[3] = O.normal_f32((1, 64), 9)[0] * np.float32(100)
    w[1, 32:] = -0.0
    assert_bytes_equal(host(gpu.quantize_q4_0(dev(w))), C.quantize_q4_0(w), "Q4_0 blocks")


# ------------------------------------------------------------------ gemv

GEMV_CASES = [
    (16, 256, 100, 101),       # nb = 8: each lane holds one block
    (64, 2048, 102, 103),
    (16, 8192, 104, 105),
    (32, 512, 106, 107),
    (2048, 2048, 0, 1),        # the o_proj shape
    (3072, 2048, 10, 20),      # q|k|v
    (2048, 8192, 13, 23),      # down
    (1, 2048, 108, 109),       # one row
    (33, 1024, 110, 111),      # ragged rows
    (1000, 4096, 112, 113),
    (7, 16384, 114, 115),      # the library's maximum K
    (257, 2304, 116, 117),     # K/256 = 9 chunks: tiles that do not divide 256 threads
]


@pytest.mark.parametrize("rows,k,ws,xs", GEMV_CASES)
def test_gemv_engine_layout(gpu, rows, k, ws, xs):
    _, x, blocks, xq, xd = _case(rows, k, ws, xs)
    want = C.gemv_q4_0(blocks, k, xq, xd)
    y = poisoned_f32(rows)
    gpu.gemv_engine(dev(blocks), k, dev(C.pack_x_for_engine(xq, xd)), out=y)
    assert_bytes_equal(host(y), want)


@pytest.mark.parametrize("rows,k,ws,xs", GEMV_CASES[:6])
def test_gemv_contract_interface_and_fused_f32(gpu, rows, k, ws, xs):
    _, x, blocks, xq, xd = _case(rows, k, ws, xs)
    want = C.gemv_q4_0(blocks, k, xq, xd)
    b = dev(blocks)
    assert_bytes_equal(host(gpu.gemv_q4_0(b, k, dev(xq), dev(xd))), want, "gemv_q4_0")
    y = poisoned_f32(rows)
    gpu.gemv_q4_0_f32(b, k, dev(x), out=y)
    assert_bytes_equal(host(y), want, "gemv_q4_0_f32 (fused quantize)")
    xb = O.pack_q8_0_blocks(xq, xd)
    y2 = poisoned_f32(rows)
    gpu.gemv_q8_0_blocks(b, k, dev(xb), out=y2)
    assert_bytes_equal(host(y2), want, "gemv with ggml Q8_0 blocks")


def test_gemv_golden_vector(gpu):
    """The reference-held golden digest (tests/test_q4_0_contract.py:181-191), on the GPU."""
    import hashlib
    w = O.normal_f32((96, 2048), 2024)
    x = O.normal_f32((1, 2048), 2025)[0]
    blocks = gpu.quantize_q4_0(dev(w))
    y = host(gpu.gemv_q4_0_f32(blocks, 2048, dev(x)))
    assert hashlib.sha256(y.tobytes()).hexdigest() == \
        "efa9eda8cef689d6392ddf2e1b3e945d19797aff1cbd55398c87ffffec7c29cc"


def test_gemv_special_values(gpu):
    """Zero blocks, -0 terms (+0 from the 0.0f + t start), subnormal scales,
    large terms that cancel, and the lane-order construction."""
    k, rows = 512, 8
    w = O.normal_f32((rows, k), 55, 0.02)
    w[1] = 0.0                                   # whole zero row
    w[2, :32] = 0.0                              # one zero block
    w[3] *= np.float32(1e-4)                     # tiny scales (fp16 subnormal d)
    w[4] *= np.float32(1e4)                      # large
    w[5, 32:] = 0.0
    x = O.normal_f32((1, k), 56)[0]
    x[:32] = 0.0                                 # zero activation block: d_x = 0
    x[64:96] *= np.float32(1e-5)
    blocks = C.quantize_q4_0(w)
    xq, xd = C.quantize_q8_0(x)
    want = C.gemv_q4_0(blocks, k, xq, xd)
    y = poisoned_f32(rows)
    gpu.gemv_engine(dev(blocks), k, dev(C.pack_x_for_engine(xq, xd)), out=y)
    assert_bytes_equal(host(y), want)


def test_gemv_sign_of_zero(gpu):
    """A row whose every term is -0.0 must give +0.0 (lanes start from +0.0)."""
    k = 256
    blocks = np.zeros((1, 8, 18), np.uint8)
    blocks[..., :2] = np.array([-1.0], np.float16).view(np.uint8)   # d_w = -1
    blocks[..., 2:] = 0x88                                            # every weight 0
    blocks = blocks.reshape(1, -1)
    xq = np.ones(k, np.int8)
    xd = np.ones(8, np.float16)
    want = C.gemv_q4_0(blocks, k, xq, xd)
    assert want.view(np.uint32)[0] == 0
    y = poisoned_f32(1)
    gpu.gemv_engine(dev(blocks), k, dev(C.pack_x_for_engine(xq, xd)), out=y)
    assert host(y).view(np.uint32)[0] == 0


def test_gemv_random_bytes(gpu):
    """Arbitrary block bytes (any fp16 scale, inf and nan excluded), not just quantizer output."""
    rng = np.random.default_rng(77)
    rows, k = 300, 2048
    blocks = rng.integers(0, 256, size=(rows, k // 32, 18), dtype=np.uint8)
    d = (rng.standard_normal((rows, k // 32)) * 10.0 ** rng.integers(-7, 3, (rows, k // 32))).astype(np.float16)
    blocks[..., :2] = d.view(np.uint8).reshape(rows, k // 32, 2)
    blocks = blocks.reshape(rows, -1)
    xq = rng.integers(-127, 128, size=k, dtype=np.int8)
    xd = (rng.random(k // 32) * 0.05).astype(np.float16)
    want = C.gemv_q4_0(blocks, k, xq, xd)
    assert np.array_equal(want.view(np.uint32), O.gemv_q4_0(blocks, k, xq, xd).view(np.uint32))
    y = poisoned_f32(rows)
    gpu.gemv_engine(dev(blocks), k, dev(C.pack_x_for_engine(xq, xd)), out=y)
    assert_bytes_equal(host(y), want)


def test_gemv_nonfinite_scales(gpu):
    """Infinite and NaN fp16 scales, byte for byte, NaN outputs included. A NaN's sign and
    payload are the processor's: here every NaN comes from an fp16 NaN scale (0x7E00, widened to
    0x7FC00000 and carried through every later operation) or from 0 * inf (and inf - inf in the
    sums), which x86, where the oracle runs, makes its default NaN 0xFFC00000. The GPU gives the
    same bytes in every row. (AArch64, the board's CPU, would make 0 * inf 0x7FC00000: the
    contract's NaN bytes are the platform's, and this test pins the oracle's.)"""
    rng = np.random.default_rng(91)
    rows, k = 64, 1024
    blocks = C.quantize_q4_0(O.normal_f32((rows, k), 92, 0.02)).reshape(rows, k // 32, 18)
    specials = np.array([np.inf, -np.inf, np.nan, 65504.0], np.float16)
    for r in range(0, rows, 2):                      # every other row gets one special scale
        blocks[r, rng.integers(0, k // 32), :2] = specials[(r // 2) % 4:(r // 2) % 4 + 1].view(np.uint8)
    blocks[5, :, 2:] = 0x88                           # weights all 8 - 8 = 0 ...
    blocks[5, 3, :2] = np.array([np.inf], np.float16).view(np.uint8)   # ... so 0 * inf: NaN
    blocks = blocks.reshape(rows, -1)
    xq, xd = C.quantize_q8_0(O.normal_f32((1, k), 93)[0])
    xd = xd.copy()
    xd[7] = np.float16(np.inf)                        # an infinite activation scale too
    want = C.gemv_q4_0(blocks, k, xq, xd)
    y = poisoned_f32(rows)
    gpu.gemv_engine(dev(blocks), k, dev(C.pack_x_for_engine(xq, xd)), out=y)
    got = host(y)
    nan = np.isnan(want)
    assert nan.any() and np.isinf(want).any()
    assert np.array_equal(np.isnan(got), nan), np.flatnonzero(np.isnan(got) != nan)
    assert want.view(np.uint32)[5] == 0xFFC00000         # 0 * inf
    assert want.view(np.uint32)[4] == 0x7FC00000         # the NaN scale's own NaN
    assert_bytes_equal(got, want, "every output, NaN bytes included")


@pytest.mark.parametrize("m,rows", [(8, 8200), (16, 8200), (24, 8200), (64, 8200), (4, 8200), (3, 2000),
                                    (24, 2000)])
def test_gemm_nonfinite_scales(gpu, m, rows):
    """The M > 1 kernels with infinite and NaN fp16 scales, byte for byte, NaN outputs
    included: the row-split kernels at every token tiling (8,200 rows: packed block pairs,
    one, two and four token tiles), the few-token GEMV and the class-split kernel (2,000
    rows)."""
    rng = np.random.default_rng(190 + m)
    k = 1024
    blocks = C.quantize_q4_0(O.normal_f32((rows, k), 191, 0.02)).reshape(rows, k // 32, 18)
    specials = np.array([np.inf, -np.inf, np.nan, 65504.0], np.float16)
    for r in range(0, rows, 37):                     # every 37th row gets one special scale
        blocks[r, rng.integers(0, k // 32), :2] = specials[(r // 37) % 4:(r // 37) % 4 + 1].view(np.uint8)
    blocks[5, :, 2:] = 0x88                           # weights all 8 - 8 = 0 ...
    blocks[5, 3, :2] = np.array([np.inf], np.float16).view(np.uint8)   # ... so 0 * inf: NaN
    blocks = blocks.reshape(rows, -1)
    xq, xd = C.quantize_q8_0_rows(O.normal_f32((m, k), 192 + m))
    xd = xd.copy()
    xd[m // 2, 7] = np.float16(np.inf)               # an infinite activation scale too
    want = C.gemm_q4_0_rows(blocks, k, xq, xd)
    assert np.isnan(want).any() and np.isinf(want).any()
    x_rows = np.stack([C.pack_x_for_engine(xq[i], xd[i]) for i in range(m)])
    y = poisoned_f32((m, rows))
    gpu.gemm_engine(dev(blocks), k, dev(x_rows), out=y)
    assert_bytes_equal(host(y), want, "gemm, non-finite scales, NaN bytes included")


def test_gemv_quarters_at_separate_addresses(gpu):
    """The v1 engine's layout (gemv_dev_start4): four quarters anywhere in memory."""
    import torch
    rows, k = 512, 2048
    _, _, blocks, xq, xd = _case(rows, k, 120, 121)
    want = C.gemv_q4_0(blocks, k, xq, xd)
    q = rows // 4
    pool = torch.zeros(8 << 20, dtype=torch.uint8, device="cuda")
    offs = [0, (2 << 20) + 16 * 1024, 4 << 20, (6 << 20) + 16 * 1024]    # 16 KB staggers, as the board did
    quarters = []
    for i, off in enumerate(offs):
        part = dev(blocks[i * q:(i + 1) * q].reshape(-1))
        pool[off:off + part.numel()] = part
        quarters.append(pool[off:off + part.numel()])
    y = poisoned_f32(rows)
    gpu.gemv_quarters(quarters, k, dev(C.pack_x_for_engine(xq, xd)), rows, out=y)
    assert_bytes_equal(host(y), want)


# ------------------------------------------------------------------ gemm

@pytest.mark.parametrize("m,rows,k", [(2, 64, 2048), (4, 100, 512), (16, 256, 2048), (17, 48, 8192),
                                      (24, 512, 2048), (33, 80, 1024), (64, 128, 2048),
                                      # one chunk per row; three and five chunks (rounds of one chunk);
                                      # several 64-token groups; one row
                                      (8, 16, 256), (40, 33, 768), (130, 40, 1280), (2, 1, 512),
                                      # 8192 rows and more go to the row-split kernel: ragged row
                                      # groups and workgroups, one to three token tiles, several
                                      # 64-token groups, one to four K segments
                                      (3, 8200, 512), (17, 8208, 1024), (40, 8240, 2048), (64, 8192, 512),
                                      (130, 8256, 1536),
                                      # the largest K, on both kernels
                                      (40, 64, 16384), (5, 8200, 16384),
                                      # the few-token GEMV (m = 2, or m <= 4 on large matrices, m <= 6
                                      # where they have at most four tiles per CU and a tile's tokens
                                      # are split over two waves): ragged rows, one row, 48-chunk tiles
                                      # (k = 6144), k = 8192, odd m (a wave with a token past m)
                                      (2, 1, 4096), (2, 300, 6144), (3, 8200, 2048), (4, 8197, 2048),
                                      (4, 2048, 8192), (3, 1000, 8192), (2, 5, 8192), (5, 2048, 8192),
                                      (6, 777, 8192), (5, 3, 8192),
                                      # k = 2304: 9 chunks and 72 blocks a row, 7 rows a tile (odd
                                      # divisors in the kernel's lane and staging quotients), both forms
                                      (2, 300, 2304), (2, 7, 2304), (4, 8200, 2304),
                                      # 8-row items (K >= 8192, fewer 16-row groups than CUs): the
                                      # down shape, ragged rows, one item, several token groups
                                      (8, 2048, 8192), (5, 1003, 8192), (16, 8, 8192), (12, 2050, 8192),
                                      (33, 1001, 8192),
                                      # the row-split kernel's packed tiles: 2 blocks x 8 tokens (m = 5..8)
                                      # and 4 blocks x 4 tokens (m <= 4 where the few-token GEMV does not
                                      # take the shape); ragged rows, 1-3 K segments
                                      (5, 8200, 2048), (8, 8256, 4096), (7, 9000, 1536), (6, 8192, 512),
                                      (4, 8200, 12288), (2, 8193, 1024), (69, 8200, 1024),
                                      # the row-split quads on each side of their token tilings
                                      # (8 | 9, 16 | 17, 32 | 33 tokens), ragged rows (not a whole
                                      # workgroup of 32 or 64), 1-4 K segments
                                      (9, 8200, 1024), (16, 8208, 2048), (17, 8200, 1536),
                                      (32, 8200, 512), (33, 8240, 1024), (64, 8200, 2048)])
def test_gemm_matches_rowwise_contract(gpu, m, rows, k):
    w = O.normal_f32((rows, k), 200 + m, 0.02)
    x = O.normal_f32((m, k), 300 + m)
    blocks = C.quantize_q4_0(w)
    xq, xd = C.quantize_q8_0_rows(x)
    want = C.gemm_q4_0_rows(blocks, k, xq, xd)
    x_rows = np.stack([C.pack_x_for_engine(xq[i], xd[i]) for i in range(m)])
    y = poisoned_f32((m, rows))
    gpu.gemm_engine(dev(blocks), k, dev(x_rows), out=y)
    assert_bytes_equal(host(y), want, "gemm")


@pytest.mark.parametrize("m,rows,k", [(24, 8200, 1024), (40, 2000, 1024), (2, 2000, 2048), (4, 8200, 2048),
                                      (3, 600, 8192), (9, 1003, 8192), (7, 8200, 2048), (3, 8200, 512)])
def test_gemm_random_bytes(gpu, m, rows, k):
    """Arbitrary block bytes and activations (any finite fp16 scale) through both M > 1
    kernels (8,200 rows: the row-split one), row by row against the contract."""
    rng = np.random.default_rng(78 + m)
    blocks = rng.integers(0, 256, size=(rows, k // 32, 18), dtype=np.uint8)
    d = (rng.standard_normal((rows, k // 32)) * 10.0 ** rng.integers(-7, 3, (rows, k // 32))).astype(np.float16)
    blocks[..., :2] = d.view(np.uint8).reshape(rows, k // 32, 2)
    blocks = blocks.reshape(rows, -1)
    xq = rng.integers(-127, 128, size=(m, k), dtype=np.int8)
    xd = (rng.random((m, k // 32)) * 0.05).astype(np.float16)
    want = C.gemm_q4_0_rows(blocks, k, xq, xd)
    x_rows = np.stack([C.pack_x_for_engine(xq[i], xd[i]) for i in range(m)])
    y = poisoned_f32((m, rows))
    gpu.gemm_engine(dev(blocks), k, dev(x_rows), out=y)
    assert_bytes_equal(host(y), want, "gemm, random bytes")


def test_gemm_one_row_equals_gemv(gpu):
    rows, k = 96, 2048
    _, _, blocks, xq, xd = _case(rows, k, 130, 131)
    b = dev(blocks)
    x_eng = dev(C.pack_x_for_engine(xq, xd))
    y1 = host(gpu.gemm_engine(b, k, x_eng.reshape(1, -1)))
    y0 = host(gpu.gemv_engine(b, k, x_eng))
    assert_bytes_equal(y1.reshape(-1), y0, "gemm M=1 vs gemv")


# ------------------------------------------------------------------ chain

def test_chain_equals_each_step_alone(gpu):
    """w4a8_chain_gemv over mixed shapes equals the oracle per step."""
    import ctypes
    import torch
    shapes = [(96, 2048), (64, 2048), (512, 2048), (64, 8192), (300, 2048), (48, 2048)]
    mats, xs, ys, wants = [], [], [], []
    for i, (rows, k) in enumerate(shapes):
        w, x, blocks, xq, xd = _case(rows, k, 400 + i, 500 + i)
        mats.append(dev(blocks))
        xs.append(dev(x))
        ys.append(poisoned_f32(rows))
        wants.append(C.gemv_q4_0(blocks, k, xq, xd))

    class Step(ctypes.Structure):
        _fields_ = [("w", ctypes.c_void_p), ("x", ctypes.c_void_p), ("y", ctypes.c_void_p),
                    ("rows", ctypes.c_int), ("k", ctypes.c_int)]

    steps = (Step * len(shapes))(*[Step(mats[i].data_ptr(), xs[i].data_ptr(), ys[i].data_ptr(),
                                        shapes[i][0], shapes[i][1]) for i in range(len(shapes))])
    stream = torch.cuda.current_stream().cuda_stream
    gpu.check("w4a8_chain_gemv", gpu.lib().w4a8_chain_gemv(ctypes.cast(steps, ctypes.c_void_p), len(shapes), stream))
    for i in range(len(shapes)):
        assert_bytes_equal(host(ys[i]), wants[i], f"chain step {i}")


def _steps(gpu, shapes, seed0):
    import ctypes
    mats, xs, ys, wants = [], [], [], []
    for i, (rows, k) in enumerate(shapes):
        w, x, blocks, xq, xd = _case(rows, k, seed0 + i, seed0 + 100 + i)
        mats.append(dev(blocks))
        xs.append(dev(x))
        ys.append(poisoned_f32(rows))
        wants.append(C.gemv_q4_0(blocks, k, xq, xd))

    class Step(ctypes.Structure):
        _fields_ = [("w", ctypes.c_void_p), ("x", ctypes.c_void_p), ("y", ctypes.c_void_p),
                    ("rows", ctypes.c_int), ("k", ctypes.c_int)]

    steps = (Step * len(shapes))(*[Step(mats[i].data_ptr(), xs[i].data_ptr(), ys[i].data_ptr(),
                                        shapes[i][0], shapes[i][1]) for i in range(len(shapes))])
    return steps, (mats, xs), ys, wants


@pytest.mark.parametrize("shapes", [
    [(96, 2048), (64, 2048), (512, 2048), (64, 8192), (300, 2048), (48, 2048)],
    [(1, 256)],
    [(3072, 2048), (2048, 2048), (16384, 2048), (2048, 8192), (5000, 2048)],
    [(7, 16384), (33, 1024), (257, 2304), (1000, 4096)] * 3,
])
def test_batch_equals_each_gemv_alone(gpu, shapes):
    """w4a8_gemv_batch: every matrix in one launch, each byte-equal to the oracle."""
    import ctypes
    import torch
    steps, keep, ys, wants = _steps(gpu, shapes, 600)
    stream = torch.cuda.current_stream().cuda_stream
    gpu.check("w4a8_gemv_batch", gpu.lib().w4a8_gemv_batch(ctypes.cast(steps, ctypes.c_void_p), len(shapes), stream))
    for i in range(len(shapes)):
        assert_bytes_equal(host(ys[i]), wants[i], f"batch entry {i} {shapes[i]}")


def test_batch_rejects_bad_steps(gpu):
    import ctypes
    import torch
    steps, keep, ys, wants = _steps(gpu, [(64, 2048), (64, 2048)], 700)
    L = gpu.lib()
    stream = torch.cuda.current_stream().cuda_stream
    steps[1].k = 2000
    assert L.w4a8_gemv_batch(ctypes.cast(steps, ctypes.c_void_p), 2, stream) == -2
    steps[1].k = 2048
    steps[0].y = None
    assert L.w4a8_gemv_batch(ctypes.cast(steps, ctypes.c_void_p), 2, stream) == -1
    assert L.w4a8_gemv_batch(ctypes.cast(steps, ctypes.c_void_p), 0, stream) == -2
    assert L.w4a8_gemv_batch(ctypes.cast(steps, ctypes.c_void_p), 97, stream) == -2
    torch.cuda.synchronize()


# ------------------------------------------------------------ C ABI errors

def test_c_abi_rejects_bad_arguments_on_device(gpu):
    import torch
    L = gpu.lib()
    w = torch.zeros(2 * 1152 + 64, dtype=torch.uint8, device="cuda")
    x = torch.zeros(2304 + 64, dtype=torch.uint8, device="cuda")
    y = torch.zeros(16, dtype=torch.float32, device="cuda")
    s = torch.cuda.current_stream().cuda_stream
    assert L.w4a8_gemv(w.data_ptr(), x.data_ptr(), y.data_ptr(), 2, 2048, s) == 0
    assert L.w4a8_gemv(w.data_ptr(), x.data_ptr(), y.data_ptr(), 2, 2000, s) == -2
    assert L.w4a8_gemv(w.data_ptr(), x.data_ptr(), y.data_ptr(), 0, 2048, s) == -2
    assert L.w4a8_gemv(w.data_ptr() + 2, x.data_ptr(), y.data_ptr(), 2, 2048, s) == -3
    assert L.w4a8_gemv(w.data_ptr(), x.data_ptr() + 4, y.data_ptr(), 2, 2048, s) == -3
    assert L.w4a8_gemv(None, x.data_ptr(), y.data_ptr(), 2, 2048, s) == -1
    torch.cuda.synchronize()
    with pytest.raises(ValueError):
        gpu.gemv_q4_0_f32(torch.zeros((2, 1152), dtype=torch.uint8, device="cuda"), 2048,
                          torch.zeros(1024, dtype=torch.float32, device="cuda"))
    with pytest.raises(TypeError):
        gpu.gemv_q4_0(torch.zeros((2, 1152), dtype=torch.uint8, device="cuda"), 2048,
                      torch.zeros(2048, dtype=torch.int32, device="cuda"),
                      torch.zeros(64, dtype=torch.float16, device="cuda"))
