"""The reference's activation producers on the GPU, byte for byte against the
oracle: rmsnorm (board/tp/tp_llama.cpp:557-569) and silu(gate) * up
(:612-619, ggml's vector expf), each standalone (to the engine layout) and
fused into the GEMV's activation staging, and the LM head's whole step
(rmsnorm, Q8_0, GEMV, greedy pick) in one kernel. The inputs include the
constructed float64-order cases that pin the oracle's rmsnorm and the
expf's scaling branches (|n| > 126, |n| > 192, overflow)."""

from __future__ import annotations

import numpy as np
import pytest

import c_oracle as C
import q4_0_oracle as O
from gpu_helpers import assert_bytes_equal, dev, host
from test_gpu_argmax import scan_argmax
from test_oracle_producers import _order_case

pytestmark = pytest.mark.gpu


def _engine(h):
    xq, xd = C.quantize_q8_0(h)
    return C.pack_x_for_engine(xq, xd)


def _gate_up(k, seed):
    rng = np.random.default_rng(seed)
    gu = (rng.standard_normal(2 * k) * 4).astype(np.float32)
    edges = np.array([0.0, -0.0, 100.0, -100.0, 90.0, -90.0, 130.0, -130.0, 200.0, -200.0, 1e-30, 88.7, -88.7],
                     np.float32)
    gu[:edges.size] = edges                            # gate edges (their up values are random)
    return gu


@pytest.mark.parametrize("k,m", [(256, 1), (2048, 3), (8192, 2), (16384, 1)])
def test_rmsnorm_q8_0(gpu, k, m):
    rng = np.random.default_rng(k + m)
    x = (rng.standard_normal((m, k)) * 3).astype(np.float32)
    w = rng.standard_normal(k).astype(np.float32)
    got = host(gpu.rmsnorm_q8_0_engine(dev(x), dev(w), 1e-5))
    want = np.stack([_engine(C.rmsnorm(x[i], w, 1e-5)) for i in range(m)])
    assert_bytes_equal(got, want, "rmsnorm_q8_0")


@pytest.mark.parametrize("k,m", [(256, 1), (8192, 2), (2048, 5)])
def test_silu_mul_q8_0(gpu, k, m):
    gu = np.stack([_gate_up(k, 10 * k + i) for i in range(m)])
    got = host(gpu.silu_mul_q8_0_engine(dev(gu)))
    want = np.stack([_engine(C.silu_mul(gu[i, :k], gu[i, k:])) for i in range(m)])
    assert_bytes_equal(got, want, "silu_mul_q8_0")


@pytest.mark.parametrize("rows,k", [(3072, 2048), (100, 256), (512, 8192), (16384, 2048), (40, 768), (1024, 4096),
                                    (64, 2048), (136, 2048)])
def test_gemv_rmsnorm(gpu, rows, k):
    blocks = C.quantize_q4_0(O.normal_f32((rows, k), 70 + rows, 0.02))
    rng = np.random.default_rng(rows)
    x = (rng.standard_normal(k) * 2).astype(np.float32)
    w = rng.standard_normal(k).astype(np.float32)
    xq, xd = C.quantize_q8_0(C.rmsnorm(x, w, 1e-5))
    y = host(gpu.gemv_rmsnorm(dev(blocks), k, dev(x), dev(w), 1e-5))
    assert_bytes_equal(y, C.gemv_q4_0(blocks, k, xq, xd), f"gemv_rmsnorm {rows}x{k}")


def test_gemv_rmsnorm_rejects_k_past_8192(gpu):
    k = 16384
    blocks = dev(C.quantize_q4_0(O.normal_f32((16, k), 1, 0.02)))
    x = dev(O.normal_f32((1, k), 2)[0])
    with pytest.raises(gpu.W4A8Error) as e:
        gpu.gemv_rmsnorm(blocks, k, x, x, 1e-5)
    assert e.value.status == -2


@pytest.mark.parametrize("case", [{1: 512, 2: 512, 3: 512}, {0: 511}, {1: 2, 3: 2}])
def test_gemv_rmsnorm_float64_order_cases(gpu, case):
    k = 2048
    blocks = C.quantize_q4_0(O.normal_f32((256, k), 91, 0.02))
    x = _order_case(case)
    w = np.ones(k, np.float32)
    xq, xd = C.quantize_q8_0(C.rmsnorm(x, w, 0.0))
    y = host(gpu.gemv_rmsnorm(dev(blocks), k, dev(x), dev(w), 0.0))
    assert_bytes_equal(y, C.gemv_q4_0(blocks, k, xq, xd), f"order case {case}")


@pytest.mark.parametrize("rows,k", [(2048, 8192), (64, 256), (300, 2048)])
def test_gemv_silu_mul(gpu, rows, k):
    blocks = C.quantize_q4_0(O.normal_f32((rows, k), 80 + rows, 0.02))
    gu = _gate_up(k, rows)
    xq, xd = C.quantize_q8_0(C.silu_mul(gu[:k], gu[k:]))
    y = host(gpu.gemv_silu_mul(dev(blocks), k, dev(gu)))
    assert_bytes_equal(y, C.gemv_q4_0(blocks, k, xq, xd), f"gemv_silu_mul {rows}x{k}")


def test_lm_head_step(gpu):
    """rmsnorm(x, output_norm) -> Q8_0 -> LM head GEMV -> argmax (tp_llama.cpp:878-880), one kernel."""
    rows, k = 128256, 2048
    blocks = C.quantize_q4_0(O.normal_f32((rows, k), 95, 0.02))
    ws = gpu.argmax_workspace()
    for seed in (96, 97):
        rng = np.random.default_rng(seed)
        x = (rng.standard_normal(k) * 2).astype(np.float32)
        w = rng.standard_normal(k).astype(np.float32)
        xq, xd = C.quantize_q8_0(C.rmsnorm(x, w, 1e-5))
        want = C.gemv_q4_0(blocks, k, xq, xd)
        y, best = gpu.gemv_rmsnorm_argmax(dev(blocks), k, dev(x), dev(w), 1e-5, ws)
        assert_bytes_equal(host(y), want, "lm head step")
        assert int(host(best)[0]) == scan_argmax(want)


@pytest.mark.parametrize("rows,k,rms", [(16384, 2048, True), (16384, 2048, False), (256, 8192, True),
                                        (4096, 4096, False), (16, 2048, True), (8, 4096, True), (48, 2048, False),
                                        (40, 8192, True)])
def test_gemv_gate_up_silu(gpu, rows, k, rms):
    """gate|up with silu(gate) * up as the epilogue: act = silu_mul(y[:n], y[n:])
    of the plain (or rmsnorm-fed) GEMV, byte for byte."""
    print(f"gate_up_silu rows={rows} k={k} rms={rms}", flush=True)
    blocks = C.quantize_q4_0(O.normal_f32((rows, k), 90 + rows, 0.02))
    rng = np.random.default_rng(rows + k)
    x = (rng.standard_normal(k) * 2).astype(np.float32)
    w = rng.standard_normal(k).astype(np.float32) if rms else None
    h = C.rmsnorm(x, w, 1e-5) if rms else x
    xq, xd = C.quantize_q8_0(h)
    y = C.gemv_q4_0(blocks, k, xq, xd)
    n = rows // 2
    want = C.silu_mul(y[:n], y[n:])
    got = gpu.gemv_gate_up_silu(dev(blocks), k, dev(x), None if w is None else dev(w), 1e-5)
    assert_bytes_equal(host(got), want, f"gate_up_silu {rows}x{k}")


@pytest.mark.parametrize("rows,rms", [(16384, True), (16384, False), (64, True), (192, False)])
def test_gemv_gate_up_silu_q8_0(gpu, rows, rms):
    """gate|up with silu(gate) * up quantized in the epilogue: the engine
    layout of Q8_0(silu_mul(y[:n], y[n:])), byte for byte, and down on it
    equal to down on the fp32 act (its own fused quantize)."""
    import torch
    k = 2048
    print(f"gate_up_silu_q8_0 rows={rows} rms={rms}", flush=True)
    blocks = C.quantize_q4_0(O.normal_f32((rows, k), 190 + rows, 0.02))
    rng = np.random.default_rng(rows + 7)
    x = (rng.standard_normal(k) * 2).astype(np.float32)
    w = rng.standard_normal(k).astype(np.float32) if rms else None
    h = C.rmsnorm(x, w, 1e-5) if rms else x
    xq, xd = C.quantize_q8_0(h)
    y = C.gemv_q4_0(blocks, k, xq, xd)
    n = rows // 2
    act = C.silu_mul(y[:n], y[n:])
    want = _engine(act)
    got = gpu.gemv_gate_up_silu(dev(blocks), k, dev(x), None if w is None else dev(w), 1e-5, q8=True)
    assert_bytes_equal(host(got), want, f"gate_up_silu_q8_0 {rows}x{k}")
    if n >= 256:
        down = C.quantize_q4_0(O.normal_f32((256, n), 300 + rows, 0.02))
        aq, ad = C.quantize_q8_0(act)
        y_down = gpu.gemv_engine(dev(down), n, got)
        assert_bytes_equal(host(y_down), C.gemv_q4_0(down, n, aq, ad), "down on the quantized act")
    torch.cuda.synchronize()


def test_gemv_gate_up_silu_q8_0_rejects(gpu):
    import torch
    L = gpu.lib()
    w = torch.zeros(64 * 4096 // 32 * 18, dtype=torch.uint8, device="cuda")
    x = torch.zeros(4096, dtype=torch.float32, device="cuda")
    act = torch.zeros(256, dtype=torch.uint8, device="cuda")
    call = lambda rows, k, a=act: L.w4a8_gemv_gate_up_silu_q8_0(w.data_ptr(), x.data_ptr(), None, 1e-5, a.data_ptr(),
                                                                 rows, k, None)
    assert call(64, 4096) == -2        # k = 4096: 16 rows per workgroup, not a Q8_0 block
    assert call(16, 2048) == -2        # one tile per half: no workgroup of four gate tiles
    assert call(48, 2048) == -2        # three tiles per half
    assert call(64, 2048, act[4:]) == -3   # act not 16-byte aligned
    torch.cuda.synchronize()


def test_gemv_gate_up_silu_rejects(gpu):
    import torch
    L = gpu.lib()
    w = torch.zeros(64 * 2048 // 32 * 18, dtype=torch.uint8, device="cuda")
    x = torch.zeros(2048, dtype=torch.float32, device="cuda")
    act = torch.zeros(64, dtype=torch.float32, device="cuda")
    call = lambda rows, k: L.w4a8_gemv_gate_up_silu(w.data_ptr(), x.data_ptr(), None, 1e-5, act.data_ptr(), rows, k, None)
    assert call(63, 2048) == -2        # odd rows
    assert call(12, 2048) == -2        # n = 6 is not a multiple of 8 rows per tile
    assert call(64, 1024) == -2        # k below 2048
    assert call(4, 8192) == -2         # one tile per half at k = 8192: not a multiple of 2
    assert call(12, 8192) == -2        # three tiles per half at k = 8192
    assert call(4, 4096) == -2         # two rows per half at k = 4096: not a whole tile of 4
    assert call(64, 2048) == 0
    torch.cuda.synchronize()
