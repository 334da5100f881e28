"""The LM head's greedy pick fused into its GEMV (w4a8_gemv_f32_argmax): y is
byte-identical to the plain fused GEMV, and the index is the reference's scan
over y (board/tp/tp_llama.cpp:879-880: best = 0, then "if (y[i] > y[best])
best = i"), restated here in Python over the oracle's y, on the LM-head shape,
on constructed ties, +-0, NaN rows (at row 0 too) and K < 2048 (several row
passes per tile), with the workspace reused call after call."""

from __future__ import annotations

import numpy as np
import pytest

import c_oracle as C
import q4_0_oracle as O
from gpu_helpers import assert_bytes_equal, dev, host

pytestmark = pytest.mark.gpu


def scan_argmax(y: np.ndarray) -> int:
    best = 0
    for i in range(1, len(y)):
        if y[i] > y[best]:
            best = i
    return best


def _blocks(rows, k, seed):
    return C.quantize_q4_0(O.normal_f32((rows, k), seed, 0.02))


def _check(gpu, ws, blocks, k, x, label):
    rows = blocks.shape[0]
    xq, xd = C.quantize_q8_0(x)
    want = C.gemv_q4_0(blocks, k, xq, xd)
    y, best = gpu.gemv_q4_0_f32_argmax(dev(blocks), k, dev(x), ws)
    assert_bytes_equal(host(y), want, label)
    expect = scan_argmax(want)
    assert int(host(best)[0]) == expect, (label, int(host(best)[0]), expect)


def test_lm_head_shape(gpu):
    ws = gpu.argmax_workspace()
    blocks = _blocks(128256, 2048, 30)
    for seed in (31, 32, 33):
        _check(gpu, ws, blocks, 2048, O.normal_f32((1, 2048), seed)[0], f"lm_head x{seed}")


@pytest.mark.parametrize("rows,k", [(1, 256), (3000, 512), (1000, 2048), (4097, 8192), (20000, 1024)])
def test_shapes_and_ties(gpu, rows, k):
    ws = gpu.argmax_workspace()
    blocks = _blocks(rows, k, 40 + rows)
    x = O.normal_f32((1, k), 41)[0]
    _check(gpu, ws, blocks, k, x, f"{rows}x{k}")
    if rows > 10:
        # The largest row copied to a lower and a higher index: equal values,
        # the lowest of the three wins.
        xq, xd = C.quantize_q8_0(x)
        top = int(np.argmax(C.gemv_q4_0(blocks, k, xq, xd)))
        tied = blocks.copy()
        tied[rows // 3] = blocks[top]
        tied[rows - 1] = blocks[top]
        _check(gpu, ws, tied, k, x, f"{rows}x{k} ties")


def test_zeros_and_nans(gpu):
    ws = gpu.argmax_workspace()
    rows, k = 600, 2048
    x = O.normal_f32((1, k), 50)[0]
    zero = C.quantize_q4_0(np.zeros((rows, k), dtype=np.float32))     # every y is +-0: row 0 wins
    _check(gpu, ws, zero, k, x, "zeros")
    blocks = _blocks(rows, k, 51)
    nan5 = blocks.copy()
    nan5[5, 0:2] = np.frombuffer(np.float16(np.nan).tobytes(), dtype=np.uint8)
    _check(gpu, ws, nan5, k, x, "NaN at row 5")
    nan0 = blocks.copy()
    nan0[0, 0:2] = np.frombuffer(np.float16(np.nan).tobytes(), dtype=np.uint8)
    _check(gpu, ws, nan0, k, x, "NaN at row 0")
    _check(gpu, ws, blocks, k, x, "after NaNs")


def test_workspace_is_checked(gpu):
    import torch
    blocks = dev(_blocks(64, 256, 60))
    x = dev(O.normal_f32((1, 256), 61)[0])
    small = torch.zeros(8, dtype=torch.uint8, device="cuda")
    with pytest.raises(gpu.W4A8Error):
        gpu.gemv_q4_0_f32_argmax(blocks, 256, x, small)
