"""The Python front end refuses a caller's out= tensor that the call would write
past (too short, wrong dtype, not contiguous, another device), and inputs of
the wrong length, before anything is launched: the C ABI sees only
addresses, so a short tensor would otherwise be written out of bounds."""

from __future__ import annotations

import pytest

pytestmark = pytest.mark.gpu

K = 2048
ROWS = 64


@pytest.fixture(scope="module")
def t(gpu):
    import torch
    d = "cuda"
    return {
        "blocks": torch.zeros((ROWS, K // 32 * 18), dtype=torch.uint8, device=d),
        "x": torch.zeros(K, dtype=torch.float32, device=d),
        "xe": torch.zeros(K + K // 8, dtype=torch.uint8, device=d),
        "xq8": torch.zeros(K // 32 * 34, dtype=torch.uint8, device=d),
        "gu": torch.zeros(2 * K, dtype=torch.float32, device=d),
        "short": torch.zeros(ROWS - 1, dtype=torch.float32, device=d),
        "half": torch.zeros(ROWS, dtype=torch.float16, device=d),
        "strided": torch.zeros(2 * ROWS, dtype=torch.float32, device=d)[::2],
        "ws": None,
    }


def _cases(gpu, t):
    import torch
    ws = gpu.argmax_workspace()
    b, x = t["blocks"], t["x"]
    return {
        "gemv_engine": lambda out: gpu.gemv_engine(b, K, t["xe"], out=out),
        "gemv_q4_0_f32": lambda out: gpu.gemv_q4_0_f32(b, K, x, out=out),
        "gemv_q4_0_f32_argmax": lambda out: gpu.gemv_q4_0_f32_argmax(b, K, x, ws, out=out),
        "gemv_rmsnorm": lambda out: gpu.gemv_rmsnorm(b, K, x, x, 1e-5, out=out),
        "gemv_rmsnorm_argmax": lambda out: gpu.gemv_rmsnorm_argmax(b, K, x, x, 1e-5, ws, out=out),
        "gemv_silu_mul": lambda out: gpu.gemv_silu_mul(b, K, t["gu"], out=out),
        "gemv_q8_0_blocks": lambda out: gpu.gemv_q8_0_blocks(b, K, t["xq8"], out=out),
        "gemv_quarters": lambda out: gpu.gemv_quarters([b[:ROWS // 4]] * 4, K, t["xe"], ROWS, out=out),
        "gemm_engine": lambda out: gpu.gemm_engine(b, K, t["xe"].reshape(1, -1), out=out),
        "gemv_gate_up_silu": lambda out: gpu.gemv_gate_up_silu(b, K, x, out=None if out is None else out[: out.numel() // 2]),
    }


@pytest.mark.parametrize("name", ["gemv_engine", "gemv_q4_0_f32", "gemv_q4_0_f32_argmax", "gemv_rmsnorm",
                                  "gemv_rmsnorm_argmax", "gemv_silu_mul", "gemv_q8_0_blocks", "gemv_quarters",
                                  "gemm_engine", "gemv_gate_up_silu"])
def test_bad_out_is_refused(gpu, t, name):
    call = _cases(gpu, t)[name]
    with pytest.raises(ValueError, match="elements"):
        call(t["short"])
    with pytest.raises(TypeError, match="float32"):
        call(t["half"])
    with pytest.raises(ValueError, match="contiguous"):
        call(t["strided"])


def test_quantize_out_is_refused(gpu, t):
    import torch
    with pytest.raises(ValueError, match="elements"):
        gpu.quantize_q8_0_engine(t["x"], out=torch.zeros(K, dtype=torch.uint8, device="cuda"))


def test_bad_inputs_are_refused(gpu, t):
    import torch
    b, x = t["blocks"], t["x"]
    short_w = torch.zeros(K - 256, dtype=torch.float32, device="cuda")
    ws = gpu.argmax_workspace()
    with pytest.raises(ValueError):
        gpu.gemv_rmsnorm_argmax(b, K, x, short_w, 1e-5, ws)
    with pytest.raises(ValueError):
        gpu.gemv_rmsnorm_argmax(b, K, short_w, x, 1e-5, ws)
    with pytest.raises(ValueError):
        gpu.gemv_gate_up_silu(b, K, x, norm_w=short_w)
    with pytest.raises(ValueError):
        gpu.gemv_gate_up_silu(b[:ROWS - 1], K, x)
    with pytest.raises(ValueError):
        gpu.rmsnorm_q8_0_engine(x, short_w, 1e-5)
    with pytest.raises(ValueError):
        gpu.gemv_quarters([b[:2]] * 4, K, t["xe"], ROWS)          # quarters shorter than rows / 4
    with pytest.raises(ValueError):
        gpu.gemv_quarters([b[:ROWS // 4]] * 4, K, t["xe"][:-16], ROWS)


def test_good_out_still_works(gpu, t):
    import torch
    y = torch.full((ROWS + 5,), float("nan"), dtype=torch.float32, device="cuda")
    got = gpu.gemv_q4_0_f32(t["blocks"], K, t["x"], out=y)
    torch.cuda.synchronize()
    assert got.data_ptr() == y.data_ptr()
    assert bool(torch.all(y[:ROWS] == 0)) and bool(torch.all(torch.isnan(y[ROWS:])))
