"""The sampler's candidates on the GPU (w4a8_topk) against the oracle's
restatement of the reference's insertion sort (board/tp/tp_llama.cpp:894-909):
values bit for bit and indices, at the LM-head size and its ragged and
maximum sizes, with heavy ties, +-0, -1e30 / -inf (never admitted) and fewer
admitted values than k; the first candidate equals the fused argmax of the
same logits; bad arguments are refused before any launch."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

import c_oracle as C
from gpu_helpers import dev, host

pytestmark = pytest.mark.gpu

F32 = np.float32


def _logits(n, seed, grid=0):
    rng = np.random.default_rng(seed)
    y = (rng.standard_normal(n) * 3).astype(np.float32)
    if grid:
        y = (np.round(y * grid) / grid).astype(np.float32)
    return y


def _check(gpu, y, k, label):
    vals, idx = gpu.topk(dev(y), k)
    want_v, want_i = C.topk(y, k)
    got_v, got_i = host(vals), host(idx)
    assert np.array_equal(got_i, want_i), (label, got_i[:8], want_i[:8])
    assert np.array_equal(got_v.view(np.uint32), want_v.view(np.uint32)), label


@pytest.mark.parametrize("n,k,seed,grid", [(128256, 40, 0, 0), (128256, 64, 1, 0), (128256, 1, 2, 0),
                                           (128256, 64, 3, 2), (262144, 64, 4, 8), (1000, 17, 5, 1),
                                           (1025, 64, 6, 0), (64, 64, 7, 0)])
def test_topk_matches_the_oracle(gpu, n, k, seed, grid):
    print(f"topk n={n} k={k} seed={seed} grid={grid}", flush=True)
    _check(gpu, _logits(n, seed, grid), k, f"n={n} k={k}")


def test_special_values(gpu):
    y = _logits(5000, 11, 1)
    y[:50] = F32(-1e30)
    y[50:100] = -np.inf
    y[100:110] = 0.0
    y[110:120] = -0.0
    y[200] = np.inf
    _check(gpu, y, 64, "specials")
    z = np.full(3000, F32(-1e30), dtype=np.float32)        # fewer admitted values than k
    z[[7, 1500, 2999]] = [1.0, -2.0, 1.0]
    z[[3, 4]] = [-np.inf, -5e30]
    _check(gpu, z, 64, "few admitted")
    _check(gpu, np.zeros(4096, dtype=np.float32), 64, "all zero")


def test_first_candidate_is_the_fused_argmax(gpu):
    import q4_0_oracle as O
    rows, k = 128256, 2048
    blocks = C.quantize_q4_0(O.normal_f32((rows, k), 21, 0.02))
    x = O.normal_f32(k, 22)
    ws = gpu.argmax_workspace()
    y, best = gpu.gemv_q4_0_f32_argmax(dev(blocks), k, dev(x), ws)
    vals, idx = gpu.topk(y, 40)
    assert int(host(idx)[0]) == int(host(best)[0])
    _check(gpu, host(y), 40, "lm head logits")


def test_rejections(gpu):
    import torch
    L = gpu.lib()
    y = torch.zeros(1000, dtype=torch.float32, device="cuda")
    v = torch.empty(64, dtype=torch.float32, device="cuda")
    i = torch.empty(64, dtype=torch.int32, device="cuda")
    ws = torch.empty(L.w4a8_topk_workspace_bytes(262144), dtype=torch.uint8, device="cuda")
    nbytes = ws.numel()
    call = lambda n, k, wsb=nbytes, yp=y.data_ptr(): L.w4a8_topk(yp, n, k, v.data_ptr(), i.data_ptr(),
                                                                 ws.data_ptr(), wsb, None)
    assert call(1000, 0) == -2 and call(1000, 65) == -2 and call(0, 8) == -2 and call(262145, 8) == -2
    assert call(1000, 8, wsb=L.w4a8_topk_workspace_bytes(1000) - 1) == -2
    assert call(1000, 8, yp=y.data_ptr() + 2) == -3
    assert L.w4a8_topk(None, 1000, 8, v.data_ptr(), i.data_ptr(), ws.data_ptr(), nbytes, None) == -1
    assert call(1000, 8) == 0
    torch.cuda.synchronize()


def _check_nan(gpu, y, k, label):
    """Indices equal, NaN slots in the same places, every other value bit for bit."""
    vals, idx = gpu.topk(dev(y), k)
    want_v, want_i = C.topk(y, k)
    got_v, got_i = host(vals), host(idx)
    assert np.array_equal(got_i, want_i), (label, got_i[:8], want_i[:8])
    assert np.array_equal(np.isnan(got_v), np.isnan(want_v)), label
    ok = ~np.isnan(want_v)
    assert np.array_equal(got_v[ok].view(np.uint32), want_v[ok].view(np.uint32)), label
    # A NaN slot holds y's own NaN, bit for bit.
    for j in np.flatnonzero(~ok):
        assert got_v[j:j + 1].view(np.uint32)[0] == y[got_i[j]:got_i[j] + 1].view(np.uint32)[0], label


@pytest.mark.parametrize("n,k,seed,where", [(128256, 40, 20, "spread"), (128256, 64, 21, "last"),
                                            (128256, 1, 22, "spread"), (5000, 17, 23, "runs"),
                                            (1025, 64, 24, "first"), (64, 64, 25, "spread"),
                                            (262144, 40, 26, "late")])
def test_nan_logits_follow_the_reference_loop(gpu, n, k, seed, where):
    """NaN logits take the last slot and let the next logit in, as the
    reference's loop does (tp_llama.cpp:902-908), wherever they stand."""
    print(f"topk NaN n={n} k={k} seed={seed} where={where}", flush=True)
    rng = np.random.default_rng(seed)
    y = _logits(n, seed, grid=2 if where == "runs" else 0)
    if where == "spread":
        y[rng.integers(0, n, 12)] = np.nan
        y[rng.integers(0, n, 6)] = -np.inf
    elif where == "last":
        y[-1] = np.nan
    elif where == "first":
        y[0] = np.nan
        y[1] = -np.inf
    elif where == "runs":
        y[100:104] = np.nan
        y[2000:2002] = [np.nan, -np.inf]
        y[4999] = np.nan
    else:
        y[n - 5000] = np.nan
        y[n - 4999] = F32(-3e30)
    y[rng.integers(0, n, 2)] = F32(np.frombuffer(np.uint32(0xFFC00123).tobytes(), np.float32)[0])  # a payload
    _check_nan(gpu, y, k, f"n={n} k={k} {where}")
    clean = y.copy()
    clean[np.isnan(clean)] = 0.0
    _check(gpu, clean, k, f"n={n} k={k} without NaN")          # the parallel path again afterwards
