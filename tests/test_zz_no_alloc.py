"""w4a8_topk_no_alloc (the top-k candidates with the library's own device
array for the stage-1 lists, for callers that cannot allocate) against
w4a8_topk, the entry point it is a variant of: values bit for bit and
indices, on two calls in a row, the second with a smaller input (the array
keeps the first call's lists, which the second must not see), then a third
with NaN logits. Sizes beyond the array are refused before any launch."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

from gpu_helpers import dev, host

pytestmark = pytest.mark.gpu


def _logits(n, seed):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal(n) * 3).astype(np.float32)


def _no_alloc(gpu, y, k):
    import torch
    vals = torch.full((k,), float("nan"), dtype=torch.float32, device=y.device)
    idx = torch.full((k,), -7, dtype=torch.int32, device=y.device)
    rc = gpu.lib().w4a8_topk_no_alloc(y.data_ptr(), y.numel(), k, vals.data_ptr(), idx.data_ptr(),
                                      torch.cuda.current_stream().cuda_stream)
    assert rc == 0, gpu.strerror(rc)
    torch.cuda.synchronize()
    return host(vals), host(idx)


@pytest.mark.parametrize("calls", [((262144, 64, 31), (128256, 40, 32), (5000, 17, 33))])
def test_no_alloc_matches_topk(gpu, calls):
    for n, k, seed in calls:
        print(f"topk_no_alloc n={n} k={k} seed={seed}", flush=True)
        y_host = _logits(n, seed)
        if seed == 33:
            y_host[[10, 2000, 4999]] = np.nan
        y = dev(y_host)
        want_v, want_i = gpu.topk(y, k)
        got_v, got_i = _no_alloc(gpu, y, k)
        want_v, want_i = host(want_v), host(want_i)
        assert np.array_equal(got_i, want_i), (n, k, got_i[:8], want_i[:8])
        assert np.array_equal(got_v.view(np.uint32), want_v.view(np.uint32)), (n, k)


def test_no_alloc_refuses_sizes_beyond_its_array(gpu):
    import torch
    L = gpu.lib()
    y = torch.zeros(262145, dtype=torch.float32, device="cuda")
    vals = torch.zeros(64, dtype=torch.float32, device="cuda")
    idx = torch.zeros(64, dtype=torch.int32, device="cuda")
    s = torch.cuda.current_stream().cuda_stream
    assert L.w4a8_topk_no_alloc(y.data_ptr(), 262145, 40, vals.data_ptr(), idx.data_ptr(), s) == -2
    assert L.w4a8_topk_no_alloc(y.data_ptr(), 1000, 65, vals.data_ptr(), idx.data_ptr(), s) == -2
    assert L.w4a8_topk_no_alloc(None, 1000, 40, vals.data_ptr(), idx.data_ptr(), s) == -1
    assert L.w4a8_topk_no_alloc(y.data_ptr() + 2, 1000, 40, vals.data_ptr(), idx.data_ptr(), s) == -3
