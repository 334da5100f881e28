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


def _capture_and_replay(gpu, n, k, seeds):
    """w4a8_topk_no_alloc captured into a graph once, then replayed on each
    seed's logits copied into the captured input (eager work and a
    synchronization between replays); every replay against w4a8_topk."""
    import torch
    L = gpu.lib()
    y = torch.zeros(n, dtype=torch.float32, device="cuda")
    vals = torch.full((k,), float("nan"), dtype=torch.float32, device="cuda")
    idx = torch.full((k,), -7, dtype=torch.int32, device="cuda")
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        rc = L.w4a8_topk_no_alloc(y.data_ptr(), n, k, vals.data_ptr(), idx.data_ptr(),
                                  torch.cuda.current_stream().cuda_stream)
    assert rc == 0, gpu.strerror(rc)
    for seed in seeds:
        y.copy_(dev(_logits(n, seed)))
        vals.fill_(float("nan"))
        idx.fill_(-7)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        want_v, want_i = gpu.topk(y, k)
        assert np.array_equal(host(idx), host(want_i)), (n, k, seed)
        assert np.array_equal(host(vals).view(np.uint32), host(want_v).view(np.uint32)), (n, k, seed)


def test_no_alloc_captured_in_a_graph(gpu):
    print("topk_no_alloc under capture, n=128256 k=40", flush=True)
    _capture_and_replay(gpu, 128256, 40, (41, 42, 43))


def test_no_alloc_first_call_under_capture():
    """In a fresh process, the first call on the device is the captured one
    (the array's address is looked up inside the capture)."""
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    code = (
        "import sys; sys.path[:0] = [%r, %r, %r]\n"
        "import torch, kv260gemv, test_zz_no_alloc as t\n"
        "kv260gemv.require_device()\n"
        "t._capture_and_replay(kv260gemv, 5000, 17, (51, 52))\n"
        "print('replays ok', flush=True)\n"
    ) % (os.path.join(root, "tests"), os.path.join(root, "llm-kv260_amd"), os.path.join(root, "oracle"))
    p = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=300)
    assert p.returncode == 0 and "replays ok" in p.stdout, p.stdout[-2000:] + p.stderr[-4000:]
