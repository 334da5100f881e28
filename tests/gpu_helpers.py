"""Shared helpers of the GPU parity tests: device transfer, poisoned outputs and
row-by-row byte comparison (the discipline of hls/gemv2/tb_gemv2.cpp:50-70 and
board/kv260gemv/bench_gemv2.c:63-71)."""

from __future__ import annotations

import numpy as np

POISON = 0xAA


def dev(a: np.ndarray):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t) -> np.ndarray:
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy()


def poisoned_f32(shape):
    """A float32 device tensor whose every byte is 0xAA, so an unwritten row shows."""
    import torch
    shape = (shape,) if isinstance(shape, int) else tuple(shape)
    n = int(np.prod(shape))
    return torch.full((4 * n,), POISON, dtype=torch.uint8, device="cuda").view(torch.float32).reshape(shape)


def assert_bytes_equal(got: np.ndarray, want: np.ndarray, what: str = "y", show: int = 8) -> None:
    """Byte-exact comparison; on failure print the first differing rows."""
    g = np.ascontiguousarray(got).reshape(-1)
    w = np.ascontiguousarray(want).reshape(-1)
    assert g.dtype == w.dtype and g.shape == w.shape, (g.dtype, w.dtype, g.shape, w.shape)
    gb = g.view(np.uint8).reshape(g.shape[0], -1)
    wb = w.view(np.uint8).reshape(w.shape[0], -1)
    bad = np.nonzero(np.any(gb != wb, axis=1))[0]
    if bad.size:
        lines = [f"{what}: {bad.size}/{g.shape[0]} rows differ"]
        for r in bad[:show]:
            lines.append(f"  row {r}: got {g[r]!r} want {w[r]!r}")
        raise AssertionError("\n".join(lines))
