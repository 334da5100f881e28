"""Pinning the oracle's restatement of the reference's sampler candidates
(board/tp/tp_llama.cpp:894-909: an insertion sort of the k best logits of a
shard, slots starting at {-1e30, 0}). It is pinned by hand-worked cases and
by an independent definition: for inputs without NaN, the candidates are the
admitted values (v > -1e30) sorted by value descending and then by index,
first k, padded with {-1e30, 0}. A plausible slip in the loop (the larger
index first among equals, admitting a value equal to the last slot, a
sentinel other than -1e30) fails one of them."""

from __future__ import annotations

import numpy as np
import pytest

import c_oracle as C

F32 = np.float32


def by_definition(y, k):
    y = np.asarray(y, dtype=np.float32)
    cand = [(-float(v), i) for i, v in enumerate(y) if v > F32(-1e30)]
    cand.sort()                      # value descending (-0 == +0), then index ascending
    cand = cand[:k]
    vals = np.full(k, F32(-1e30), dtype=np.float32)
    idx = np.zeros(k, dtype=np.int32)
    for j, (_, i) in enumerate(cand):
        vals[j] = y[i]
        idx[j] = i
    return vals, idx


def same(a, b):
    return np.array_equal(a[0].view(np.uint32), b[0].view(np.uint32)) and np.array_equal(a[1], b[1])


@pytest.mark.parametrize("y,k,vals,idx", [
    ([1, 3, 3, 2], 2, [3, 3], [1, 2]),                      # equal values: the smaller index first
    ([1, 3, 3, 2], 3, [3, 3, 2], [1, 2, 3]),
    ([2, 1, 1, 1], 2, [2, 1], [0, 1]),                      # a tie at the last slot keeps the earlier index
    ([-1e30, -np.inf, 5], 3, [5, -1e30, -1e30], [2, 0, 0]),  # -1e30 and below are never admitted
    ([-0.0, 0.0], 2, [-0.0, 0.0], [0, 1]),                  # -0 equals +0: index order, own bits
    ([7], 1, [7], [0]),
])
def test_hand_worked(y, k, vals, idx):
    got = C.topk(np.array(y, dtype=np.float32), k)
    want = (np.array(vals, dtype=np.float32), np.array(idx, dtype=np.int32))
    assert same(got, want), (got, want)


@pytest.mark.parametrize("n,k,seed,grid", [(128256, 40, 0, 0), (128256, 64, 1, 4), (5000, 1, 2, 2),
                                           (3000, 64, 3, 1), (70, 64, 4, 0)])
def test_loop_matches_definition(n, k, seed, grid):
    rng = np.random.default_rng(seed)
    y = (rng.standard_normal(n) * 3).astype(np.float32)
    if grid:
        y = (np.round(y * grid) / grid).astype(np.float32)  # many equal values
    y[rng.integers(0, n, max(1, n // 100))] = F32(-1e30)
    y[rng.integers(0, n, max(1, n // 200))] = -np.inf
    assert same(C.topk(y, k), by_definition(y, k))


NAN = np.nan


@pytest.mark.parametrize("y,k,vals,idx", [
    # A NaN is admitted (v <= NaN is false) into the last slot, evicting the
    # k-th candidate held then; the next logit enters whatever its value.
    ([3, 2, NAN, 1], 2, [3, 1], [0, 3]),                    # 2 is lost to the NaN, 1 takes its place
    ([1, NAN, 0.5], 2, [1, 0.5], [0, 2]),
    ([5, 4, NAN], 2, [5, NAN], [0, 2]),                     # a NaN at the end stays in the last slot
    ([NAN, -np.inf], 2, [-1e30, -np.inf], [0, 1]),          # -inf enters after a NaN, below the sentinel
    ([NAN, -np.inf, 2], 2, [2, -1e30], [2, 0]),             # ... and is the one the next value evicts
    ([4, NAN, NAN, 3], 3, [4, 3, -1e30], [0, 3, 0]),        # each NaN replaces the last slot again
    ([NAN, 9, 8], 1, [9], [1]),                             # k = 1: the NaN is the only slot, then 9
    ([2, 7, NAN, 6, 5], 3, [7, 6, 5], [1, 3, 4]),
])
def test_hand_worked_nan(y, k, vals, idx):
    """Worked by hand through tp_llama.cpp:902-908 with IEEE comparisons."""
    got = C.topk(np.array(y, dtype=np.float32), k)
    want = (np.array(vals, dtype=np.float32), np.array(idx, dtype=np.int32))
    assert np.array_equal(got[1], want[1]), (got, want)
    assert np.array_equal(np.isnan(got[0]), np.isnan(want[0]))
    ok = ~np.isnan(want[0])
    assert np.array_equal(got[0][ok].view(np.uint32), want[0][ok].view(np.uint32)), (got, want)


def test_first_candidate_is_the_argmax_scan():
    rng = np.random.default_rng(9)
    y = (np.round(rng.standard_normal(20000) * 2) / 2).astype(np.float32)
    best = 0
    for i in range(1, y.size):                              # tp_llama.cpp:879-880
        if y[i] > y[best]:
            best = i
    assert C.topk(y, 40)[1][0] == best
