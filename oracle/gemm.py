"""CPU oracle of the expert grouped GEMM and its routing sort — TEST
INFRASTRUCTURE ONLY (tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg; never imported by the product).

Restates grouped_gemm_loop (kernels/grouped_gemm_baseline.py:14-57):
    Y = zeros(R, I)
    for e in range(E):
        mask = expert_indices == e
        Y[mask] = X[mask] @ W[e].T
with fp32 (here fp64) accumulation; rows whose id lies outside [0, E) stay
zero.  ``topk > 1`` reads token r // topk for routed row r, which equals the
reference applied to X.repeat_interleave(topk, 0).

The routing sort restates the host-side metadata of grouped_gemm_tilelang_v2
(kernels/grouped_gemm_tilelang.py:700-725: argsort, bincount, exclusive
offsets) with one fixed order inside each expert segment: ascending row.

Pinned by (tests/test_oracle.py): a triple-loop brute force on tiny shapes,
the per-row closed form against numpy's matmul, linearity in X, and a
pure-Python counting sort for route_sort.
"""
from __future__ import annotations

from typing import Tuple

import numpy as np


def _bucket(ids: np.ndarray, E: int) -> np.ndarray:
    ids = np.asarray(ids).reshape(-1).astype(np.int64)
    return np.where((ids >= 0) & (ids < E), ids, E)


def route_sort(ids: np.ndarray, E: int) -> Tuple[np.ndarray, np.ndarray, np.ndarray]:
    """(counts [E], offsets [E+1], sorted_rows [R]) as int32; invalid ids last."""
    b = _bucket(ids, E)
    counts_all = np.bincount(b, minlength=E + 1)
    offsets = np.zeros(E + 1, dtype=np.int64)
    offsets[1:] = np.cumsum(counts_all[:E])
    sorted_rows = np.argsort(b, kind="stable")
    return counts_all[:E].astype(np.int32), offsets.astype(np.int32), sorted_rows.astype(np.int32)


def route_sort_bruteforce(ids, E: int):
    """Pure-Python counting sort (tiny inputs)."""
    ids = [int(v) for v in np.asarray(ids).reshape(-1)]
    buckets = [[] for _ in range(E + 1)]
    for r, v in enumerate(ids):
        buckets[v if 0 <= v < E else E].append(r)
    counts = [len(b) for b in buckets[:E]]
    offsets = [0]
    for c in counts:
        offsets.append(offsets[-1] + c)
    return counts, offsets, [r for b in buckets for r in b]


def grouped_gemm(X: np.ndarray, W: np.ndarray, ids: np.ndarray, topk: int = 1) -> np.ndarray:
    """Y [R, I] in fp64 for X [T, H], W [E, I, H], ids [T*topk]."""
    X = np.asarray(X, dtype=np.float64)
    W = np.asarray(W, dtype=np.float64)
    ids = np.asarray(ids).reshape(-1).astype(np.int64)
    E, I, _ = W.shape
    R = ids.shape[0]
    Y = np.zeros((R, I), dtype=np.float64)
    for e in range(E):
        rows = np.nonzero(ids == e)[0]
        if rows.size:
            Y[rows] = X[rows // topk] @ W[e].T
    return Y


def grouped_gemm_bruteforce(X, W, ids, topk: int = 1):
    """Triple loop, tiny shapes only."""
    X = np.asarray(X, dtype=np.float64)
    W = np.asarray(W, dtype=np.float64)
    ids = np.asarray(ids).reshape(-1)
    E, I, H = W.shape
    Y = np.zeros((len(ids), I))
    for r, e in enumerate(ids):
        if not 0 <= e < E:
            continue
        for j in range(I):
            acc = 0.0
            for h in range(H):
                acc += X[r // topk, h] * W[e, j, h]
            Y[r, j] = acc
    return Y
