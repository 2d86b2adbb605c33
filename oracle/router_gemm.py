"""CPU oracle of the router GEMM and the fused router GEMM + TopK + softmax —
TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use
this module, and only as the checker; the product never imports it.

What it restates: ref_topk_softmax of the reference's correctness test
(tests/test_router_fusion_correctness.py:21-25):
    logits = X.float() @ W.float()
    vals, idx = torch.topk(logits, K, dim=-1)
    scores = torch.softmax(vals, dim=-1)
Here the logits are exact sums in float64 of the bf16/fp16 inputs (every
product of two 16-bit floats is exact in float64; the sum's rounding error
is far below fp32's), the top-K order is fixed as in oracle.router (value
descending, ties to the lower expert index), and the softmax is taken in
float64.  A GPU result accumulated in fp32 differs from these logits by
rounding only; tests bound that difference and check the selection
against these logits with that bound.

Pinned by (tests/test_oracle.py): a pure-Python triple-loop matmul on
small exact-integer inputs (logits exact), brute-force top-K on those, the
closed form K == E (a full stable sort), and softmax rows summing to 1.
"""
from __future__ import annotations

from typing import Tuple

import numpy as np


def logits_fp64(X: np.ndarray, W: np.ndarray) -> np.ndarray:
    """X [T, H] @ W [H, E] in float64 (inputs are any float arrays)."""
    return np.asarray(X, dtype=np.float64) @ np.asarray(W, dtype=np.float64)


def topk_order(logits: np.ndarray, k: int) -> np.ndarray:
    """Indices [T, k]: value descending, ties to the lower index (stable)."""
    order = np.argsort(-logits, axis=1, kind="stable")
    return order[:, :k]


def topk_softmax_fp64(logits: np.ndarray, k: int) -> Tuple[np.ndarray, np.ndarray]:
    """(scores float64 [T, k], indices int64 [T, k]) of softmax over the top-k."""
    idx = topk_order(logits, k)
    vals = np.take_along_axis(logits, idx, axis=1)
    e = np.exp(vals - vals[:, :1])
    return e / e.sum(axis=1, keepdims=True), idx


def softmax_at(logits: np.ndarray, idx: np.ndarray) -> np.ndarray:
    """Softmax over the logits at the given indices (row-wise, float64)."""
    vals = np.take_along_axis(logits, np.asarray(idx, dtype=np.int64), axis=1)
    e = np.exp(vals - vals.max(axis=1, keepdims=True))
    return e / e.sum(axis=1, keepdims=True)


def brute_logits(X, W):
    """Pure-Python triple loop (small inputs only)."""
    T, H = len(X), len(X[0])
    E = len(W[0])
    return [[sum(float(X[t][h]) * float(W[h][e]) for h in range(H)) for e in range(E)] for t in range(T)]


def brute_topk(row, k):
    """k indices of the largest values, ties to the lower index, by repeated scans."""
    taken, out = set(), []
    for _ in range(k):
        best = None
        for j, v in enumerate(row):
            if j in taken:
                continue
            if best is None or v > row[best]:
                best = j
        taken.add(best)
        out.append(best)
    return out
