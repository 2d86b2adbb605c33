"""CPU oracle of the fused TopK+softmax router — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use
this module, and only as the checker; the product (tilelang_moe_amd) never
imports it.

What it restates: the reference's PyTorch baseline topk_softmax_fused
(kernels/topk_softmax_baseline.py:39-66):
    v, i = torch.topk(logits, k, dim=-1)          # sorted, descending
    scores = F.softmax(v, dim=-1, dtype=float32)
torch.topk leaves the order of equal values unspecified (its CPU kernel is a
partial sort), so the oracle fixes one: value descending, then column index
ascending (= torch.sort(descending=True, stable=True)); -0.0 equals +0.0 and
NaN ranks above +inf.  On rows without ties at or above the k-th value this
is exactly torch.topk's answer.

Pinned by (tests/test_oracle.py):
  * pure-Python brute force (explicit comparisons, no key mapping) on small
    random rows with ties, +-0.0, +-inf and NaN;
  * torch.topk, bit-exact, on tie-free rows of the golden fixtures
    (tests/golden/), and the closed forms K == N (full stable sort) and
    K == 1 (first argmax, score 1.0);
  * scores: fp64 softmax of the selected values, sum to 1, and the
    reference's convention identity (Conv A-renorm == Conv B,
    tests/test_topk_softmax_conventions.py:58-69 of the reference);
  * Convention A (topk_softmax_conv_a): torch CPU softmax-then-topk of the
    reference baseline on tie-free rows, and all-N scores summing to 1.
"""
from __future__ import annotations

import math
from typing import List, Tuple

import numpy as np


def sortable_keys(x: np.ndarray) -> np.ndarray:
    """Order-preserving uint32 keys of float32 values.

    key(a) > key(b) iff a > b; -0.0 and +0.0 share a key; every NaN gets the
    largest key.  The same mapping the HIP kernels use.
    """
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).copy()
    nan = (u & np.uint32(0x7FFFFFFF)) > np.uint32(0x7F800000)
    u[u == np.uint32(0x80000000)] = 0
    neg = (u & np.uint32(0x80000000)) != 0
    key = np.where(neg, ~u, u | np.uint32(0x80000000)).astype(np.uint32)
    key[nan] = np.uint32(0xFFFFFFFF)
    return key


def topk_order(logits: np.ndarray, k: int) -> np.ndarray:
    """Column indices [M, k] of the k largest values per row (int64), in
    value-descending / index-ascending order."""
    x = np.asarray(logits, dtype=np.float32)
    if x.ndim != 2 or not 1 <= k <= x.shape[1]:
        raise ValueError("need 2-D logits and 1 <= k <= N")
    keys = sortable_keys(x)
    # Stable ascending sort of ~key == descending key with ties by index.
    return np.argsort(~keys, axis=1, kind="stable")[:, :k].astype(np.int64)


def softmax64(v: np.ndarray) -> np.ndarray:
    """fp64 softmax over the last axis, exp(v - max) / sum (Convention B)."""
    v = np.asarray(v, dtype=np.float64)
    m = v[..., :1]
    with np.errstate(invalid="ignore"):  # inf - inf -> NaN, as in torch
        e = np.exp(v - m)
        return e / e.sum(axis=-1, keepdims=True)


def topk_softmax(logits: np.ndarray, k: int) -> Tuple[np.ndarray, np.ndarray]:
    """(scores fp64 [M,k], indices int64 [M,k]) with the oracle's tie rule."""
    x = np.asarray(logits, dtype=np.float32)
    idx = topk_order(x, k)
    vals = np.take_along_axis(x, idx, axis=1)
    return softmax64(vals), idx


def topk_softmax_conv_a(logits: np.ndarray, k: int) -> Tuple[np.ndarray, np.ndarray]:
    """Convention A (topk_softmax_separate, kernels/topk_softmax_baseline.py:15-36):
    the same k indices as topk_softmax, scored by the float64 softmax over
    the whole row.  A row holding NaN scores NaN (as torch.softmax)."""
    x = np.asarray(logits, dtype=np.float32)
    idx = topk_order(x, k)
    xd = x.astype(np.float64)
    with np.errstate(invalid="ignore", over="ignore"):
        m = np.max(np.where(np.isnan(xd), -np.inf, xd), axis=1, keepdims=True)
        e = np.exp(xd - m)
        p = np.take_along_axis(e, idx, 1) / e.sum(axis=1, keepdims=True)
    p[np.isnan(x).any(axis=1)] = np.nan
    return p, idx


def tie_rows(logits: np.ndarray, k: int) -> np.ndarray:
    """Boolean [M]: rows where the k-th largest key also occurs at a rank
    outside the top k or where two of the top k share a value, i.e. rows on
    which torch.topk's order or set may legitimately differ from the oracle's."""
    keys = sortable_keys(np.asarray(logits, dtype=np.float32))
    s = -np.sort(-keys.astype(np.int64), axis=1)
    head = s[:, :k]
    dup_in_head = (np.diff(head, axis=1) == 0).any(axis=1) if k > 1 else np.zeros(len(s), bool)
    boundary = (s[:, k - 1] == s[:, k]) if k < s.shape[1] else np.zeros(len(s), bool)
    return dup_in_head | boundary


# ---------------------------------------------------------------------------
# Brute force for tiny rows: explicit comparisons on Python floats.
# ---------------------------------------------------------------------------
def _greater(a: float, ia: int, b: float, ib: int) -> bool:
    """Is (a, ia) ranked before (b, ib)?  NaN first, then larger value, then
    smaller index; -0.0 == +0.0 falls out of float comparison."""
    an, bn = math.isnan(a), math.isnan(b)
    if an or bn:
        if an and bn:
            return ia < ib
        return an
    if a != b:
        return a > b
    return ia < ib


def topk_bruteforce(row: List[float], k: int) -> List[int]:
    """Repeated selection of the best remaining element; O(N*k)."""
    taken = [False] * len(row)
    out = []
    for _ in range(k):
        best = -1
        for j, v in enumerate(row):
            if taken[j]:
                continue
            if best < 0 or _greater(v, j, row[best], best):
                best = j
        taken[best] = True
        out.append(best)
    return out
