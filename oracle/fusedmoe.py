"""CPU oracle of the routed-expert FFN (FusedMoE) — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use
this module, and only as the checker; the product never imports it.

What it restates: fusedmoe_pytorch (kernels/fusedmoe_baseline.py:41-168),
in float64:
    logits = x @ router_weight.T
    scores = softmax(logits); w, ids = topk(scores, k)            (Convention A)
    expert(x, g, u, d) = (silu(x @ g.T) * (x @ u.T)) @ d.T
    out = expert(x, shared) + sum_j w[:, j] * expert(x, routed[ids[:, j]])
The top-k order is value descending, ties to the lower expert index (the
reference asks torch.topk for an unsorted set; the sum does not depend on
the order).  `route` may be given to evaluate the FFN under a routing chosen
elsewhere (the GPU's), which separates routing from arithmetic in tests.

Pinned by (tests/test_oracle.py): closed forms — one expert with k = 1 is
the dense SwiGLU FFN; zero router weights route every token to all E
experts with weight 1/E (k = E); the shared part is additive — and the
routing equals oracle.router's Convention A on the same logits.
"""
from __future__ import annotations

from typing import Optional, Tuple

import numpy as np


def silu(a: np.ndarray) -> np.ndarray:
    return a / (1.0 + np.exp(-a))


def expert(x: np.ndarray, g: np.ndarray, u: np.ndarray, d: np.ndarray) -> np.ndarray:
    return (silu(x @ g.T) * (x @ u.T)) @ d.T


def route(x: np.ndarray, router_weight: np.ndarray, k: int) -> Tuple[np.ndarray, np.ndarray]:
    """(weights [T, k], ids [T, k]) of Convention A on float64 logits."""
    logits = x @ router_weight.T
    ids = np.argsort(-logits, axis=1, kind="stable")[:, :k]
    e = np.exp(logits - logits.max(axis=1, keepdims=True))
    p = e / e.sum(axis=1, keepdims=True)
    return np.take_along_axis(p, ids, 1), ids


def fusedmoe(x, router_weight, shared_gate, shared_up, shared_down, routed_gate, routed_up, routed_down, k,
             routing: Optional[Tuple[np.ndarray, np.ndarray]] = None) -> np.ndarray:
    """x [T, Dh] -> out [T, Dh] in float64 (all inputs are cast to float64)."""
    f = lambda a: None if a is None else np.asarray(a, dtype=np.float64)  # noqa: E731
    x, rw = f(x), f(router_weight)
    sg, su, sd = f(shared_gate), f(shared_up), f(shared_down)
    rg, ru, rd = f(routed_gate), f(routed_up), f(routed_down)
    w, ids = route(x, rw, k) if routing is None else (np.asarray(routing[0], np.float64), np.asarray(routing[1]))
    out = expert(x, sg, su, sd) if sg is not None else np.zeros_like(x)
    for e in np.unique(ids):
        rows, slot = np.nonzero(ids == e)
        out[rows] += w[rows, slot][:, None] * expert(x[rows], rg[e], ru[e], rd[e])
    return out
