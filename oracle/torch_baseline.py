"""The reference's CPU PyTorch path, restated — TEST/BASELINE INFRASTRUCTURE.

Used by bench.py's cpu_baseline leg (timed on the host cores) and by tests
that report how torch.topk orders ties.  Never imported by the product.

  topk_softmax_fused   kernels/topk_softmax_baseline.py:39-66  (Convention B)
  topk_softmax_separate / conv_a_renorm
                       kernels/topk_softmax_baseline.py:15-36, :223-237
  grouped_gemm_loop    kernels/grouped_gemm_baseline.py:14-57
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


def topk_softmax_fused(logits: torch.Tensor, k: int):
    v, i = torch.topk(logits, k, dim=-1)
    return F.softmax(v, dim=-1, dtype=torch.float32), i


def topk_softmax_separate(logits: torch.Tensor, k: int):
    s = F.softmax(logits, dim=-1, dtype=torch.float32)
    return torch.topk(s, k, dim=-1)


def topk_softmax_conv_a_renorm(logits: torch.Tensor, k: int):
    s, i = topk_softmax_separate(logits, k)
    return s / s.sum(dim=-1, keepdim=True), i


def grouped_gemm_loop(X: torch.Tensor, W: torch.Tensor, expert_indices: torch.Tensor) -> torch.Tensor:
    R = X.shape[0]
    E, I, _ = W.shape
    Y = torch.zeros(R, I, dtype=X.dtype, device=X.device)
    for e in range(E):
        mask = expert_indices == e
        if not mask.any():
            continue
        Y[mask] = X[mask] @ W[e].T
    return Y


def fusedmoe_torch(x, router_weight, shared_gate, shared_up, shared_down, routed_gate, routed_up, routed_down,
                   k: int):
    """The reference's fusedmoe_pytorch (kernels/fusedmoe_baseline.py:41-168) on
    flat tokens x [T, Dh], restated: torch matmuls in the input dtype, a
    per-expert loop and scatter_reduce.  Used as the torch GPU baseline."""
    logits = x @ router_weight.T
    scores = F.softmax(logits, dim=-1)
    w, ids = torch.topk(scores, k, dim=-1, sorted=False)

    def ffn(t, g, u, d):
        return (F.silu(t @ g.T) * (t @ u.T)) @ d.T

    out = ffn(x, shared_gate, shared_up, shared_down)
    flat, fw = ids.view(-1), w.view(-1, 1)
    order = flat.argsort()
    counts = flat.bincount(minlength=routed_gate.shape[0]).cpu().tolist()
    tok = order // k
    cache = torch.zeros_like(x)
    start = 0
    for e, c in enumerate(counts):
        if c == 0:
            continue
        rows = tok[start:start + c]
        y = ffn(x[rows], routed_gate[e], routed_up[e], routed_down[e]) * fw[order[start:start + c]]
        cache.scatter_reduce_(0, rows.view(-1, 1).expand(-1, x.shape[1]), y, reduce="sum")
        start += c
    return out + cache
