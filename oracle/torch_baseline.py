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
