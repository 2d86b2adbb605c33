"""Write the golden fixtures of tests/golden/*.npz.

Inputs are seeded (torch.Generator().manual_seed); expected outputs come from
torch's CPU operators — torch.topk + F.softmax (the reference's Convention-B
baseline, kernels/topk_softmax_baseline.py:39-66) and the per-expert matmul
loop of kernels/grouped_gemm_baseline.py:14-57 — i.e. from the torch library,
not from the reference's code, which is not imported.  Each router fixture
also stores the canonical (value desc, index asc) order computed here with
torch.sort(stable=True), independent of the numpy oracle.

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import os

import numpy as np
import torch
import torch.nn.functional as F

HERE = os.path.dirname(os.path.abspath(__file__))


def _bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def router_fixture(name: str, logits: torch.Tensor, k: int) -> None:
    x = logits.float()
    v, i = torch.topk(x, k, dim=-1)
    s = F.softmax(v, dim=-1, dtype=torch.float32)
    # Canonical order: stable descending sort (ties by ascending index).
    canon = torch.sort(x, dim=-1, descending=True, stable=True).indices[:, :k]
    cv = torch.gather(x, 1, canon).double()
    s64 = torch.softmax(cv, dim=-1)
    payload = dict(logits=x.numpy(), k=np.int64(k), torch_idx=i.numpy(), torch_scores=s.numpy(),
                   canon_idx=canon.numpy(), canon_scores64=s64.numpy())
    if logits.dtype == torch.bfloat16:
        payload["logits_bf16_bits"] = _bf16_bits(logits)
    np.savez_compressed(os.path.join(HERE, f"{name}.npz"), **payload)


def gemm_fixture(name: str, T: int, H: int, I: int, E: int, ids: torch.Tensor, seed: int) -> None:
    g = torch.Generator().manual_seed(seed)
    X = torch.randn(T, H, generator=g).to(torch.bfloat16)
    W = (0.02 * torch.randn(E, I, H, generator=g)).to(torch.bfloat16)
    Yf = torch.zeros(T, I)
    Yb = torch.zeros(T, I, dtype=torch.bfloat16)
    for e in range(E):
        m = ids == e
        if m.any():
            Yf[m] = X[m].float() @ W[e].float().T
            Yb[m] = X[m] @ W[e].T
    np.savez_compressed(os.path.join(HERE, f"{name}.npz"), X_bits=_bf16_bits(X), W_bits=_bf16_bits(W),
                        ids=ids.numpy().astype(np.int64), Y_fp32=Yf.numpy(), Y_bf16_bits=_bf16_bits(Yb),
                        E=np.int64(E))


def main() -> None:
    g = torch.Generator().manual_seed(1234)
    router_fixture("router_f32_32x128_k6", torch.randn(32, 128, generator=g), 6)
    router_fixture("router_f32_8x4096_k256", torch.randn(8, 4096, generator=g), 256)
    router_fixture("router_bf16_256x64_k6", torch.randn(256, 64, generator=g).to(torch.bfloat16), 6)
    router_fixture("router_bf16_256x256_k8", torch.randn(256, 256, generator=g).to(torch.bfloat16), 8)
    # Degenerate rows: all equal, signed zeros, infinities.
    sp = torch.randn(6, 96, generator=g)
    sp[0] = 0.5
    sp[1] = 0.0
    sp[1, ::2] = -0.0
    sp[2, 10] = float("inf")
    sp[2, 20] = float("inf")
    sp[3] = float("-inf")
    sp[3, 5] = 1.0
    sp[4, :48] = 2.0
    sp[5] = sp[5].round()
    router_fixture("router_special_6x96_k8", sp, 8)

    ids_small = torch.randint(0, 8, (64,), generator=g)
    gemm_fixture("gemm_small_64x64x32_e8", 64, 64, 32, 8, ids_small, 7)
    ids_skew = torch.tensor([0] * 40 + [3] * 9 + [15] * 2 + [5] * 13, dtype=torch.int64)
    ids_skew = ids_skew[torch.randperm(64, generator=g)]
    gemm_fixture("gemm_skew_64x128x48_e16", 64, 128, 48, 16, ids_skew, 8)
    print("fixtures written to", HERE)


if __name__ == "__main__":
    main()
