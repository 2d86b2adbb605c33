"""Fused TopK + softmax router (drop-in for the reference's topk_softmax).

Reference interface (kernels/topk_softmax_tilelang.py):
  topk_softmax_best(logits, k) -> (scores fp32 [M,k], indices int32 [M,k])   :1103-1135
  topk_softmax_bitonic(logits, k)                                            :895-921
  topk_softmax_selection(logits, k)   (alias topk_softmax_sonic)             :983-1004
  topk_radix_tilelang(logits, topk) -> indices int32 [M,topk]                :205-235
  _select_strategy(num_experts, k)                                           :1056-1100

Semantics follow the reference's PyTorch baseline topk_softmax_fused
(kernels/topk_softmax_baseline.py:39-66): the k largest logits of each row in
descending order, softmax over those k values in fp32.  Ties are broken by
ascending column index (torch.sort(stable=True) order); -0.0 == +0.0; NaN
ranks above +inf.  Every call runs a hand-written gfx950 kernel from
libmoe_hip.so on the tensor's device and current stream; CPU tensors are
rejected.
"""
from __future__ import annotations

from typing import Tuple

import torch

from .. import _lib

_IDX_DTYPES = {torch.int32: _lib.MOE_I32, torch.int64: _lib.MOE_I64}
_ALGOS = {"auto": _lib.MOE_TOPK_AUTO, "bitonic": _lib.MOE_TOPK_BITONIC,
          "selection": _lib.MOE_TOPK_SELECTION, "radix": _lib.MOE_TOPK_RADIX}
_ALGO_NAMES = {v: k for k, v in _ALGOS.items()}


def select_strategy(num_experts: int, k: int) -> str:
    """Name of the algorithm ``topk_softmax`` uses for rows of ``num_experts``.

    Thresholds of the reference README (README.md:120-122): N<=64 bitonic,
    65..512 selection, N>512 radix.  (The reference code's _select_strategy,
    kernels/topk_softmax_tilelang.py:1056-1100, agrees on every BASELINE shape.)
    """
    return _ALGO_NAMES[_lib.lib().moe_topk_select_algo(int(num_experts), int(k))]


_NEED_WORKSPACE = -100  # the binding's code for "workspace too small, nothing launched"
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None) or (
    lambda i: torch.cuda.current_stream(i).cuda_stream)


def _run(logits: torch.Tensor, k, algo: int, with_scores: bool,
         index_dtype: torch.dtype = torch.int32, score_mode: int = _lib.MOE_SCORES_TOPK):
    """One call of moe_topk_softmax_ex through the torch binding, which
    checks the arguments (ValueError as in the reference), allocates the
    outputs and launches on the current stream."""
    if not isinstance(logits, torch.Tensor):
        raise TypeError("logits must be a torch.Tensor")
    if k.__class__ is not int:
        k = int(k.item()) if isinstance(k, torch.Tensor) else int(k)
    fast = _lib.fast or (_lib.lib(), _lib.fast)[1]
    idx64 = index_dtype is torch.int64
    rc, need, scores, indices = fast.topk_softmax(logits, k, algo, with_scores, idx64, score_mode)
    if rc == _NEED_WORKSPACE:
        didx = logits.get_device()
        ws = _lib.workspace_ptr(didx, _raw_stream(didx), need)
        rc, need, scores, indices = fast.topk_softmax(logits, k, algo, with_scores, idx64, score_mode, ws, need)
    if rc:
        _lib.check(rc)
    return scores, indices


def topk_softmax(logits: torch.Tensor, k: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """Auto-selected fused TopK+softmax: ``(scores fp32 [M,k], indices int32 [M,k])``.

    Drop-in for topk_softmax / topk_softmax_best (kernels/__init__.py:21,
    kernels/topk_softmax_tilelang.py:1103-1135).  Unlike the reference's radix
    branch, the radix path also returns indices sorted by descending score.
    """
    return _run(logits, k, _lib.MOE_TOPK_AUTO, True)


topk_softmax_best = topk_softmax


def topk_softmax_bitonic(logits: torch.Tensor, k: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """Wave64 bitonic-network TopK+softmax, num_experts <= 64
    (reference: topk_softmax_bitonic, kernels/topk_softmax_tilelang.py:895-921,
    which allows up to 1024 and raises ValueError beyond)."""
    return _run(logits, k, _lib.MOE_TOPK_BITONIC, True)


def topk_softmax_selection(logits: torch.Tensor, k: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """Selection TopK+softmax (K rounds of wave argmax), num_experts <= 1024
    (reference: topk_softmax_selection, kernels/topk_softmax_tilelang.py:983-1001)."""
    return _run(logits, k, _lib.MOE_TOPK_SELECTION, True)


topk_softmax_sonic = topk_softmax_selection


def topk_softmax_radix(logits: torch.Tensor, k: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """Radix-select TopK with the softmax fused in the same kernel (the
    reference's radix branch of topk_softmax_best, :1126-1131, runs radix,
    then torch.gather and torch.softmax)."""
    return _run(logits, k, _lib.MOE_TOPK_RADIX, True)


def topk_radix(logits: torch.Tensor, topk: int = 6) -> torch.Tensor:
    """Indices-only radix TopK, int32 [M, topk], sorted by descending value.

    Drop-in for topk_radix_tilelang (kernels/topk_softmax_tilelang.py:205-235),
    which returns the same index set in unspecified order.
    """
    return _run(logits, topk, _lib.MOE_TOPK_RADIX, False)[1]


# Name used by the reference's package API (kernels/__init__.py:11).
topk_radix_tilelang = topk_radix


def topk_softmax_int64(logits: torch.Tensor, k: int, algo: str = "auto"
                       ) -> Tuple[torch.Tensor, torch.Tensor]:
    """Same as ``topk_softmax`` with int64 indices (the dtype torch.topk and the
    reference baseline return); ``algo`` forces one of auto/bitonic/selection/radix."""
    return _run(logits, k, _ALGOS[algo], True, torch.int64)


# ---------------------------------------------------------------------------
# Score conventions of the reference's baselines (kernels/topk_softmax_baseline.py).
# Every variant selects the same experts in the same order (value
# descending, ties to the lower index); they differ in the normaliser.
# ---------------------------------------------------------------------------
def topk_softmax_fused(logits: torch.Tensor, k: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """Convention B: softmax over the k selected logits (reference
    topk_softmax_fused, :39-66).  Same as ``topk_softmax``."""
    return _run(logits, k, _lib.MOE_TOPK_AUTO, True)


topk_softmax_conv_b_unfused = topk_softmax_fused


def topk_softmax_separate(logits: torch.Tensor, k: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """Convention A: softmax over all experts, read at the top-k (reference
    topk_softmax_separate, :15-36, softmax then torch.topk).  The top-k are
    chosen by logit, the order the rounded probabilities refine only on
    exact ties."""
    return _run(logits, k, _lib.MOE_TOPK_AUTO, True, score_mode=_lib.MOE_SCORES_ALL)


def topk_softmax_conv_a_renorm(logits: torch.Tensor, k: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """Convention A + renormalisation (reference topk_softmax_conv_a_renorm,
    :223-237): softmax over all experts, top-k, divided by their sum, which
    equals Convention B algebraically and is computed as such."""
    return _run(logits, k, _lib.MOE_TOPK_AUTO, True, score_mode=_lib.MOE_SCORES_TOPK_RENORM)


def topk_softmax_scores(logits: torch.Tensor, k: int, convention: str = "B", algo: str = "auto",
                        index_dtype: torch.dtype = torch.int32) -> Tuple[torch.Tensor, torch.Tensor]:
    """TopK+softmax with an explicit score convention ("A", "A_renorm" or
    "B") and algorithm (auto/bitonic/selection/radix)."""
    modes = {"B": _lib.MOE_SCORES_TOPK, "A": _lib.MOE_SCORES_ALL, "A_renorm": _lib.MOE_SCORES_TOPK_RENORM}
    if convention not in modes:
        raise ValueError(f"convention must be one of {list(modes)}, got {convention!r}")
    if index_dtype not in _IDX_DTYPES:
        raise ValueError("index_dtype must be torch.int32 or torch.int64")
    return _run(logits, k, _ALGOS[algo], True, index_dtype, modes[convention])
