"""Expert grouped GEMM (drop-in for the reference's grouped_gemm).

Reference interface (kernels/grouped_gemm_tilelang.py):
  grouped_gemm_best(X [R,H], W [E,I,H], expert_indices [R]) -> Y [R,I]   :859-890
    H*I <= 2048*1024 -> grouped_gemm_tilelang_v2 (:682-766)
    otherwise        -> grouped_gemm_pytorch, a per-expert torch.mm loop (:542-601)

Here every shape runs one device pipeline from libmoe_hip.so: a routing sort
(per-expert counts, segment offsets, stable row permutation, M-tile table),
then one bf16/fp16 MFMA kernel whose A-tile load gathers X rows through the
permutation and whose epilogue stores rows back in routed order.  There is no
host synchronisation, no per-routing recompilation and no per-call weight
transpose.  Semantics are those of grouped_gemm_loop
(kernels/grouped_gemm_baseline.py:14-57): fp32 accumulation, output in X's
dtype, rows whose expert id lies outside [0, E) are zero.
"""
from __future__ import annotations

from typing import Tuple

import torch

from .. import _lib

_DTYPES = {torch.bfloat16: _lib.MOE_BF16, torch.float16: _lib.MOE_F16}
_IDX = {torch.int32: _lib.MOE_I32, torch.int64: _lib.MOE_I64}
_WS_SIZES = {}  # (T, topk, E, I) -> workspace bytes (the C ABI's answer, cached)
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None) or (
    lambda i: torch.cuda.current_stream(i).cuda_stream)


def _check_ids(expert_indices: torch.Tensor, dev: torch.device) -> torch.Tensor:
    if not isinstance(expert_indices, torch.Tensor):
        raise TypeError("expert_indices must be a torch.Tensor")
    if expert_indices.dtype not in _IDX:
        raise ValueError(f"expert_indices must be int32 or int64, got {expert_indices.dtype}")
    if expert_indices.device != dev:
        raise ValueError("expert_indices must be on the same device as X")
    return expert_indices.contiguous()


def grouped_gemm(X: torch.Tensor, W: torch.Tensor, expert_indices: torch.Tensor) -> torch.Tensor:
    """``Y[r] = X[r] @ W[expert_indices[r]].T`` for every routed row r.

    X: [R, H] bf16/fp16; W: [E, I, H] same dtype; expert_indices: [R] int32/int64.
    Also accepts expert_indices of shape [T, topk] with X [T, H]: routed row
    r = t*topk + j then reads token t, which equals the reference applied to
    ``X.repeat_interleave(topk, 0)`` and ``expert_indices.flatten()`` without
    materialising the repeated X.  Returns Y [R, I] (R = T*topk) in X's dtype.
    """
    if not isinstance(X, torch.Tensor) or not isinstance(W, torch.Tensor):
        raise TypeError("X and W must be torch.Tensors")
    if X.dim() != 2 or W.dim() != 3:
        raise ValueError(f"expected X [R,H] and W [E,I,H], got {tuple(X.shape)} and {tuple(W.shape)}")
    if X.device.type != "cuda" or W.device != X.device:
        raise ValueError("grouped_gemm runs on the GPU only: X and W must be cuda (HIP) tensors "
                         "on one device")
    if X.dtype not in _DTYPES or W.dtype != X.dtype:
        raise ValueError(f"X and W must both be bfloat16 or both float16, got {X.dtype} and {W.dtype}")
    T, H = X.shape
    E, I, H2 = W.shape
    if H2 != H:
        raise ValueError(f"hidden size mismatch: X has H={H}, W has H={H2}")
    ids = _check_ids(expert_indices, X.device)
    if ids.dim() == 1:
        topk = 1
        if ids.shape[0] != T:
            raise ValueError(f"expert_indices has {ids.shape[0]} rows, X has {T}")
    elif ids.dim() == 2:
        topk = ids.shape[1]
        if ids.shape[0] != T:
            raise ValueError(f"expert_indices [T, topk] has T={ids.shape[0]}, X has {T}")
    else:
        raise ValueError("expert_indices must be [R] or [T, topk]")
    R = T * topk
    X = X.contiguous()
    W = W.contiguous()
    L = _lib.lib()
    didx = X.get_device()
    stream = _raw_stream(didx)
    key = (T, topk, E, I)
    ws_bytes = _WS_SIZES.get(key)
    if ws_bytes is None:
        if len(_WS_SIZES) > 4096:
            _WS_SIZES.clear()
        ws_bytes = _WS_SIZES[key] = L.moe_grouped_gemm_workspace_size(T, topk, E, I) if R else 0
    ws = _lib.workspace_ptr(didx, stream, ws_bytes)
    rc, Y = _lib.fast.grouped_gemm(X, W, ids, _DTYPES[X.dtype], _IDX[ids.dtype], T, topk, H, I, E, ws,
                                   ws_bytes, stream)
    if rc:
        _lib.check(rc)
    return Y


grouped_gemm_best = grouped_gemm


def grouped_gemm_reuse_routing(X: torch.Tensor, W: torch.Tensor, topk: int = 1) -> torch.Tensor:
    """``grouped_gemm`` without its routing sort, on the routing the previous
    ``grouped_gemm`` call on this stream computed; that call must have had
    the same expert_indices (so the same row count T * topk, experts E and
    output width I), and no other call of this package may have run on the
    stream since (they share its workspace).  The reference benchmark does
    its routing once outside the timed region
    (benchmarks/benchmark_grouped_gemm.py:116-130); this is that split.
    """
    if X.dim() != 2 or W.dim() != 3 or X.dtype not in _DTYPES or W.dtype != X.dtype or not X.is_cuda:
        raise ValueError("expected X [T,H] and W [E,I,H] of one dtype (bf16/fp16) on the GPU")
    T, H = X.shape
    E, I, H2 = W.shape
    if H2 != H:
        raise ValueError(f"hidden size mismatch: X has H={H}, W has H={H2}")
    X = X.contiguous()
    W = W.contiguous()
    Y = torch.empty((T * topk, I), dtype=X.dtype, device=X.device)
    if T * topk == 0:
        return Y
    L = _lib.lib()
    didx = X.get_device()
    stream = _raw_stream(didx)
    ws_bytes = L.moe_grouped_gemm_workspace_size(T, topk, E, I)
    ws = _lib.workspace_ptr(didx, stream, ws_bytes)
    _lib.check(L.moe_grouped_gemm_routed(X.data_ptr(), W.data_ptr(), _DTYPES[X.dtype], T, topk, H, I, E,
                                         Y.data_ptr(), ws, ws_bytes, stream))
    return Y


def route_sort(expert_indices: torch.Tensor, num_experts: int
               ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Device counting sort of routed rows by expert.

    Returns ``(counts int32 [E], offsets int32 [E+1], sorted_rows int32 [R])``:
    rows of expert e are ``sorted_rows[offsets[e]:offsets[e+1]]`` in ascending
    order, rows with an id outside [0, E) follow from ``offsets[E]``.  This is
    the device replacement of the reference's argsort + bincount().tolist() +
    Python offset loops (kernels/grouped_gemm_tilelang.py:700-729).
    """
    if not isinstance(expert_indices, torch.Tensor) or expert_indices.device.type != "cuda":
        raise ValueError("route_sort runs on the GPU only: expert_indices must be a cuda tensor")
    ids = _check_ids(expert_indices, expert_indices.device).reshape(-1)
    E = int(num_experts)
    R = ids.numel()
    dev = ids.device
    counts = torch.empty(E, dtype=torch.int32, device=dev)
    offsets = torch.empty(E + 1, dtype=torch.int32, device=dev)
    sorted_rows = torch.empty(R, dtype=torch.int32, device=dev)
    L = _lib.lib()
    stream = _lib.current_stream(dev)
    ws_bytes = L.moe_route_sort_workspace_size(R, E)
    ws = _lib.workspace(dev, stream, ws_bytes)
    _lib.check(L.moe_route_sort(ids.data_ptr(), _IDX[ids.dtype], R, E, counts.data_ptr(),
                                offsets.data_ptr(), sorted_rows.data_ptr(),
                                ws.data_ptr() if ws is not None else None, ws_bytes, stream))
    return counts, offsets, sorted_rows
