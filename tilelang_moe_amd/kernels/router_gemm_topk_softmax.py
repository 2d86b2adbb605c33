"""Router GEMM and fused router GEMM + TopK + softmax (drop-in for the
reference's kernels/router_gemm_topk_softmax.py).

Reference interface:
  get_fused_router_kernel(algo, num_tokens, H, E, top_k, dtype, block_M,
                          block_K, num_stages, threads) -> f(X, W)     :1169-1203
      algo in cpasync_selection, cpasync_bitonic, tma_selection, tma_bitonic,
      tma_auto_selection, tma_auto_bitonic; W is [H, E] (unpadded);
      f returns (scores fp32 [T, top_k], indices int32 [T, top_k])
  fused_router_<algo>_kernel(num_tokens, H, E, E_padded, top_k, ...)
      -> f(X, W_padded [H, E_padded])                                  :148-1150
  get_router_gemm_kernel(num_tokens, H, E, dtype) -> f(X, W) -> logits
      fp32 [T, E]                                                      :125-145
  _next_pow2(n)                                                        :44-45

Here every algo name runs the same gfx950 kernel: the six reference
variants differ only in their NVIDIA copy/MMA strategy (cp.async, TMA,
warp specialisation).  The kernel reads the weights transposed, Wt [E, H];
the transpose of each weight tensor is made once and cached while that
tensor exists unchanged (keyed on its storage and version counter, with a
reference held so the storage cannot be reused under the key).

Semantics: logits = X.float() @ W.float() with fp32 accumulation; the fused
form returns the top_k logits of each token in descending order with their
softmax (as topk_softmax) and int32 expert indices.  Ties go to the lower
expert index, the rule of every router entry point of this package; the
reference's fused kernels pick the higher index on exact ties
(kernels/router_gemm_topk_softmax.py:224-229), and its correctness test
compares index sets (tests/test_router_fusion_correctness.py:51).
Limits of the fused kernel: E <= 256, top_k <= 32; beyond them the callable
runs the router GEMM and topk_softmax (two launches, same results).
"""
from __future__ import annotations

import math
import threading
from collections import OrderedDict
from typing import Callable, Tuple

import torch

from .. import _lib
from .topk_softmax import topk_softmax, topk_softmax_int64

_DTYPES = {torch.bfloat16: _lib.MOE_BF16, torch.float16: _lib.MOE_F16}
FUSED_ALGOS = ("cpasync_selection", "cpasync_bitonic", "tma_selection", "tma_bitonic",
               "tma_auto_selection", "tma_auto_bitonic")
FUSED_MAX_E = 256
FUSED_MAX_K = 32


def _next_pow2(n: int) -> int:
    return 1 << math.ceil(math.log2(max(n, 2)))


def _torch_dtype(dtype) -> torch.dtype:
    """Accepts torch dtypes and the reference's dtype spellings ("bfloat16",
    "float16", or objects whose str() names one of them)."""
    if isinstance(dtype, torch.dtype):
        return dtype
    name = str(dtype).lower()
    if "bfloat16" in name or name == "bf16":
        return torch.bfloat16
    if "float16" in name or name == "fp16" or name == "half":
        return torch.float16
    raise ValueError(f"router dtype must be bfloat16 or float16, got {dtype!r}")


# ---------------------------------------------------------------------------
# Transposed-weight cache.
# ---------------------------------------------------------------------------
_wt_lock = threading.Lock()
_wt_cache: "OrderedDict[tuple, Tuple[torch.Tensor, torch.Tensor]]" = OrderedDict()
_WT_CACHE_MAX = 16


def transposed_weight(W: torch.Tensor, E: int) -> torch.Tensor:
    """Wt [E, H] (contiguous) from W [H, >=E] (row stride >= E, unit column
    stride), computed on the device and cached per weight tensor.

    The cache key includes torch's version counter of W, so an eager call
    after an in-place update of W transposes again.  A captured HIP graph
    cannot consult that counter at replay, so while the current stream is
    capturing, the transpose is always recorded into the graph (and not
    cached): every replay then reads W as it is at replay time, as the
    reference's kernels do."""
    H = W.shape[0]
    if W.stride(0) == 1 and W.stride(1) == H and (W.data_ptr() % 16) == 0:
        # W is the transposed view of a contiguous [>=E, H] tensor: its first
        # E rows are already the kernels' layout and are read in place.
        return W.t()[:E]
    if W.stride(1) != 1:
        # Other layouts: one contiguous copy, transposed, not cached (the
        # copy's storage would make a new cache key on every call).
        W = W.contiguous()
        Wt = torch.empty((E, H), dtype=W.dtype, device=W.device)
        _lib.check(_lib.lib().moe_router_weight_transpose(W.data_ptr(), _DTYPES[W.dtype], H, E, W.stride(0),
                                                          Wt.data_ptr(), _lib.current_stream(W.device)))
        return Wt
    capturing = torch.cuda.is_current_stream_capturing()
    key = (W.device.index, W.untyped_storage().data_ptr(), W.storage_offset(), W._version,
           tuple(W.shape), tuple(W.stride()), W.dtype, E)
    if not capturing:
        with _wt_lock:
            hit = _wt_cache.get(key)
            if hit is not None:
                _wt_cache.move_to_end(key)
                return hit[1]
    Wt = torch.empty((E, H), dtype=W.dtype, device=W.device)
    L = _lib.lib()
    _lib.check(L.moe_router_weight_transpose(W.data_ptr(), _DTYPES[W.dtype], H, E, W.stride(0),
                                             Wt.data_ptr(), _lib.current_stream(W.device)))
    if capturing:
        return Wt
    with _wt_lock:
        _wt_cache[key] = (W, Wt)  # W is held so its storage cannot be reused under this key
        while len(_wt_cache) > _WT_CACHE_MAX:
            _wt_cache.popitem(last=False)
    return Wt


def _check(X: torch.Tensor, W: torch.Tensor, E: int) -> Tuple[torch.Tensor, torch.Tensor, int, int]:
    """Validates X [T, H] and W [H, >=E]; returns (X, W, T, H) with X
    contiguous (W keeps its layout: transposed_weight handles any)."""
    if not isinstance(X, torch.Tensor) or not isinstance(W, torch.Tensor):
        raise TypeError("X and W must be torch.Tensors")
    if X.dim() != 2 or W.dim() != 2:
        raise ValueError(f"expected X [T, H] and W [H, E], got {tuple(X.shape)} and {tuple(W.shape)}")
    if X.device.type != "cuda" or W.device != X.device:
        raise ValueError("the router runs on the GPU only: X and W must be cuda (HIP) tensors on one device")
    if X.dtype not in _DTYPES or W.dtype != X.dtype:
        raise ValueError(f"X and W must both be bfloat16 or both float16, got {X.dtype} and {W.dtype}")
    T, H = X.shape
    if W.shape[0] != H:
        raise ValueError(f"hidden size mismatch: X has H={H}, W has {W.shape[0]} rows")
    if not 1 <= E <= W.shape[1]:
        raise ValueError(f"E={E} must be in [1, {W.shape[1]}]")
    X = X.contiguous()
    return X, W, T, H


def prepare_router_weight(W: torch.Tensor, E: int = None) -> torch.Tensor:
    """The router weight in the kernels' layout, Wt [E, H] (K-contiguous rows,
    the MFMA B operand), from W [H, >=E].  For callers that prepare weights
    once at load time and call router_topk_softmax_prepared, e.g. from a
    replayed HIP graph, so that no transpose runs per call.  Not cached: the
    result is a snapshot of W."""
    E = W.shape[1] if E is None else int(E)
    _, W, _, H = _check(W.new_empty((0, W.shape[0])), W, E)
    if W.stride(1) != 1:
        W = W.contiguous()
    Wt = torch.empty((E, H), dtype=W.dtype, device=W.device)
    _lib.check(_lib.lib().moe_router_weight_transpose(W.data_ptr(), _DTYPES[W.dtype], H, E, W.stride(0),
                                                      Wt.data_ptr(), _lib.current_stream(W.device)))
    return Wt


def _check_prepared(X: torch.Tensor, Wt: torch.Tensor) -> Tuple[torch.Tensor, int, int, int]:
    if not isinstance(X, torch.Tensor) or not isinstance(Wt, torch.Tensor):
        raise TypeError("X and Wt must be torch.Tensors")
    if X.dim() != 2 or Wt.dim() != 2:
        raise ValueError(f"expected X [T, H] and Wt [E, H], got {tuple(X.shape)} and {tuple(Wt.shape)}")
    if not Wt.is_contiguous():
        raise ValueError("Wt must be contiguous [E, H] (prepare_router_weight returns it so)")
    if X.device.type != "cuda" or Wt.device != X.device:
        raise ValueError("the router runs on the GPU only: X and Wt must be cuda (HIP) tensors on one device")
    if X.dtype not in _DTYPES or Wt.dtype != X.dtype:
        raise ValueError(f"X and Wt must both be bfloat16 or both float16, got {X.dtype} and {Wt.dtype}")
    T, H = X.shape
    E = Wt.shape[0]
    if Wt.shape[1] != H or E < 1:
        raise ValueError(f"hidden size mismatch: X has H={H}, Wt is {tuple(Wt.shape)}")
    return X.contiguous(), T, H, E


def _router_gemm_wt(X: torch.Tensor, Wt: torch.Tensor, T: int, H: int, E: int) -> torch.Tensor:
    logits = torch.empty((T, E), dtype=torch.float32, device=X.device)
    if T == 0:
        return logits
    L = _lib.lib()
    stream = _lib.current_stream(X.device)
    ws_bytes = L.moe_router_workspace_size(T, H, E)
    ws = _lib.workspace(X.device, stream, ws_bytes)
    _lib.check(L.moe_router_gemm(X.data_ptr(), Wt.data_ptr(), _DTYPES[X.dtype], T, H, E, logits.data_ptr(),
                                 ws.data_ptr(), ws_bytes, stream))
    return logits


def _router_topk_wt(X: torch.Tensor, Wt: torch.Tensor, T: int, H: int, E: int, k: int,
                    index_dtype: torch.dtype) -> Tuple[torch.Tensor, torch.Tensor]:
    k = int(k)
    if not 1 <= k <= E:
        raise ValueError(f"k must satisfy 1 <= k <= E={E}, got {k}")
    if index_dtype not in (torch.int32, torch.int64):
        raise ValueError("index_dtype must be torch.int32 or torch.int64")
    if E > FUSED_MAX_E or k > FUSED_MAX_K:
        logits = _router_gemm_wt(X, Wt, T, H, E)
        if index_dtype == torch.int64:
            return topk_softmax_int64(logits, k)
        return topk_softmax(logits, k)
    scores = torch.empty((T, k), dtype=torch.float32, device=X.device)
    indices = torch.empty((T, k), dtype=index_dtype, device=X.device)
    if T == 0:
        return scores, indices
    L = _lib.lib()
    stream = _lib.current_stream(X.device)
    ws_bytes = L.moe_router_workspace_size(T, H, E)
    ws = _lib.workspace(X.device, stream, ws_bytes)
    _lib.check(L.moe_router_topk_softmax(X.data_ptr(), Wt.data_ptr(), _DTYPES[X.dtype], T, H, E, k,
                                         scores.data_ptr(), indices.data_ptr(),
                                         _lib.MOE_I64 if index_dtype == torch.int64 else _lib.MOE_I32,
                                         ws.data_ptr(), ws_bytes, stream))
    return scores, indices


def router_topk_softmax_prepared(X: torch.Tensor, Wt: torch.Tensor, k: int,
                                 index_dtype: torch.dtype = torch.int32) -> Tuple[torch.Tensor, torch.Tensor]:
    """router_topk_softmax with the weight already in the kernels' layout
    (Wt [E, H] from prepare_router_weight): no transpose, no cache lookup."""
    X, T, H, E = _check_prepared(X, Wt)
    return _router_topk_wt(X, Wt, T, H, E, k, index_dtype)


def router_gemm(X: torch.Tensor, W: torch.Tensor, E: int = None) -> torch.Tensor:
    """logits fp32 [T, E] = X [T, H] @ W [H, E] (W may carry padding columns
    past E)."""
    E = W.shape[1] if E is None else int(E)
    X, W, T, H = _check(X, W, E)
    logits = torch.empty((T, E), dtype=torch.float32, device=X.device)
    if T == 0:
        return logits
    Wt = transposed_weight(W, E)
    L = _lib.lib()
    stream = _lib.current_stream(X.device)
    ws_bytes = L.moe_router_workspace_size(T, H, E)
    ws = _lib.workspace(X.device, stream, ws_bytes)
    _lib.check(L.moe_router_gemm(X.data_ptr(), Wt.data_ptr(), _DTYPES[X.dtype], T, H, E, logits.data_ptr(),
                                 ws.data_ptr(), ws_bytes, stream))
    return logits


def router_topk_softmax(X: torch.Tensor, W: torch.Tensor, k: int, E: int = None,
                        index_dtype: torch.dtype = torch.int32) -> Tuple[torch.Tensor, torch.Tensor]:
    """(scores fp32 [T, k], indices [T, k]) of softmax(top-k(X @ W)) per token,
    fused in one kernel (logits stay in LDS) when E <= 256 and k <= 32."""
    E = W.shape[1] if E is None else int(E)
    X, W, T, H = _check(X, W, E)
    k = int(k)
    if not 1 <= k <= E:
        raise ValueError(f"k must satisfy 1 <= k <= E={E}, got {k}")
    if E > FUSED_MAX_E or k > FUSED_MAX_K:
        # Validated first, like the fused path; router_gemm transposes itself.
        if index_dtype not in (torch.int32, torch.int64):
            raise ValueError("index_dtype must be torch.int32 or torch.int64")
        logits = router_gemm(X, W, E)
        if index_dtype == torch.int64:
            return topk_softmax_int64(logits, k)
        return topk_softmax(logits, k)
    Wt = transposed_weight(W, E) if T > 0 else None
    return _router_topk_wt(X, Wt, T, H, E, k, index_dtype)


# ---------------------------------------------------------------------------
# Reference-shaped factories.
# ---------------------------------------------------------------------------
def _bind(num_tokens: int, H: int, E: int, dtype, fn: Callable) -> Callable:
    dt = _torch_dtype(dtype)

    def run(X, W):
        if X.shape[0] != num_tokens or X.shape[1] != H:
            raise ValueError(f"kernel built for X [{num_tokens}, {H}], got {tuple(X.shape)}")
        if X.dtype != dt:
            raise ValueError(f"kernel built for {dt}, got {X.dtype}")
        return fn(X, W)

    return run


def get_router_gemm_kernel(num_tokens: int, H: int, E: int, dtype=torch.bfloat16) -> Callable:
    """f(X [num_tokens, H], W [H, E]) -> logits fp32 [num_tokens, E]."""
    return _bind(num_tokens, H, E, dtype, lambda X, W: router_gemm(X, W, E))


def get_fused_router_kernel(algo: str, num_tokens: int, H: int, E: int, top_k: int, dtype=torch.bfloat16,
                            block_M: int = 64, block_K: int = 64, num_stages: int = 2,
                            threads: int = 256) -> Callable:
    """f(X [num_tokens, H], W [H, E]) -> (scores fp32, indices int32) [num_tokens, top_k].

    ``algo`` must be one of the reference's six names; block_M, block_K,
    num_stages and threads are accepted for signature compatibility (the
    gfx950 kernel picks its own tiles)."""
    if algo not in FUSED_ALGOS:
        raise ValueError(f"Unknown algorithm: {algo}. Valid: {list(FUSED_ALGOS)}")
    if not 1 <= int(top_k) <= int(E):
        raise ValueError(f"top_k must satisfy 1 <= top_k <= E={E}, got {top_k}")
    return _bind(num_tokens, H, E, dtype, lambda X, W: router_topk_softmax(X, W, top_k, E))


def _factory(algo: str) -> Callable:
    def make(num_tokens, H, E, E_padded, top_k, block_M=64, block_K=64, num_stages=2, threads=256,
             dtype=torch.bfloat16):
        """f(X [num_tokens, H], W_padded [H, E_padded]) -> (scores, indices);
        columns past E are ignored."""
        if E_padded < E:
            raise ValueError(f"E_padded={E_padded} < E={E}")
        return _bind(num_tokens, H, E, dtype, lambda X, W: router_topk_softmax(X, W, top_k, E))

    make.__name__ = f"fused_router_{algo}_kernel"
    return make


fused_router_cpasync_selection_kernel = _factory("cpasync_selection")
fused_router_cpasync_bitonic_kernel = _factory("cpasync_bitonic")
fused_router_tma_selection_kernel = _factory("tma_selection")
fused_router_tma_bitonic_kernel = _factory("tma_bitonic")
fused_router_tma_auto_selection_kernel = _factory("tma_auto_selection")
fused_router_tma_auto_bitonic_kernel = _factory("tma_auto_bitonic")
