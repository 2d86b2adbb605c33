"""ctypes binding of ``libmoe_hip.so`` (the C ABI declared in include/moe_hip.h).

The library is loaded after ``import torch`` so that its HIP runtime
dependency (SONAME libamdhip64.so.7) resolves to the runtime torch already
loaded: device pointers and hipStream_t handles from torch are then valid in
the library.  There is no fallback: if the library is missing or fails to
load, every operator raises.
"""
from __future__ import annotations

import ctypes
import os
import threading

from ._build import LIB_PATH

MOE_F32, MOE_BF16, MOE_F16, MOE_I32, MOE_I64 = 0, 1, 2, 3, 4
MOE_TOPK_AUTO, MOE_TOPK_BITONIC, MOE_TOPK_SELECTION, MOE_TOPK_RADIX = -1, 0, 1, 2
MOE_OK, MOE_EINVAL, MOE_EUNSUP, MOE_EHIP = 0, -1, -2, -3
MOE_SCORES_TOPK, MOE_SCORES_ALL, MOE_SCORES_TOPK_RENORM = 0, 1, 2

_c_i64 = ctypes.c_int64
_c_int = ctypes.c_int
_c_size = ctypes.c_size_t
_c_ptr = ctypes.c_void_p

# name -> (restype, argtypes); must list every function of include/moe_hip.h.
SIGNATURES = {
    "moe_last_error": (ctypes.c_char_p, []),
    "moe_version": (_c_int, []),
    "moe_topk_select_algo": (_c_int, [_c_i64, _c_i64]),
    "moe_topk_softmax_workspace_size": (_c_size, [_c_i64, _c_i64, _c_i64, _c_int]),
    "moe_topk_softmax": (_c_int, [_c_ptr, _c_int, _c_i64, _c_i64, _c_i64, _c_i64, _c_ptr, _c_ptr,
                                  _c_int, _c_int, _c_ptr, _c_size, _c_ptr]),
    "moe_topk_softmax_ex": (_c_int, [_c_ptr, _c_int, _c_i64, _c_i64, _c_i64, _c_i64, _c_ptr, _c_ptr,
                                     _c_int, _c_int, _c_int, _c_ptr, _c_size, _c_ptr]),
    "moe_route_sort_workspace_size": (_c_size, [_c_i64, _c_i64]),
    "moe_grouped_gemm_workspace_size": (_c_size, [_c_i64, _c_i64, _c_i64, _c_i64]),
    "moe_route_sort": (_c_int, [_c_ptr, _c_int, _c_i64, _c_i64, _c_ptr, _c_ptr, _c_ptr, _c_ptr,
                                _c_size, _c_ptr]),
    "moe_grouped_gemm": (_c_int, [_c_ptr, _c_ptr, _c_ptr, _c_int, _c_int, _c_i64, _c_i64, _c_i64,
                                  _c_i64, _c_i64, _c_ptr, _c_ptr, _c_size, _c_ptr]),
    "moe_grouped_gemm_swiglu": (_c_int, [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_int, _c_int, _c_i64, _c_i64,
                                         _c_i64, _c_i64, _c_i64, _c_ptr, _c_ptr, _c_size, _c_ptr]),
    "moe_combine": (_c_int, [_c_ptr, _c_ptr, _c_ptr, _c_int, _c_i64, _c_i64, _c_i64, _c_ptr, _c_ptr]),
    "moe_fused_moe_workspace_size": (_c_size, [_c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64]),
    "moe_fused_moe": (_c_int, [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_int, _c_i64,
                               _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_size,
                               _c_ptr]),
    "moe_router_weight_transpose": (_c_int, [_c_ptr, _c_int, _c_i64, _c_i64, _c_i64, _c_ptr, _c_ptr]),
    "moe_router_workspace_size": (_c_size, [_c_i64, _c_i64, _c_i64]),
    "moe_router_gemm": (_c_int, [_c_ptr, _c_ptr, _c_int, _c_i64, _c_i64, _c_i64, _c_ptr, _c_ptr,
                                 _c_size, _c_ptr]),
    "moe_router_topk_softmax": (_c_int, [_c_ptr, _c_ptr, _c_int, _c_i64, _c_i64, _c_i64, _c_i64, _c_ptr,
                                         _c_ptr, _c_int, _c_ptr, _c_size, _c_ptr]),
}

_lock = threading.Lock()
_lib = None


def lib() -> ctypes.CDLL:
    """Load (once) and return the library; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            import torch  # noqa: F401  (binds the library to torch's HIP runtime)

            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    f"{LIB_PATH} is missing: build it with `python -m tilelang_moe_amd._build` "
                    "(or __graft_entry__.build()); there is no CPU fallback")
            handle = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype = res
                fn.argtypes = args
            _lib = handle
    return _lib


def current_stream(dev) -> int:
    """Raw hipStream_t of torch's current stream on `dev` (fast path via
    torch's internal accessor when present)."""
    import torch

    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    raw = getattr(torch._C, "_cuda_getCurrentRawStream", None)
    if raw is not None:
        return raw(idx)
    return torch.cuda.current_stream(idx).cuda_stream


_ws_cache = {}
_ws_lock = threading.Lock()


def workspace(dev, stream: int, nbytes: int):
    """Device workspace of at least `nbytes` for calls on (`dev`, `stream`).

    Calls on one stream are ordered, so they may share one buffer; calls on
    different streams get different buffers.  The buffer only grows.  It is
    zero-initialised once, as the C ABI requires."""
    import torch

    if nbytes == 0:
        return None
    key = (dev.index, stream)
    buf = _ws_cache.get(key)
    if buf is None or buf.numel() < nbytes:
        with _ws_lock:
            buf = _ws_cache.get(key)
            if buf is None or buf.numel() < nbytes:
                buf = torch.zeros(max(nbytes, 1 << 16), dtype=torch.uint8, device=dev)
                _ws_cache[key] = buf
    return buf


def check(rc: int) -> None:
    """Turn a C-ABI return code into the reference's exception style."""
    if rc == MOE_OK:
        return
    msg = lib().moe_last_error().decode(errors="replace")
    if rc in (MOE_EINVAL, MOE_EUNSUP):
        raise ValueError(msg)
    raise RuntimeError(msg)
