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

from ._build import FAST_PATH, LIB_PATH

MOE_F32, MOE_BF16, MOE_F16, MOE_I32, MOE_I64 = 0, 1, 2, 3, 4
MOE_TOPK_AUTO, MOE_TOPK_BITONIC, MOE_TOPK_SELECTION, MOE_TOPK_RADIX = -1, 0, 1, 2
MOE_OK, MOE_EINVAL, MOE_EUNSUP, MOE_EHIP = 0, -1, -2, -3
MOE_SCORES_TOPK, MOE_SCORES_ALL, MOE_SCORES_TOPK_RENORM = 0, 1, 2
MOE_NOALLOC_SCRATCH_BYTES = 4 << 20  # include/moe_hip.h

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
    "moe_grouped_gemm_routed": (_c_int, [_c_ptr, _c_ptr, _c_int, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
                                         _c_ptr, _c_ptr, _c_size, _c_ptr]),
    "moe_grouped_gemm_noalloc": (_c_int, [_c_ptr, _c_ptr, _c_ptr, _c_int, _c_int, _c_i64, _c_i64, _c_i64,
                                          _c_i64, _c_i64, _c_ptr, _c_ptr]),
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
            _bind_fast(handle)
            _lib = handle
    return _lib


fast = None  # the torch binding (_moe_torch), bound by lib()


def _bind_fast(handle) -> None:
    """Hand the addresses of the two drop-in entry points to the torch
    binding, which allocates their outputs in C++ and calls them with plain
    integers (no ctypes conversion per call)."""
    global fast
    try:
        from . import _moe_torch
    except ImportError as e:
        raise RuntimeError(f"the torch binding {FAST_PATH} is missing or stale ({e}): build with "
                           "`python -m tilelang_moe_amd._build` (or __graft_entry__.build())") from e
    addr = lambda f: ctypes.cast(f, ctypes.c_void_p).value  # noqa: E731
    _moe_torch.bind(addr(handle.moe_topk_softmax_ex), addr(handle.moe_grouped_gemm),
                    addr(handle.moe_topk_softmax_workspace_size))
    fast = _moe_torch


def current_stream(dev) -> int:
    """Raw hipStream_t of torch's current stream on `dev` (fast path via
    torch's internal accessor when present)."""
    import torch

    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    raw = getattr(torch._C, "_cuda_getCurrentRawStream", None)
    if raw is not None:
        return raw(idx)
    return torch.cuda.current_stream(idx).cuda_stream


_ws_cache = {}    # (device index, raw stream handle) -> (tensor, data_ptr, bytes), made outside capture
_ws_capture = {}  # the same key -> buffer made during a graph capture (graph-pool memory)
_ws_retired = []  # replaced buffers: a captured graph may still reference them
_ws_lock = threading.Lock()


def workspace_ptr(dev_index: int, stream: int, nbytes: int) -> int:
    """Device address of a zero-initialised workspace of at least `nbytes`
    for calls on (`dev_index`, `stream`); 0 when nbytes is 0.

    Calls on one stream are ordered, so they share one buffer; calls on
    different streams get different buffers.  Every call leaves the
    buffer's control block zero, so a buffer stays valid for the next call
    on its stream, also when torch hands a stream handle to a new stream
    (its streams live in pools and are never destroyed).  A buffer that is
    outgrown is replaced but kept alive: a graph captured earlier may still
    use it.

    Inside a graph capture the stream's buffer is used if it is large
    enough.  Otherwise a buffer is made in the capture (it comes from the
    graph's memory pool, and its zero fill is recorded in the graph, so it
    is zero at the start of every replay); such a buffer serves later
    captured calls on that stream, is never used by eager calls, and is kept
    alive for the life of the process.  Graphs that share a buffer must not
    be replayed concurrently."""
    if nbytes == 0:
        return 0
    ent = _ws_cache.get((dev_index, stream))
    if ent is not None and ent[2] >= nbytes:
        return ent[1]
    return _grow(dev_index, stream, nbytes)[1]


def _grow(dev_index: int, stream: int, nbytes: int):
    import torch

    key = (dev_index, stream)
    capturing = torch.cuda.is_current_stream_capturing()
    cache = _ws_capture if capturing else _ws_cache
    with _ws_lock:
        ent = cache.get(key)
        if ent is not None and ent[2] >= nbytes:
            return ent
        size = max(nbytes, 1 << 16, 2 * (ent[2] if ent is not None else 0))
        buf = torch.zeros(size, dtype=torch.uint8, device=torch.device("cuda", dev_index))
        if ent is not None:
            _ws_retired.append(ent[0])
        ent = (buf, buf.data_ptr(), size)
        cache[key] = ent
        if capturing:
            _ws_retired.append(buf)  # graph-pool memory: never released by this package
        elif fast is not None:
            fast.set_workspace(dev_index, stream, ent[1], size)  # the router call looks it up in C++
        return ent


def workspace(dev, stream: int, nbytes: int):
    """The workspace of workspace_ptr as a uint8 tensor (None when nbytes is 0)."""
    if nbytes == 0:
        return None
    idx = dev.index if dev.index is not None else __import__("torch").cuda.current_device()
    ent = _ws_cache.get((idx, stream))
    if ent is None or ent[2] < nbytes:
        ent = _grow(idx, stream, nbytes)
    return ent[0]


def check(rc: int) -> None:
    """Turn a C-ABI return code into the reference's exception style."""
    if rc == MOE_OK:
        return
    msg = lib().moe_last_error().decode(errors="replace")
    if rc in (MOE_EINVAL, MOE_EUNSUP):
        raise ValueError(msg)
    raise RuntimeError(msg)
