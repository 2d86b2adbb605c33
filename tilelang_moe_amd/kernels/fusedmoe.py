"""Routed-expert FFN (FusedMoE) — drop-in for the reference's
kernels/fusedmoe_tilelang.py and the grouped pieces it is built from.

Reference interface:
  fusedmoe_best(x, router_weight, shared_gate, shared_up, shared_down,
                routed_gate, routed_up, routed_down, n_experts_per_token)  :654-690
      aliases fusedmoe (:694), fusedmoe_tilelang (:605-651),
      fusedmoe_tilelang_streams (:559-602)
  FusedMoETileLang(d_hidden, d_expert, n_routed_experts, n_shared_experts,
                   n_experts_per_token, batch_size, seq_len, dtype,
                   block_token).forward(x, router_weight, ...)            :241-425
  x [B, S, Dh]; router_weight [E, Dh]; shared_gate/up [Ds, Dh],
  shared_down [Dh, Ds]; routed_gate/up [E, De, Dh]; routed_down [E, Dh, De].

Semantics are those of fusedmoe_pytorch (kernels/fusedmoe_baseline.py:41-168):
softmax over all E router logits, the top n_experts_per_token of them
weight the routed experts' SwiGLU FFNs, plus the shared expert on every
token.  One call runs moe_fused_moe from libmoe_hip.so: router GEMM,
Convention-A top-k, routed SwiGLU and down grouped GEMMs, shared-expert
GEMMs and a deterministic combine, all on the current stream with no host
synchronisation.  The router works in fp32 where the reference rounds its
logits and softmax to the input dtype, so on near-ties of those rounded
scores the two may route a token differently.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch

from .. import _lib

_DTYPES = {torch.bfloat16: _lib.MOE_BF16, torch.float16: _lib.MOE_F16}


def _check_same(name: str, t: torch.Tensor, dev: torch.device, dt: torch.dtype, shape) -> torch.Tensor:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if t.device != dev or t.dtype != dt:
        raise ValueError(f"{name} must be a {dt} tensor on {dev}, got {t.dtype} on {t.device}")
    if tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} must have shape {tuple(shape)}, got {tuple(t.shape)}")
    return t.contiguous()


def fused_moe_routed(x: torch.Tensor, router_weight: torch.Tensor, shared_gate: Optional[torch.Tensor],
                     shared_up: Optional[torch.Tensor], shared_down: Optional[torch.Tensor],
                     routed_gate: torch.Tensor, routed_up: torch.Tensor, routed_down: torch.Tensor,
                     n_experts_per_token: int, return_routing: bool = False):
    """FusedMoE on flat tokens x [T, Dh] -> out [T, Dh] (and, with
    return_routing, the routing weights fp32 [T, k] and expert ids int32
    [T, k]).  shared_* may be None (no shared expert)."""
    if not isinstance(x, torch.Tensor) or x.dim() != 2:
        raise ValueError("x must be a 2-D tensor [num_tokens, d_hidden]")
    if x.device.type != "cuda":
        raise ValueError("fused MoE runs on the GPU only: x must be a cuda (HIP) tensor")
    if x.dtype not in _DTYPES:
        raise ValueError(f"x must be bfloat16 or float16, got {x.dtype}")
    dev, dt = x.device, x.dtype
    T, Dh = x.shape
    if routed_gate.dim() != 3:
        raise ValueError("routed_gate must be [E, d_expert, d_hidden]")
    E, De = routed_gate.shape[0], routed_gate.shape[1]
    k = int(n_experts_per_token)
    if not 1 <= k <= E:
        raise ValueError(f"n_experts_per_token must be in [1, {E}], got {k}")
    x = x.contiguous()
    router_weight = _check_same("router_weight", router_weight, dev, dt, (E, Dh))
    routed_gate = _check_same("routed_gate", routed_gate, dev, dt, (E, De, Dh))
    routed_up = _check_same("routed_up", routed_up, dev, dt, (E, De, Dh))
    routed_down = _check_same("routed_down", routed_down, dev, dt, (E, Dh, De))
    if shared_gate is None:
        Ds = 0
        sg = su = sd = None
    else:
        Ds = shared_gate.shape[0]
        sg = _check_same("shared_gate", shared_gate, dev, dt, (Ds, Dh))
        su = _check_same("shared_up", shared_up, dev, dt, (Ds, Dh))
        sd = _check_same("shared_down", shared_down, dev, dt, (Dh, Ds))
    out = torch.empty((T, Dh), dtype=dt, device=dev)
    w = torch.empty((T, k), dtype=torch.float32, device=dev) if return_routing else None
    ids = torch.empty((T, k), dtype=torch.int32, device=dev) if return_routing else None
    if T > 0:
        L = _lib.lib()
        stream = _lib.current_stream(dev)
        ws_bytes = L.moe_fused_moe_workspace_size(T, Dh, De, Ds, E, k)
        ws = _lib.workspace(dev, stream, ws_bytes)
        ptr = lambda t: t.data_ptr() if t is not None else None  # noqa: E731
        _lib.check(L.moe_fused_moe(x.data_ptr(), router_weight.data_ptr(), ptr(sg), ptr(su), ptr(sd),
                                   routed_gate.data_ptr(), routed_up.data_ptr(), routed_down.data_ptr(),
                                   _DTYPES[dt], T, Dh, De, Ds, E, k, out.data_ptr(), ptr(w), ptr(ids),
                                   ws.data_ptr(), ws_bytes, stream))
    return (out, w, ids) if return_routing else out


def fusedmoe_best(x: torch.Tensor, router_weight: torch.Tensor, shared_gate: torch.Tensor,
                  shared_up: torch.Tensor, shared_down: torch.Tensor, routed_gate: torch.Tensor,
                  routed_up: torch.Tensor, routed_down: torch.Tensor, n_experts_per_token: int) -> torch.Tensor:
    """x [B, S, Dh] -> [B, S, Dh] (reference fusedmoe_best signature)."""
    if x.dim() != 3:
        raise ValueError("x must be [batch_size, seq_len, d_hidden]")
    B, S, Dh = x.shape
    out = fused_moe_routed(x.reshape(B * S, Dh), router_weight, shared_gate, shared_up, shared_down,
                           routed_gate, routed_up, routed_down, n_experts_per_token)
    return out.view(B, S, Dh)


fusedmoe = fusedmoe_best
fusedmoe_tilelang = fusedmoe_best
fusedmoe_tilelang_streams = fusedmoe_best


class FusedMoETileLang:
    """Reference-shaped module object; the constructor arguments fix the
    shapes a ``forward`` accepts (block_token is accepted and ignored: the
    gfx950 kernels choose their own tiles)."""

    def __init__(self, d_hidden: int, d_expert: int, n_routed_experts: int, n_shared_experts: int,
                 n_experts_per_token: int, batch_size: int, seq_len: int, dtype: torch.dtype = torch.float16,
                 block_token: int = 128):
        self.d_hidden, self.d_expert = d_hidden, d_expert
        self.n_routed_experts, self.n_shared_experts = n_routed_experts, n_shared_experts
        self.n_experts_per_token = n_experts_per_token
        self.batch_size, self.seq_len, self.dtype = batch_size, seq_len, dtype

    def forward(self, x, router_weight, shared_gate, shared_up, shared_down, routed_gate, routed_up,
                routed_down) -> torch.Tensor:
        expect = (self.batch_size, self.seq_len, self.d_hidden)
        if tuple(x.shape) != expect or x.dtype != self.dtype:
            raise ValueError(f"module built for x {expect} {self.dtype}, got {tuple(x.shape)} {x.dtype}")
        return fusedmoe_best(x, router_weight, shared_gate, shared_up, shared_down, routed_gate, routed_up,
                             routed_down, self.n_experts_per_token)

    __call__ = forward


FusedMoETileLangStreams = FusedMoETileLang


def grouped_gemm_swiglu(X: torch.Tensor, Wg: torch.Tensor, Wu: torch.Tensor,
                        expert_indices: torch.Tensor) -> torch.Tensor:
    """``silu(X[r] @ Wg[e].T) * (X[r] @ Wu[e].T)`` per routed row (e =
    expert_indices[r]) in one kernel; ids [R] or [T, topk] as grouped_gemm.
    Returns [R, I] in X's dtype; rows with an id outside [0, E) are zero."""
    from .grouped_gemm import _check_ids, _IDX

    if X.dim() != 2 or Wg.dim() != 3 or Wu.shape != Wg.shape:
        raise ValueError("expected X [T, H] and Wg, Wu [E, I, H] of one shape")
    if X.device.type != "cuda" or Wg.device != X.device or Wu.device != X.device:
        raise ValueError("grouped_gemm_swiglu runs on the GPU only")
    if X.dtype not in _DTYPES or Wg.dtype != X.dtype or Wu.dtype != X.dtype:
        raise ValueError("X, Wg and Wu must share a bfloat16 or float16 dtype")
    T, H = X.shape
    E, I, H2 = Wg.shape
    if H2 != H:
        raise ValueError(f"hidden size mismatch: X has H={H}, weights have {H2}")
    ids = _check_ids(expert_indices, X.device)
    topk = 1 if ids.dim() == 1 else ids.shape[1]
    if ids.shape[0] != T:
        raise ValueError(f"expert_indices has {ids.shape[0]} rows, X has {T}")
    Y = torch.empty((T * topk, I), dtype=X.dtype, device=X.device)
    if Y.shape[0] == 0:
        return Y
    L = _lib.lib()
    stream = _lib.current_stream(X.device)
    ws_bytes = L.moe_grouped_gemm_workspace_size(T, topk, E, I)
    ws = _lib.workspace(X.device, stream, ws_bytes)
    _lib.check(L.moe_grouped_gemm_swiglu(X.contiguous().data_ptr(), Wg.contiguous().data_ptr(),
                                         Wu.contiguous().data_ptr(), ids.data_ptr(), _DTYPES[X.dtype],
                                         _IDX[ids.dtype], T, topk, H, I, E, Y.data_ptr(), ws.data_ptr(),
                                         ws_bytes, stream))
    return Y


def moe_combine(Yr: torch.Tensor, weights: torch.Tensor, shared: Optional[torch.Tensor] = None) -> torch.Tensor:
    """out[t] = shared[t] + sum_j weights[t, j] * Yr[t*k + j] (fp32 sums, fixed order)."""
    T, k = weights.shape
    D = Yr.shape[1]
    if Yr.shape[0] != T * k or weights.dtype != torch.float32 or Yr.dtype not in _DTYPES:
        raise ValueError("expected Yr [T*k, D] bf16/fp16 and weights [T, k] fp32")
    if shared is not None and (shared.shape != (T, D) or shared.dtype != Yr.dtype):
        raise ValueError("shared must be [T, D] in Yr's dtype")
    out = torch.empty((T, D), dtype=Yr.dtype, device=Yr.device)
    L = _lib.lib()
    _lib.check(L.moe_combine(Yr.contiguous().data_ptr(), shared.contiguous().data_ptr() if shared is not None else None,
                             weights.contiguous().data_ptr(), _DTYPES[Yr.dtype], T, k, D, out.data_ptr(),
                             _lib.current_stream(Yr.device)))
    return out
