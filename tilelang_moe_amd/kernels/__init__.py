"""Drop-in package API for the MoE routed-expert hot path.

Mirrors the hot-path names of the reference's kernels/__init__.py
(:11-22 TopK+softmax, :31-35 grouped GEMM): ``topk_softmax`` and
``grouped_gemm`` are the recommended entry points, the other names are the
per-algorithm variants the reference also exports.  The router GEMM and
the fused router GEMM + TopK + softmax (kernels/router_gemm_topk_softmax.py
in the reference) live in the submodule of the same name.  Every function runs a
hand-written gfx950 HIP kernel from libmoe_hip.so.
"""
from .topk_softmax import (
    select_strategy,
    topk_radix,
    topk_radix_tilelang,
    topk_softmax,
    topk_softmax_best,
    topk_softmax_bitonic,
    topk_softmax_conv_a_renorm,
    topk_softmax_conv_b_unfused,
    topk_softmax_fused,
    topk_softmax_int64,
    topk_softmax_radix,
    topk_softmax_scores,
    topk_softmax_selection,
    topk_softmax_separate,
    topk_softmax_sonic,
)
from .grouped_gemm import grouped_gemm, grouped_gemm_best, grouped_gemm_reuse_routing, route_sort
from .fusedmoe import (
    FusedMoETileLang,
    FusedMoETileLangStreams,
    fused_moe_routed,
    fusedmoe,
    fusedmoe_best,
    fusedmoe_tilelang,
    fusedmoe_tilelang_streams,
    grouped_gemm_swiglu,
    moe_combine,
)
from .router_gemm_topk_softmax import (
    get_fused_router_kernel,
    get_router_gemm_kernel,
    prepare_router_weight,
    router_gemm,
    router_topk_softmax,
    router_topk_softmax_prepared,
)

__all__ = [
    "topk_softmax",
    "topk_softmax_best",
    "topk_softmax_bitonic",
    "topk_softmax_selection",
    "topk_softmax_sonic",
    "topk_softmax_radix",
    "topk_softmax_int64",
    "topk_softmax_fused",
    "topk_softmax_conv_b_unfused",
    "topk_softmax_separate",
    "topk_softmax_conv_a_renorm",
    "topk_softmax_scores",
    "topk_radix",
    "topk_radix_tilelang",
    "select_strategy",
    "grouped_gemm",
    "grouped_gemm_best",
    "grouped_gemm_reuse_routing",
    "route_sort",
    "router_gemm",
    "router_topk_softmax",
    "prepare_router_weight",
    "router_topk_softmax_prepared",
    "get_router_gemm_kernel",
    "get_fused_router_kernel",
    "fusedmoe",
    "fusedmoe_best",
    "fusedmoe_tilelang",
    "fusedmoe_tilelang_streams",
    "FusedMoETileLang",
    "FusedMoETileLangStreams",
    "fused_moe_routed",
    "grouped_gemm_swiglu",
    "moe_combine",
]
