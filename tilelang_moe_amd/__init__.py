"""MI355X (gfx950) MoE routed-expert hot path: fused TopK+softmax router and
expert grouped GEMM as hand-written HIP kernels behind a C ABI.

    from tilelang_moe_amd.kernels import topk_softmax, grouped_gemm
"""
from .kernels import *  # noqa: F401,F403
from .kernels import __all__  # noqa: F401

__version__ = "0.1.0"
