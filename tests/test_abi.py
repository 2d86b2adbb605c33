"""CPU checks of the C-ABI library: it loads, exports every function that
include/moe_hip.h declares, and its host-only entry points (algorithm
choice, workspace sizes, argument validation) behave.  No kernel runs here."""
import ctypes
import os
import re

import pytest

from conftest import REPO
from tilelang_moe_amd import _lib

HEADER = os.path.join(REPO, "include", "moe_hip.h")


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(moe_[a-z0-9_]+)\s*\(", text)))


def test_header_and_binding_agree():
    assert header_functions() == sorted(_lib.SIGNATURES)


def test_library_exports_every_declared_symbol():
    L = _lib.lib()
    for name in header_functions():
        assert hasattr(L, name), name
        assert isinstance(getattr(L, name), ctypes._CFuncPtr)


def test_version_and_error_string():
    L = _lib.lib()
    assert L.moe_version() >= 100
    assert isinstance(L.moe_last_error(), bytes)


@pytest.mark.parametrize("n,algo", [(1, 0), (8, 0), (64, 0), (65, 1), (128, 1), (512, 1), (513, 2), (32768, 2)])
def test_select_algo_thresholds(n, algo):
    assert _lib.lib().moe_topk_select_algo(n, 1) == algo


def test_select_strategy_names():
    from tilelang_moe_amd.kernels import select_strategy
    assert [select_strategy(n, 6) for n in (64, 128, 256, 32768)] == ["bitonic", "selection", "selection", "radix"]


def test_workspace_sizes():
    L = _lib.lib()
    assert L.moe_topk_softmax_workspace_size(64, 32768, 2048, 2) >= 0
    small = L.moe_grouped_gemm_workspace_size(4096, 2, 8, 256)
    big = L.moe_grouped_gemm_workspace_size(4096, 8, 256, 2048)
    assert 0 < small < big < (64 << 20)
    assert L.moe_route_sort_workspace_size(32768, 256) > 0


def test_argument_validation_without_gpu():
    L = _lib.lib()
    nul = None
    # k > N
    assert L.moe_topk_softmax(nul, 0, 4, 8, 8, 9, nul, nul, 3, -1, nul, 0, nul) == _lib.MOE_EINVAL
    assert b"k" in L.moe_last_error().lower() or b"K" in L.moe_last_error()
    # bad dtype of indices
    assert L.moe_topk_softmax(1, 0, 4, 8, 8, 2, nul, 1, 7, -1, nul, 0, nul) == _lib.MOE_EINVAL
    # bitonic beyond 64
    assert L.moe_topk_softmax(1, 0, 4, 100, 100, 2, nul, 1, 3, 0, nul, 0, nul) == _lib.MOE_EUNSUP
    # radix K limit
    assert L.moe_topk_softmax(1, 0, 4, 40000, 40000, 20000, nul, 1, 3, 2, nul, 0, nul) == _lib.MOE_EUNSUP
    # M == 0 is a no-op success
    assert L.moe_topk_softmax(nul, 0, 0, 8, 8, 2, nul, 1, 3, -1, nul, 0, nul) == _lib.MOE_OK
    # grouped GEMM: H not a multiple of 8, too many experts, workspace too small, R == 0
    assert L.moe_grouped_gemm(16, 16, 16, 1, 3, 4, 1, 12, 8, 2, 16, 16, 1 << 20, nul) == _lib.MOE_EUNSUP
    assert L.moe_grouped_gemm(16, 16, 16, 1, 3, 4, 1, 16, 8, 5000, 16, 16, 1 << 20, nul) == _lib.MOE_EUNSUP
    assert L.moe_grouped_gemm(16, 16, 16, 1, 3, 4, 1, 16, 8, 2, 16, 16, 8, nul) == _lib.MOE_EINVAL
    assert L.moe_grouped_gemm(16, 16, 16, 0, 3, 4, 1, 16, 8, 2, 16, 16, 1 << 20, nul) == _lib.MOE_EINVAL
    assert L.moe_grouped_gemm(nul, nul, nul, 1, 3, 0, 1, 16, 8, 2, nul, nul, 0, nul) == _lib.MOE_OK
    assert L.moe_route_sort(nul, 3, 10, 0, 16, 16, 16, 16, 1 << 20, nul) == _lib.MOE_EUNSUP
    # X, or one expert's weights, beyond 2^32 16-byte chunks (the tiles' 32-bit row offsets)
    assert L.moe_grouped_gemm(16, 16, 16, 1, 3, 1 << 20, 1, 1 << 16, 8, 2, 16, 16, 1 << 20, nul) == _lib.MOE_EUNSUP
    assert b"64 GiB" in L.moe_last_error()
    assert L.moe_grouped_gemm(16, 16, 16, 1, 3, 4, 1, 1 << 16, 1 << 20, 2, 16, 16, 1 << 20, nul) == _lib.MOE_EUNSUP


def test_python_api_rejects_cpu_tensors():
    """No CPU fallback: the product path refuses host tensors loudly."""
    import torch
    from tilelang_moe_amd.kernels import grouped_gemm, topk_softmax

    with pytest.raises(ValueError, match="GPU only"):
        topk_softmax(torch.randn(4, 16), 2)
    with pytest.raises(ValueError, match="GPU only"):
        grouped_gemm(torch.randn(4, 16).bfloat16(), torch.randn(2, 8, 16).bfloat16(), torch.zeros(4, dtype=torch.int64))
    with pytest.raises(ValueError):
        topk_softmax(torch.randn(4, 16, 2), 2)


def test_router_gemm_host_checks():
    L = _lib.lib()
    nul = None
    # workspace: control block alone once there are 512 tiles (32768 tokens of
    # 64-row tiles), plus the split-H partials [G][T][E] below that
    assert L.moe_router_workspace_size(32768, 5120, 160) == 4096
    assert L.moe_router_workspace_size(16384, 5120, 160) == 4096 + 2 * 16384 * 160 * 4
    assert L.moe_router_workspace_size(256, 5120, 160) > 4096
    # fused limits: E > 256 or K > 32 -> unsupported; K > E -> invalid
    assert L.moe_router_topk_softmax(16, 16, 1, 4, 64, 300, 8, 16, 16, 3, 16, 1 << 20, nul) == _lib.MOE_EUNSUP
    assert L.moe_router_topk_softmax(16, 16, 1, 4, 64, 64, 33, 16, 16, 3, 16, 1 << 20, nul) == _lib.MOE_EUNSUP
    assert L.moe_router_topk_softmax(16, 16, 1, 4, 64, 8, 9, 16, 16, 3, 16, 1 << 20, nul) == _lib.MOE_EINVAL
    # H not a multiple of 8, bad dtype, misaligned operand, small workspace
    assert L.moe_router_gemm(16, 16, 1, 4, 12, 8, 16, 16, 1 << 20, nul) == _lib.MOE_EUNSUP
    assert L.moe_router_gemm(16, 16, 0, 4, 16, 8, 16, 16, 1 << 20, nul) == _lib.MOE_EINVAL
    assert L.moe_router_gemm(18, 16, 1, 4, 16, 8, 16, 16, 1 << 20, nul) == _lib.MOE_EINVAL
    assert L.moe_router_gemm(16, 16, 1, 4, 16, 8, 16, 16, 8, nul) == _lib.MOE_EINVAL
    # T == 0 is a no-op success; the transpose checks its stride
    assert L.moe_router_gemm(nul, nul, 1, 0, 16, 8, nul, 16, 1 << 20, nul) == _lib.MOE_OK
    assert L.moe_router_weight_transpose(16, 1, 16, 8, 4, 16, nul) == _lib.MOE_EINVAL


def test_router_python_api_shapes_and_names():
    import torch
    from tilelang_moe_amd.kernels import router_gemm_topk_softmax as R

    assert R._next_pow2(160) == 256 and R._next_pow2(64) == 64
    with pytest.raises(ValueError, match="Unknown algorithm"):
        R.get_fused_router_kernel("wgmma", 256, 4096, 128, 8)
    with pytest.raises(ValueError, match="GPU only"):
        R.router_topk_softmax(torch.randn(4, 16).bfloat16(), torch.randn(16, 8).bfloat16(), 2)
    for algo in R.FUSED_ALGOS:
        assert callable(getattr(R, f"fused_router_{algo}_kernel")(256, 4096, 160, 256, 8))


def test_noalloc_host_checks():
    L = _lib.lib()
    m = re.search(r"#define MOE_NOALLOC_SCRATCH_BYTES \((\d+)u << (\d+)\)", open(HEADER).read())
    assert m and int(m[1]) << int(m[2]) == _lib.MOE_NOALLOC_SCRATCH_BYTES
    # T == 0 is a no-op; bad shapes and problems beyond the fixed scratch are
    # rejected before any device call.
    assert L.moe_grouped_gemm_noalloc(None, None, None, 1, 3, 0, 8, 64, 64, 256, None, None) == _lib.MOE_OK
    assert L.moe_grouped_gemm_noalloc(16, 16, 16, 1, 3, 4, 0, 64, 64, 8, 16, None) == _lib.MOE_EINVAL
    assert L.moe_grouped_gemm_noalloc(16, 16, 16, 1, 3, 4, 1, 64, 64, 5000, 16, None) == _lib.MOE_EUNSUP
    assert L.moe_grouped_gemm_noalloc(16, 16, 16, 1, 3, 200000, 8, 64, 64, 256, 16, None) == _lib.MOE_EUNSUP
    assert b"scratch" in L.moe_last_error()
    assert L.moe_grouped_gemm_workspace_size(200000, 8, 256, 64) > _lib.MOE_NOALLOC_SCRATCH_BYTES
