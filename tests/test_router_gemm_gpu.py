"""GPU parity of the router GEMM and the fused router GEMM + TopK + softmax.

Bars:
  * router_gemm: logits within the fp32 accumulation bound of the float64
    oracle logits: |gpu - ref| <= 1e-5 * (|X| @ |W|) + 1e-6 elementwise.
  * fused router vs router_gemm + topk_softmax (same kernels for the
    logits): indices bit-exact, scores within 1e-6 relative.
  * fused router vs the float64 oracle (the reference test's
    ref_topk_softmax, tests/test_router_fusion_correctness.py:21-25): the
    chosen experts are a top-K of the oracle logits up to the logit bound
    above, and the scores are the softmax of the oracle logits at the chosen
    experts within 2 max|logit error| + 2e-6 relative (the softmax's
    sensitivity to its inputs; the logit error is measured per row), with
    an absolute floor of 1e-30 for scores that underflow fp32.
Covers E in {8, 64, 128, 160, 256}, K in {1, 6, 8, 32}, the split-H path
(few tokens) and the unsplit path (many tokens), ragged T and H (H tail
past a k-tile), bf16 and fp16, int64 indices, exact ties, the six reference
factory names with a column-padded W, and the two-launch path past the
fused limits (E > 256 or K > 32).
"""
import numpy as np
import pytest
import torch

from oracle import router_gemm as org
from tilelang_moe_amd import kernels as K
from tilelang_moe_amd.kernels import router_gemm_topk_softmax as R

pytestmark = pytest.mark.gpu


def make(T, H, E, seed=0, dtype=torch.bfloat16, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    X = torch.randn(T, H, generator=g).to(dtype)
    W = (scale * torch.randn(H, E, generator=g)).to(dtype)
    return X.cuda(), W.cuda()


def ref_logits(X, W):
    """float64 oracle logits and the elementwise accumulation bound."""
    Xd, Wd = X.double(), W.double()
    lg = (Xd @ Wd).cpu().numpy()
    bound = (1e-5 * (Xd.abs() @ Wd.abs()) + 1e-6).cpu().numpy()
    return lg, bound


def check_against_oracle(X, W, k, scores, idx, logits=None):
    lg, bound = ref_logits(X, W)
    idx = idx.long().cpu().numpy()
    chosen = np.take_along_axis(lg, idx, 1)
    # K-th largest oracle logit per row, and the largest unchosen one.
    kth = np.sort(lg, axis=1)[:, ::-1][:, k - 1]
    mask = np.ones_like(lg, dtype=bool)
    np.put_along_axis(mask, idx, False, 1)
    other = np.where(mask, lg, -np.inf).max(axis=1) if k < lg.shape[1] else np.full(lg.shape[0], -np.inf)
    tol = bound.max(axis=1) * 2
    assert (chosen.min(axis=1) >= kth - tol).all(), "a chosen expert is not in the top-K"
    assert (other <= chosen.min(axis=1) + tol).all(), "an unchosen expert beats a chosen one"
    # Chosen experts in descending oracle order up to the bound.
    assert (np.diff(chosen, axis=1) <= tol[:, None]).all()
    # Scores: softmax is 1-Lipschitz in log space per logit pair, so with
    # d = (gpu logits - oracle logits) at the chosen experts the relative
    # score error is at most 2 max|d| (plus fp32 rounding of the softmax).
    ref_s = org.softmax_at(lg, idx)
    if logits is not None:
        d = np.abs(np.take_along_axis(logits.double().cpu().numpy(), idx, 1) - chosen).max(axis=1)
        assert (d <= bound.max(axis=1)).all()
    else:
        d = bound.max(axis=1)
    # Scores below fp32's normal range underflow (to a denormal or 0):
    # an absolute floor of 1e-30 covers them.
    err = np.abs(scores.double().cpu().numpy() - ref_s)
    lim = (2 * d + 2e-6)[:, None] * ref_s + 1e-30
    assert (err <= lim).all(), f"score error {(err - lim).max()} above bound"


def check_fused(X, W, k, E=None, index_dtype=torch.int32):
    E = W.shape[1] if E is None else E
    s, i = K.router_topk_softmax(X, W, k, E, index_dtype=index_dtype)
    logits = K.router_gemm(X, W, E)
    s2, i2 = K.topk_softmax(logits, k)
    torch.cuda.synchronize()
    assert s.shape == (X.shape[0], k) and i.dtype == index_dtype
    assert torch.equal(i.long(), i2.long()), "fused indices differ from router_gemm + topk_softmax"
    torch.testing.assert_close(s, s2, rtol=1e-6, atol=0)
    check_against_oracle(X, W[:, :E], k, s, i, logits)
    return s, i


@pytest.mark.parametrize("T,H,E", [(1, 64, 8), (37, 520, 64), (256, 3584, 64), (256, 4096, 128),
                                   (256, 5120, 160), (1000, 1024, 256), (4096, 2048, 160), (70, 8, 100)])
def test_router_gemm_logits(cuda, T, H, E):
    X, W = make(T, H, E, seed=T + H + E)
    lg = K.router_gemm(X, W)
    torch.cuda.synchronize()
    ref, bound = ref_logits(X, W)
    assert lg.shape == (T, E) and lg.dtype == torch.float32
    err = np.abs(lg.cpu().numpy().astype(np.float64) - ref)
    assert (err <= bound).all(), f"max excess {(err - bound).max()}"


@pytest.mark.parametrize("T,H,E,k", [(256, 3584, 64, 8), (256, 4096, 128, 8), (256, 5120, 160, 6),
                                     (1, 512, 160, 6), (63, 1032, 256, 32), (65, 776, 8, 1),
                                     (3000, 2048, 160, 6), (4096, 1024, 128, 8), (513, 4096, 256, 8),
                                     (16384, 5120, 160, 6)])
def test_fused_router_parity(cuda, T, H, E, k):
    X, W = make(T, H, E, seed=7 * T + E + k)
    check_fused(X, W, k)


# H < 512 is never split over workgroups (splits keep >= 256 of H), nor is a
# problem of >= 512 tiles, so these run the selection epilogue inside the
# GEMM kernel: the filtered path (K <= 16) and the rounds path (K > 16), E
# not a multiple of 16, all three tile widths (128, 192, 256 experts).
@pytest.mark.parametrize("T,H,E,k", [(3000, 504, 160, 6), (2000, 264, 256, 32), (1000, 392, 64, 16),
                                     (777, 456, 200, 17), (64, 8, 33, 3), (40000, 256, 160, 6)])
def test_fused_router_epilogue_in_kernel(cuda, T, H, E, k):
    X, W = make(T, H, E, seed=T + H + k, scale=0.1)
    check_fused(X, W, k)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_fused_router_dtypes_and_int64(cuda, dtype):
    X, W = make(300, 1536, 160, seed=3, dtype=dtype, scale=0.05)
    check_fused(X, W, 8)
    check_fused(X, W, 8, index_dtype=torch.int64)


def test_fused_router_exact_ties(cuda):
    """Zero tokens give all-equal logits; duplicated weight columns give
    equal pairs: the lower expert index comes first."""
    X, W = make(96, 256, 64, seed=9)
    X[:10] = 0
    W[:, 33] = W[:, 5]
    W[:, 40] = W[:, 5]
    s, i = check_fused(X, W, 8)
    assert (i[:10].cpu() == torch.arange(8, dtype=torch.int32)).all()
    torch.testing.assert_close(s[:10], torch.full((10, 8), 0.125, device=s.device), rtol=1e-6, atol=0)


def test_reference_factories_with_padded_weights(cuda):
    T, H, E, k = 256, 5120, 160, 6
    X, W = make(T, H, E, seed=11)
    Wp = torch.zeros(H, R._next_pow2(E), dtype=W.dtype, device=W.device)
    Wp[:, :E] = W
    s0, i0 = K.router_topk_softmax(X, W, k)
    for algo in R.FUSED_ALGOS:
        s, i = getattr(R, f"fused_router_{algo}_kernel")(T, H, E, R._next_pow2(E), k)(X, Wp)
        assert torch.equal(i, i0) and torch.equal(s, s0)
        s, i = R.get_fused_router_kernel(algo, T, H, E, k)(X, W)
        assert torch.equal(i, i0) and torch.equal(s, s0)
    lg = R.get_router_gemm_kernel(T, H, E)(X, W)
    assert lg.shape == (T, E)
    with pytest.raises(ValueError):
        R.get_fused_router_kernel("tma_bitonic", T + 1, H, E, k)(X, W)


def test_beyond_fused_limits_two_launches(cuda):
    X, W = make(200, 512, 300, seed=13)
    check_fused(X, W, 8)           # E > 256
    X, W = make(200, 512, 64, seed=14)
    check_fused(X, W, 40)          # K > 32


def test_weight_cache_follows_updates(cuda):
    X, W = make(128, 512, 64, seed=15)
    s0, i0 = K.router_topk_softmax(X, W, 4)
    W.mul_(-1)                     # in-place update bumps the version counter
    s1, i1 = K.router_topk_softmax(X, W, 4)
    lg = K.router_gemm(X, W)
    _, i2 = K.topk_softmax(lg, 4)
    assert torch.equal(i1, i2) and not torch.equal(i0, i1)


def test_empty_and_repeated_calls(cuda):
    X, W = make(0, 256, 64)
    s, i = K.router_topk_softmax(X, W, 4)
    assert s.shape == (0, 4)
    # The split path's counters must come back to zero: repeat with a
    # different token count on the same workspace.
    for T in (8, 200, 8, 64):
        X, W = make(T, 4096, 128, seed=T)
        check_fused(X, W, 8)


def test_strided_weight_view(cuda):
    """W given as a transposed view (unit row stride, column stride H): its
    first E rows are already the kernels' layout and are read in place (no
    copy, no cache entry), with the same results as the contiguous W."""
    g = torch.Generator(device="cuda").manual_seed(7)
    T, H, E, k = 96, 512, 48, 6
    X = torch.randn(T, H, generator=g, device="cuda").bfloat16()
    Wt_full = (torch.randn(E, H, generator=g, device="cuda") / H ** 0.5).bfloat16()
    W_view = Wt_full.t()  # [H, E], stride (1, H)
    assert W_view.stride(1) != 1
    W = W_view.contiguous()
    for a, b in zip(K.router_topk_softmax(X, W_view, k), K.router_topk_softmax(X, W, k)):
        assert torch.equal(a, b)
    assert torch.equal(K.router_gemm(X, W_view), K.router_gemm(X, W))
    Wt = R.transposed_weight(W_view, E)
    assert Wt.data_ptr() == Wt_full.data_ptr() and Wt.is_contiguous()
    # A padded transposed view (E of E + 16 rows) reads the first E rows.
    Wt_pad = (torch.randn(E + 16, H, generator=g, device="cuda") / H ** 0.5).bfloat16()
    assert torch.equal(K.router_gemm(X, Wt_pad.t(), E), K.router_gemm(X, Wt_pad[:E].t().contiguous()))
    # Neither unit stride: one contiguous copy, transposed.
    W_odd = Wt_full.t()[::2]  # [H/2, E], strides (2, H)
    X2 = X[:, : H // 2].contiguous()
    assert torch.equal(K.router_gemm(X2, W_odd), K.router_gemm(X2, W_odd.contiguous()))


@pytest.mark.parametrize("E,k", [(64, 8), (300, 4)])  # fused kernel; beyond the fused limit (two launches)
def test_prepared_weight_matches(cuda, E, k):
    g = torch.Generator(device="cuda").manual_seed(E)
    T, H = 200, 1024
    X = torch.randn(T, H, generator=g, device="cuda").bfloat16()
    W = (torch.randn(H, E, generator=g, device="cuda") / H ** 0.5).bfloat16()
    Wt = K.prepare_router_weight(W)
    assert Wt.shape == (E, H) and Wt.is_contiguous()
    assert torch.equal(Wt, W.t().contiguous())
    for a, b in zip(K.router_topk_softmax_prepared(X, Wt, k), K.router_topk_softmax(X, W, k)):
        assert torch.equal(a, b)
    with pytest.raises(ValueError):
        K.router_topk_softmax_prepared(X, W, k)  # [H, E] is not a prepared [E, H] weight


@pytest.mark.parametrize("H,E", [(136, 72), (64, 8), (520, 300), (1000, 160), (7168, 256)])
def test_weight_transpose_exact(cuda, H, E):
    """prepare_router_weight is an exact transpose: 16-byte path (H, E
    multiples of 8, partial 64x64 tiles included) and scalar path (E = 300)."""
    W = torch.randn(H, E, device="cuda").bfloat16()
    assert torch.equal(K.prepare_router_weight(W), W.t().contiguous())
    Wpad = torch.randn(H, E + 8, device="cuda").bfloat16()  # padded columns past E (row stride E + 8)
    assert torch.equal(K.prepare_router_weight(Wpad, E), Wpad[:, :E].t().contiguous())
    # Odd row stride E + 1, and a start 2 bytes past a 16-byte boundary: the
    # 16-byte transpose path must not be taken for either.
    base = torch.randn(H, E + 1, device="cuda").bfloat16()
    assert torch.equal(K.prepare_router_weight(base[:, :E]), base[:, :E].t().contiguous())
    W_mis = base[:, 1:E + 1]
    assert W_mis.data_ptr() % 16 != 0
    assert torch.equal(K.prepare_router_weight(W_mis), W_mis.t().contiguous())
