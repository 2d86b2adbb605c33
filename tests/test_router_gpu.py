"""GPU parity of the fused TopK+softmax router against the CPU oracle.

Bar: indices bit-exact with the oracle (value descending, ties by ascending
index); scores within 1e-6 relative of the fp64 softmax of the selected
values.  Covers every algorithm over ragged N and K, the three logits dtypes,
strided rows, heavy ties, signed zeros, infinities and NaN, the golden
fixtures, and the BASELINE configs at full size.
"""
import glob
import os

import numpy as np
import pytest
import torch

from conftest import GOLDEN
from oracle import router as orc
from tilelang_moe_amd import kernels as K

pytestmark = pytest.mark.gpu

SCORE_RTOL = 1e-6
ALGO_MAX_N = {"bitonic": 64, "selection": 1024, "radix": 1 << 30}


def run(x, k, algo="auto", idx=torch.int32):
    if idx == torch.int64:
        return K.topk_softmax_int64(x, k, algo)
    fn = {"auto": K.topk_softmax, "bitonic": K.topk_softmax_bitonic,
          "selection": K.topk_softmax_selection, "radix": K.topk_softmax_radix}[algo]
    return fn(x, k)


def check(x, k, algo="auto", idx=torch.int32, scores_nan_ok=False):
    s, i = run(x, k, algo, idx)
    torch.cuda.synchronize()
    assert i.dtype == idx and s.dtype == torch.float32 and tuple(i.shape) == (x.shape[0], k)
    xc = x.float().cpu().numpy()
    s_o, i_o = orc.topk_softmax(xc, k)
    i_g = i.cpu().numpy().astype(np.int64)
    bad = np.nonzero((i_g != i_o).any(axis=1))[0]
    assert bad.size == 0, f"{algo} N={x.shape[1]} k={k}: {bad.size} rows differ, first row {bad[0]}: " \
                          f"gpu {i_g[bad[0]][:16]} oracle {i_o[bad[0]][:16]}"
    s_g = s.cpu().numpy().astype(np.float64)
    if scores_nan_ok:
        assert (np.isnan(s_g) == np.isnan(s_o)).all()
        s_g, s_o = np.nan_to_num(s_g), np.nan_to_num(s_o)
    np.testing.assert_allclose(s_g, s_o, rtol=SCORE_RTOL, atol=0)
    return s, i


def _algos_for(n):
    return [a for a in ("bitonic", "selection", "radix") if n <= ALGO_MAX_N[a]]


# ---------------------------------------------------------------------------
@pytest.mark.parametrize("path", sorted(glob.glob(os.path.join(GOLDEN, "router_*.npz"))))
def test_golden_fixtures(cuda, path):
    d = np.load(path)
    k = int(d["k"])
    if "logits_bf16_bits" in d:
        x = torch.from_numpy(d["logits_bf16_bits"].view(np.int16)).view(torch.bfloat16).to(cuda)
    else:
        x = torch.from_numpy(d["logits"]).to(cuda)
    for algo in ["auto"] + _algos_for(x.shape[1]):
        s, i = check(x, k, algo, scores_nan_ok=True)
        np.testing.assert_array_equal(i.cpu().numpy(), d["canon_idx"])


@pytest.mark.parametrize("n", [1, 2, 3, 7, 16, 31, 33, 63, 64, 65, 100, 127, 128, 200, 256, 300, 511, 512,
                               513, 1000, 1024, 1500, 4096, 5000])
def test_ragged_shapes_all_algorithms(cuda, n):
    g = torch.Generator(device="cpu").manual_seed(n)
    x = torch.randn(37, n, generator=g).to(cuda)
    ks = sorted({1, min(n, 2), min(n, 6), min(n, 64), min(n, 257), n})
    for algo in _algos_for(n):
        for k in ks:
            if algo == "selection" and k > 1024:
                continue
            check(x, k, algo)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("n,k", [(8, 2), (64, 6), (160, 6), (256, 8), (2048, 64), (32768, 2048)])
def test_half_dtypes_with_ties(cuda, dtype, n, k):
    g = torch.Generator(device="cpu").manual_seed(n * 7 + k)
    x = torch.randn(96, n, generator=g).to(dtype).to(cuda)
    for algo in ["auto"] + _algos_for(n):
        check(x, k, algo)


def test_heavy_ties_and_equal_rows(cuda):
    g = torch.Generator(device="cpu").manual_seed(5)
    for n, k in [(64, 6), (48, 48), (256, 8), (300, 100), (4096, 1000), (9000, 4000)]:
        x = torch.randint(-3, 4, (24, n), generator=g).float()
        x[0] = 1.25        # all equal
        x[1, :] = 0.0
        x[1, ::3] = -0.0   # signed zeros are equal
        x = x.to(cuda)
        for algo in _algos_for(n):
            check(x, k, algo)


def test_infinities_and_nan(cuda):
    x = torch.randn(8, 700)
    x[0, 5] = float("inf")
    x[0, 600] = float("inf")
    x[1, :] = float("-inf")
    x[1, 17] = 0.0
    x[2, 3] = float("nan")
    x[2, 400] = float("nan")
    x[3, 10] = -float("inf")
    x = x.to(cuda)
    for n in (40, 200, 700):
        for algo in _algos_for(n):
            check(x[:, :n].contiguous(), 4, algo, scores_nan_ok=True)


@pytest.mark.parametrize("k", [1, 100, 2048, 6000, 8192])
def test_radix_adversarial_rows_full_length(cuda, k):
    """Rows of the C2 length whose value distributions drive the radix
    kernel off its common path: candidates crowding one ordering bucket
    (bitonic fallback), a narrow key range, ties at the K-th value (exact
    threshold, lowest columns among the ties), more candidates than the
    candidate buffer holds, two clusters, a heavy tail."""
    n = 32768
    g = torch.Generator(device="cpu").manual_seed(k)
    rows = [
        1e-4 * torch.arange(n, dtype=torch.float32),                 # sorted, unique (scores stay normal floats)
        torch.flip(1e-4 * torch.arange(n, dtype=torch.float32), [0]),  # reverse sorted
        1.0 + 1e-6 * torch.randn(n, generator=g),                    # narrow key range
        torch.cat([torch.zeros(n // 2), 100.0 + torch.rand(n // 2, generator=g)]),  # two clusters
        torch.empty(n).exponential_(1.0, generator=g),                # heavy tail
        torch.randint(0, 3, (n,), generator=g).float(),               # three values: ties everywhere
    ]
    ties = torch.randn(n, generator=g)
    kth = torch.sort(ties, descending=True).values[min(k, n) - 1]
    ties[torch.randperm(n, generator=g)[:5000]] = kth                 # many copies of the K-th value
    rows.append(ties)
    crowd = torch.randn(n, generator=g)
    crowd[:3000] = 3.0 + 1e-7 * torch.arange(3000, dtype=torch.float32)  # one dense bucket near the top
    rows.append(crowd)
    x = torch.stack(rows).to(cuda)
    for _ in range(2):
        check(x, k, "radix")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("n", [4096, 8192, 16384, 32768])
def test_radix_full_rows_and_neighbours(cuda, dtype, n):
    """Rows of exactly 1024 x (keys per thread) columns take the radix
    kernel's full-row instantiation (no per-key range checks); rows one
    column shorter or longer take the general one.  Both, on rows with
    NaN, -0.0 next to +0.0, ties at the K-th value and a plain row."""
    k = min(2048, n // 4)
    for width in (n - 1, n, n + 1):
        g = torch.Generator(device="cpu").manual_seed(width)
        x = torch.randn(6, width, generator=g)
        x[0, width - 1] = float("nan")          # last column: the end of the last vector
        x[1, :] = 0.0
        x[1, 1::2] = -0.0
        x[1, 7] = 1.0
        x[2, :] = torch.randint(0, 4, (width,), generator=g).float()
        x[3, 0] = float("inf")
        x[4, -3:] = 6.0                         # winners in the last columns (x - max stays
                                                # small enough for fp32 to round it within 5e-7)
        x = x.to(dtype).to(cuda)
        check(x, k, "radix", scores_nan_ok=True)


@pytest.mark.parametrize("m,n,k", [(8, 40000, 100), (64, 65536, 2048), (3, 65536, 512), (17, 50000, 4096),
                                   (2, 300000, 16), (256, 32769, 64), (5, 1 << 20, 8)])
def test_split_rows(cuda, m, n, k):
    """Rows longer than one workgroup's registers hold: several workgroups
    share a row (split-row radix)."""
    g = torch.Generator(device="cpu").manual_seed(n + k)
    x = torch.randn(m, n, generator=g)
    x[0, 5] = float("nan")
    x[0, 77] = float("inf")
    x[1 % m, :] = 0.0
    x[1 % m, ::5] = -0.0
    x[2 % m, 1000:] = x[2 % m, 1000]  # long run of ties
    x = x.to(cuda)
    for _ in range(3):  # the row counters of the workspace must come back to zero
        check(x, k, "radix", scores_nan_ok=True)
    check(x.bfloat16(), min(k, 64), "radix", scores_nan_ok=True)


def test_workspace_shared_across_calls(cuda):
    """Split-row calls of different row counts and a grouped GEMM share one
    workspace on one stream; each must find the control block zeroed."""
    g = torch.Generator(device="cpu").manual_seed(11)
    xs = {m: torch.randn(m, 40000, generator=g).to(cuda) for m in (4, 16, 64, 32)}
    X = torch.randn(256, 512, generator=g).bfloat16().to(cuda)
    W = torch.randn(8, 256, 512, generator=g).bfloat16().to(cuda)
    ids = torch.randint(0, 8, (256,), generator=g).int().to(cuda)
    for m in (4, 16, 64, 32, 4, 64):
        check(xs[m], 2048, "radix")
        K.grouped_gemm(X, W, ids)
    check(xs[64], 1000, "radix")


def test_strided_rows_and_int64(cuda):
    g = torch.Generator(device="cpu").manual_seed(3)
    base = torch.randn(50, 1200, generator=g).to(cuda)
    for n in (60, 300, 1100):
        x = base[:, :n]  # row stride 1200
        assert not x.is_contiguous()
        for algo in _algos_for(n):
            check(x, 5, algo)
            check(x, 5, algo, idx=torch.int64)


def test_empty_batch_and_radix_indices_only(cuda):
    s, i = K.topk_softmax(torch.empty(0, 128, device=cuda), 6)
    assert s.shape == (0, 6) and i.shape == (0, 6)
    x = torch.randn(16, 3000, device=cuda)
    idx = K.topk_radix(x, 100)
    _, i_o = orc.topk_softmax(x.cpu().numpy(), 100)
    np.testing.assert_array_equal(idx.cpu().numpy(), i_o)
    assert K.topk_radix_tilelang is K.topk_radix


def test_invalid_arguments_raise(cuda):
    x = torch.randn(4, 100, device=cuda)
    with pytest.raises(ValueError):
        K.topk_softmax(x, 0)
    with pytest.raises(ValueError):
        K.topk_softmax(x, 101)
    with pytest.raises(ValueError):
        K.topk_softmax_bitonic(x, 4)  # N > 64
    with pytest.raises(ValueError):
        K.topk_softmax(x.to(torch.int32), 4)


# ---------------------------------------------------------------------------
# BASELINE configurations at full size (seeds 0..2).
# ---------------------------------------------------------------------------
def _logits(seed, m, n, bf16=False):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(m, n, generator=g)
    return x.bfloat16() if bf16 else x


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_config1_selection_320x128_k6(cuda, seed):
    x = _logits(seed, 320, 128).to(cuda)
    assert K.select_strategy(128, 6) == "selection"
    check(x, 6)


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_config2_radix_64x32768_k2048(cuda, seed):
    x = _logits(seed, 64, 32768).to(cuda)
    assert K.select_strategy(32768, 2048) == "radix"
    s, i = check(x, 2048)
    # Size-independent properties: rows sum to 1, scores non-increasing,
    # indices unique, scores equal softmax of the gathered logits.
    torch.testing.assert_close(s.sum(-1), torch.ones(64, device=cuda), rtol=0, atol=2e-6)
    assert (s[:, 1:] <= s[:, :-1]).all()
    assert (i.sort(-1).values.diff(dim=-1) > 0).all()
    ref = torch.softmax(torch.gather(x, 1, i.long()).double(), -1)
    torch.testing.assert_close(s.double(), ref, rtol=SCORE_RTOL, atol=0)


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_config3_bf16_ties(cuda, seed):
    xa = _logits(seed, 4096, 64, bf16=True).to(cuda)
    xb = _logits(seed, 4096, 256, bf16=True).to(cuda)
    assert K.select_strategy(64, 6) == "bitonic" and K.select_strategy(256, 8) == "selection"
    for x, k in ((xa, 6), (xb, 8)):
        _, i = check(x, k)
        ties = orc.tie_rows(x.float().cpu().numpy(), k)
        assert ties.sum() > 100  # the config exists to exercise the tie rule
        # Report how torch.topk (on this GPU) orders the tied rows.
        _, it = torch.topk(x, k, dim=-1)
        diff = (it.cpu() != i.cpu().long()).any(-1).numpy()
        print(f"N={x.shape[1]} k={k}: tie rows {int(ties.sum())}, torch.topk(gpu) differs on "
              f"{int(diff.sum())} rows, all of them tie rows: {bool((diff <= ties).all())}")
        assert (diff <= ties).all()  # differences only on tie rows


# ---------------------------------------------------------------------------
# Score conventions (reference kernels/topk_softmax_baseline.py).
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("n,k,algo", [(64, 6, "bitonic"), (256, 8, "selection"), (1000, 64, "selection"),
                                      (4096, 100, "radix"), (32768, 2048, "radix"), (40000, 512, "radix")])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_convention_a_all_algorithms(cuda, n, k, algo, dtype):
    """Convention A: same indices as Convention B, scores = the float64
    softmax over the whole row read at them, within 1e-5 relative (fp32
    running sums over up to 40000 terms)."""
    g = torch.Generator(device="cpu").manual_seed(n + k)
    x = torch.randn(9, n, generator=g).to(dtype)
    x[0, :] = 0.5  # all equal: scores 1/n
    x = x.to(cuda)
    sa, ia = K.topk_softmax_scores(x, k, "A", algo)
    sb, ib = K.topk_softmax_scores(x, k, "B", algo)
    sr, ir = K.topk_softmax_scores(x, k, "A_renorm", algo)
    torch.cuda.synchronize()
    assert torch.equal(ia, ib) and torch.equal(ir, ib) and torch.equal(sr, sb)
    s_o, i_o = orc.topk_softmax_conv_a(x.float().cpu().numpy(), k)
    np.testing.assert_array_equal(ia.cpu().numpy(), i_o)
    np.testing.assert_allclose(sa.cpu().double().numpy(), s_o, rtol=1e-5, atol=0)
    # Convention A scores renormalised over the K are Convention B's.
    torch.testing.assert_close(sa / sa.sum(-1, keepdim=True), sb, rtol=2e-5, atol=0)


def test_convention_a_special_values(cuda):
    x = torch.randn(4, 300)
    x[0, 5] = float("nan")
    x[1, :] = float("-inf")
    x[1, 7] = 2.0
    x[2, 9] = float("inf")
    x = x.to(cuda)
    s, i = K.topk_softmax_separate(x, 4)
    s_o, i_o = orc.topk_softmax_conv_a(x.cpu().numpy(), 4)
    np.testing.assert_array_equal(i.cpu().numpy(), i_o)
    s = s.cpu().double().numpy()
    assert np.isnan(s[0]).all()
    np.testing.assert_allclose(s[1], s_o[1], rtol=1e-6)  # one finite value: 1, then zeros
    assert np.isnan(s[2]).all() == np.isnan(s_o[2]).all()


@pytest.mark.parametrize("m,n,k", [(64, 32768, 2048), (3, 65536, 512), (40, 5000, 1000)])
def test_radix_scores_bitwise_reproducible(cuda, m, n, k):
    """Softmax normalisers are summed in rank order, so repeated calls give
    identical bits whatever order the candidates reached threads in."""
    x = torch.randn(m, n, generator=torch.Generator().manual_seed(n)).to(cuda)
    s0, i0 = K.topk_softmax_radix(x, k)
    for _ in range(5):
        s, i = K.topk_softmax_radix(x, k)
        assert torch.equal(i, i0) and torch.equal(s, s0)
