"""Pin the CPU oracle (oracle/) before it is trusted to check the GPU.

Each oracle function is checked against something it does not share code
with: a pure-Python brute force, torch's CPU operators (via the golden
fixtures and directly), closed forms, and the reference's own convention
identity.  A plausible slip in the oracle (a sign flip in the key mapping,
ascending instead of descending, ties by the wrong index, a dropped softmax
term, a transposed weight) fails at least one test here.
"""
import glob
import math
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from conftest import GOLDEN
from oracle import gemm as og
from oracle import router as orc
from oracle import torch_baseline as tb


def _fixtures(prefix):
    paths = sorted(glob.glob(os.path.join(GOLDEN, prefix + "*.npz")))
    assert paths, f"no fixtures {prefix}*"
    return paths


# --------------------------------------------------------------------------
# Router oracle
# --------------------------------------------------------------------------
def test_sortable_keys_order_and_specials():
    vals = np.array([-np.inf, -3.5, -1e-30, -0.0, 0.0, 1e-30, 2.0, np.inf, np.nan], np.float32)
    k = orc.sortable_keys(vals)
    assert (np.diff(k[:4].astype(np.int64)) > 0).all()
    assert k[3] == k[4]  # -0 == +0
    assert (np.diff(k[4:].astype(np.int64)) > 0).all()
    assert k[-1] == 0xFFFFFFFF
    assert k.min() > 0  # key 0 is reserved for padding
    # Monotone on a dense random sample, both signs.
    x = np.sort(np.random.default_rng(0).standard_normal(10000).astype(np.float32))
    assert (np.diff(orc.sortable_keys(x).astype(np.int64)) >= 0).all()


@pytest.mark.parametrize("seed", range(6))
def test_topk_matches_bruteforce_with_ties_and_specials(seed):
    rng = np.random.default_rng(seed)
    M, N = 12, 37
    x = rng.integers(-4, 5, size=(M, N)).astype(np.float32) * 0.5  # many ties
    x[0, 3] = -0.0
    x[0, 7] = 0.0
    x[1, :] = 0.0
    x[2, 5] = np.inf
    x[3, 9] = -np.inf
    x[4, 11] = np.nan
    x[4, 2] = np.nan
    for k in (1, 3, 8, N):
        idx = orc.topk_order(x, k)
        for r in range(M):
            assert idx[r].tolist() == orc.topk_bruteforce(x[r].tolist(), k), (r, k)


def test_topk_closed_forms():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((20, 50)).astype(np.float32)
    x[::3, 10] = x[::3, 40]  # plant ties
    full = orc.topk_order(x, 50)
    ref_full = torch.sort(torch.from_numpy(x), dim=1, descending=True, stable=True).indices.numpy()
    np.testing.assert_array_equal(full, ref_full)
    one = orc.topk_order(x, 1)[:, 0]
    np.testing.assert_array_equal(one, np.argmax(x, axis=1))  # numpy argmax = first max
    s, _ = orc.topk_softmax(x, 1)
    assert (s == 1.0).all()


def test_softmax64_closed_form():
    v = np.array([[3.0, 1.0, -2.0], [0.0, 0.0, 0.0]])
    s = orc.softmax64(v)
    e = np.exp([0.0, -2.0, -5.0])
    np.testing.assert_allclose(s[0], e / e.sum(), rtol=1e-15)
    np.testing.assert_allclose(s[1], [1 / 3] * 3, rtol=1e-15)


@pytest.mark.parametrize("path", _fixtures("router_"))
def test_router_oracle_vs_golden(path):
    d = np.load(path)
    x, k = d["logits"], int(d["k"])
    scores, idx = orc.topk_softmax(x, k)
    # Canonical order from torch.sort(stable=True): identical everywhere.
    np.testing.assert_array_equal(idx, d["canon_idx"])
    np.testing.assert_allclose(scores, d["canon_scores64"], rtol=1e-12, atol=0)
    # torch.topk: identical on rows without ties.
    ties = orc.tie_rows(x, k)
    clean = ~ties
    np.testing.assert_array_equal(idx[clean], d["torch_idx"][clean])
    # torch's fp32 softmax agrees with the fp64 closed form to 1e-6 relative.
    np.testing.assert_allclose(d["torch_scores"][clean], scores[clean], rtol=1e-6, atol=0)
    # Same multiset of selected values on every row, tied or not.
    tv = np.sort(np.take_along_axis(x, d["torch_idx"], 1), axis=1)
    ov = np.sort(np.take_along_axis(x, idx, 1), axis=1)
    np.testing.assert_array_equal(np.nan_to_num(tv), np.nan_to_num(ov))


def test_router_oracle_vs_torch_topk_on_tie_free_rows():
    g = torch.Generator().manual_seed(11)
    for M, N, k in [(320, 128, 6), (64, 4096, 512), (128, 64, 6)]:
        x = torch.randn(M, N, generator=g)
        s_t, i_t = tb.topk_softmax_fused(x, k)
        s_o, i_o = orc.topk_softmax(x.numpy(), k)
        clean = ~orc.tie_rows(x.numpy(), k)
        assert clean.mean() > 0.9
        np.testing.assert_array_equal(i_o[clean], i_t.numpy()[clean])
        np.testing.assert_allclose(s_t.numpy(), s_o, rtol=1e-6)


def test_reference_convention_identity():
    """The reference's tests/test_topk_softmax_conventions.py:58-69 checks that
    Conv A-norenorm, A-renorm and B pick the same expert sets and that A-renorm
    scores equal B's (max diff 1.19e-7 published, RESULT.md:36-49).  The
    oracle's Convention-B output must satisfy the same identities."""
    g = torch.Generator().manual_seed(42)
    for E, K in [(8, 2), (16, 4), (128, 8), (160, 6), (64, 8)]:
        x = torch.randn(512, E, generator=g)
        s_b, i_b = orc.topk_softmax(x.numpy(), K)
        s_a, i_a = tb.topk_softmax_conv_a_renorm(x, K)
        assert (np.sort(i_b, 1) == np.sort(i_a.numpy(), 1)).all()
        assert np.abs(s_a.numpy() - s_b).max() < 5e-7


# --------------------------------------------------------------------------
# Routing sort and grouped GEMM oracle
# --------------------------------------------------------------------------
@pytest.mark.parametrize("seed", range(4))
def test_route_sort_vs_bruteforce(seed):
    rng = np.random.default_rng(seed)
    E = int(rng.integers(1, 20))
    ids = rng.integers(-2, E + 3, size=int(rng.integers(0, 300)))
    c, o, s = og.route_sort(ids, E)
    bc, bo, bs = og.route_sort_bruteforce(ids, E)
    assert c.tolist() == bc and o.tolist() == bo and s.tolist() == bs


def test_gemm_oracle_vs_bruteforce():
    rng = np.random.default_rng(5)
    T, H, I, E, topk = 6, 7, 5, 4, 2
    X = rng.standard_normal((T, H))
    W = rng.standard_normal((E, I, H))
    ids = rng.integers(-1, E + 1, size=T * topk)
    np.testing.assert_allclose(og.grouped_gemm(X, W, ids, topk), og.grouped_gemm_bruteforce(X, W, ids, topk),
                               rtol=1e-12, atol=1e-12)


def test_gemm_oracle_linearity_and_repeat_identity():
    rng = np.random.default_rng(6)
    T, H, I, E, topk = 10, 16, 8, 3, 3
    X1, X2 = rng.standard_normal((2, T, H))
    W = rng.standard_normal((E, I, H))
    ids = rng.integers(0, E, size=T * topk)
    y = og.grouped_gemm(2.0 * X1 - X2, W, ids, topk)
    np.testing.assert_allclose(y, 2.0 * og.grouped_gemm(X1, W, ids, topk) - og.grouped_gemm(X2, W, ids, topk),
                               atol=1e-10)
    np.testing.assert_allclose(og.grouped_gemm(X1, W, ids, topk),
                               og.grouped_gemm(np.repeat(X1, topk, axis=0), W, ids, 1), atol=0)


@pytest.mark.parametrize("path", _fixtures("gemm_"))
def test_gemm_oracle_vs_golden(path):
    d = np.load(path)
    X = torch.from_numpy(d["X_bits"].view(np.int16)).view(torch.bfloat16).float().numpy()
    W = torch.from_numpy(d["W_bits"].view(np.int16)).view(torch.bfloat16).float().numpy()
    Y = og.grouped_gemm(X, W, d["ids"])
    np.testing.assert_allclose(Y, d["Y_fp32"], rtol=1e-5, atol=1e-5)
    # The torch bf16 loop (the reference baseline's own dtype) is within bf16 rounding.
    Yb = torch.from_numpy(d["Y_bf16_bits"].view(np.int16)).view(torch.bfloat16).float().numpy()
    np.testing.assert_allclose(Yb, Y, rtol=1e-2, atol=1e-2)
    # Experts with no rows and rows of absent experts are exactly zero.
    E = int(d["E"])
    bad = (d["ids"] < 0) | (d["ids"] >= E)
    assert (Y[bad] == 0).all()


def test_torch_baseline_gemm_loop_matches_oracle():
    g = torch.Generator().manual_seed(9)
    X = torch.randn(40, 24, generator=g)
    W = torch.randn(5, 12, 24, generator=g)
    ids = torch.randint(-1, 6, (40,), generator=g)
    np.testing.assert_allclose(tb.grouped_gemm_loop(X, W, ids).numpy(), og.grouped_gemm(X.numpy(), W.numpy(), ids.numpy()),
                               rtol=1e-5, atol=1e-5)


# ---------------------------------------------------------------------------
# Router GEMM oracle
# ---------------------------------------------------------------------------
from oracle import router_gemm as org  # noqa: E402


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_router_gemm_oracle_vs_bruteforce(seed):
    """Small exact-integer inputs: the logits are exact, so the fp64 matmul
    must equal the triple loop, and the top-K must equal repeated scans
    (integer logits tie often, so the lower-index rule is exercised)."""
    rng = np.random.default_rng(seed)
    X = rng.integers(-3, 4, size=(9, 13)).astype(np.float32)
    W = rng.integers(-2, 3, size=(13, 11)).astype(np.float32)
    lg = org.logits_fp64(X, W)
    np.testing.assert_array_equal(lg, np.array(org.brute_logits(X.tolist(), W.tolist())))
    for k in (1, 3, 11):
        idx = org.topk_order(lg, k)
        for t in range(lg.shape[0]):
            assert idx[t].tolist() == org.brute_topk(lg[t].tolist(), k)


def test_router_gemm_oracle_closed_forms():
    rng = np.random.default_rng(5)
    lg = rng.standard_normal((7, 20))
    s, i = org.topk_softmax_fp64(lg, 20)  # K == E: full stable sort
    np.testing.assert_array_equal(i, np.argsort(-lg, axis=1, kind="stable"))
    np.testing.assert_allclose(s.sum(axis=1), 1.0, rtol=0, atol=1e-15)
    np.testing.assert_allclose(org.softmax_at(lg, i[:, :4]), org.topk_softmax_fp64(lg, 4)[0], rtol=1e-15)
    # Conv B softmax of the top-k equals the renormalised full softmax (Z cancels).
    full = np.exp(lg - lg.max(1, keepdims=True))
    full /= full.sum(1, keepdims=True)
    top = np.take_along_axis(full, i[:, :4], 1)
    np.testing.assert_allclose(top / top.sum(1, keepdims=True), org.topk_softmax_fp64(lg, 4)[0], rtol=1e-13)


def test_conv_a_oracle_vs_torch_separate():
    """Convention A oracle == the reference baseline topk_softmax_separate
    (torch CPU softmax then topk) on tie-free rows; with K == N the scores
    are the whole softmax and sum to 1."""
    g = torch.Generator().manual_seed(4)
    x = torch.randn(50, 300, generator=g)
    for k in (1, 6, 64):
        s_t, i_t = tb.topk_softmax_separate(x, k)
        s_o, i_o = orc.topk_softmax_conv_a(x.numpy(), k)
        clean = ~orc.tie_rows(x.numpy(), k)
        np.testing.assert_array_equal(i_o[clean], i_t.numpy()[clean])
        np.testing.assert_allclose(s_o, s_t.double().numpy(), rtol=2e-6, atol=0)
    s_all, _ = orc.topk_softmax_conv_a(x.numpy(), 300)
    np.testing.assert_allclose(s_all.sum(1), 1.0, rtol=0, atol=1e-12)
    xn = x.numpy().copy()
    xn[3, 7] = np.nan
    assert np.isnan(orc.topk_softmax_conv_a(xn, 4)[0][3]).all()


# ---------------------------------------------------------------------------
# FusedMoE oracle
# ---------------------------------------------------------------------------
from oracle import fusedmoe as ofm  # noqa: E402


def _moe_inputs(T, Dh, De, Ds, E, seed=0):
    rng = np.random.default_rng(seed)
    r = lambda *s: rng.standard_normal(s) / np.sqrt(s[-1])  # noqa: E731
    return (r(T, Dh), r(E, Dh), r(Ds, Dh), r(Ds, Dh), r(Dh, Ds), r(E, De, Dh), r(E, De, Dh), r(E, Dh, De))


def test_fusedmoe_oracle_closed_forms():
    x, rw, sg, su, sd, rg, ru, rd = _moe_inputs(7, 16, 8, 8, 3)
    # One expert, k = 1: the dense SwiGLU FFN (weight 1), plus the shared part.
    out = ofm.fusedmoe(x, rw[:1], sg, su, sd, rg[:1], ru[:1], rd[:1], 1)
    np.testing.assert_allclose(out, ofm.expert(x, sg, su, sd) + ofm.expert(x, rg[0], ru[0], rd[0]), rtol=1e-12)
    # Zero router weights, k = E: every expert with weight 1/E; no shared expert.
    out = ofm.fusedmoe(x, np.zeros_like(rw), None, None, None, rg, ru, rd, 3)
    avg = sum(ofm.expert(x, rg[e], ru[e], rd[e]) for e in range(3)) / 3
    np.testing.assert_allclose(out, avg, rtol=1e-12)
    # Routing equals Convention A of oracle.router on the same logits.
    w, ids = ofm.route(x, rw, 2)
    s_o, i_o = orc.topk_softmax_conv_a((x @ rw.T).astype(np.float32), 2)
    np.testing.assert_array_equal(ids, i_o)
    np.testing.assert_allclose(w, s_o, rtol=1e-6)
    # silu against its definition at a few points.
    np.testing.assert_allclose(ofm.silu(np.array([0.0, 1.0, -2.0])), [0.0, 1 / (1 + np.exp(-1)), -2 / (1 + np.exp(2))])
