"""GPU parity of the routing sort (bit-exact vs the oracle) and the expert
grouped GEMM (rtol = atol = 1e-2 against an fp32-accumulated reference, the
north-star tolerance), over ragged and degenerate routings and the BASELINE
GEMM configurations."""
import glob
import os

import numpy as np
import pytest
import torch

from conftest import GOLDEN
from oracle import gemm as og
from tilelang_moe_amd import kernels as K

pytestmark = pytest.mark.gpu

RTOL = ATOL = 1e-2


def ref_fp32(X, W, ids, topk=1):
    """Plain PyTorch fp32 reference: per-expert fp32 matmul, zero rows for
    ids outside [0, E) (grouped_gemm_loop semantics)."""
    ids = ids.reshape(-1).long()
    E, I, _ = W.shape
    Y = torch.zeros(ids.numel(), I, dtype=torch.float32, device=X.device)
    for e in torch.unique(ids).tolist():
        if not 0 <= e < E:
            continue
        rows = torch.nonzero(ids == e).squeeze(1)
        Y[rows] = X[rows // topk].float() @ W[e].float().T
    return Y


def check_gemm(X, W, ids, topk=1):
    Y = K.grouped_gemm(X, W, ids)
    torch.cuda.synchronize()
    assert Y.dtype == X.dtype and Y.shape == (ids.numel(), W.shape[1])
    torch.testing.assert_close(Y.float(), ref_fp32(X, W, ids, topk), rtol=RTOL, atol=ATOL)
    return Y


def make(T, H, I, E, seed=0, dtype=torch.bfloat16, device="cuda"):
    g = torch.Generator().manual_seed(seed)
    X = torch.randn(T, H, generator=g).to(dtype).to(device)
    W = (0.02 * torch.randn(E, I, H, generator=g)).to(dtype).to(device)
    return X, W


# ---------------------------------------------------------------------------
# Routing sort
# ---------------------------------------------------------------------------
# One workgroup sorts up to 2048 rows of up to 256 experts, and up to 4096
# rows of 256 experts (route_small_kernel): (2048, 8), (2048, 256) and
# (4096, 256) are its largest cases, (2049, 8), (4097, 256) and (2048, 257)
# just beyond.  Above 255 experts the sort takes three kernels, below it two
# (the scan folded into the scatter); (8192, 1) puts every row in one bucket.
@pytest.mark.parametrize("R,E", [(0, 4), (1, 1), (255, 8), (256, 8), (257, 8), (1000, 1), (2048, 8), (2049, 8),
                                 (2048, 256), (4096, 255), (4096, 256), (4097, 256),
                                 (2048, 257), (4097, 128), (6000, 9), (8192, 128), (8192, 1), (8193, 128),
                                 (8192, 129), (5000, 256), (32768, 256), (40000, 4096), (300000, 64)])
@pytest.mark.parametrize("idt", [torch.int32, torch.int64])
def test_route_sort_bit_exact(cuda, R, E, idt):
    g = torch.Generator().manual_seed(R + E)
    ids = torch.randint(-2, E + 2, (R,), generator=g).to(idt)
    c, o, s = K.route_sort(ids.to(cuda), E)
    c_o, o_o, s_o = og.route_sort(ids.numpy(), E)
    np.testing.assert_array_equal(c.cpu().numpy(), c_o)
    np.testing.assert_array_equal(o.cpu().numpy(), o_o)
    np.testing.assert_array_equal(s.cpu().numpy(), s_o)


def test_route_sort_skewed(cuda):
    g = torch.Generator().manual_seed(0)
    bias = 1.5 * torch.randn(256, generator=g)
    ids = torch.topk(torch.randn(4096, 256, generator=g) + bias, 8).indices
    c, o, s = K.route_sort(ids.to(cuda), 256)
    c_o, o_o, s_o = og.route_sort(ids.numpy(), 256)
    np.testing.assert_array_equal(s.cpu().numpy(), s_o)
    assert (c.cpu().numpy() == 0).sum() > 10  # some experts are empty


# ---------------------------------------------------------------------------
# Grouped GEMM
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("path", sorted(glob.glob(os.path.join(GOLDEN, "gemm_*.npz"))))
def test_golden_fixtures(cuda, path):
    d = np.load(path)
    X = torch.from_numpy(d["X_bits"].view(np.int16)).view(torch.bfloat16).to(cuda)
    W = torch.from_numpy(d["W_bits"].view(np.int16)).view(torch.bfloat16).to(cuda)
    ids = torch.from_numpy(d["ids"]).to(cuda)
    Y = K.grouped_gemm(X, W, ids)
    torch.testing.assert_close(Y.float().cpu(), torch.from_numpy(d["Y_fp32"]), rtol=RTOL, atol=ATOL)


@pytest.mark.parametrize("T,H,I,E", [(1, 8, 1, 1), (7, 64, 32, 3), (300, 72, 200, 5), (513, 1000, 129, 17),
                                     (2048, 512, 384, 64), (64, 4096, 256, 256)])
def test_ragged_shapes(cuda, T, H, I, E):
    X, W = make(T, H, I, E, seed=T + H)
    ids = torch.randint(0, E, (T,), generator=torch.Generator().manual_seed(T)).to(cuda)
    check_gemm(X, W, ids)


def test_degenerate_routings(cuda):
    X, W = make(777, 256, 160, 12, seed=1)
    g = torch.Generator().manual_seed(2)
    # all rows on one expert
    check_gemm(X, W, torch.full((777,), 7, device=cuda))
    # most experts empty
    ids = torch.randint(0, 2, (777,), generator=g) * 11
    check_gemm(X, W, ids.to(cuda))
    # ids outside [0, E) give zero rows
    ids = torch.randint(-3, 15, (777,), generator=g).to(cuda)
    Y = check_gemm(X, W, ids)
    bad = (ids < 0) | (ids >= 12)
    assert bad.any() and (Y[bad] == 0).all()
    # every row invalid
    Y = K.grouped_gemm(X, W, torch.full((777,), 99, device=cuda))
    assert (Y == 0).all()


def test_int32_ids_fp16_and_empty(cuda):
    X, W = make(200, 128, 96, 6, seed=4, dtype=torch.float16)
    ids = torch.randint(0, 6, (200,), generator=torch.Generator().manual_seed(4)).to(torch.int32).to(cuda)
    check_gemm(X, W, ids)
    Y = K.grouped_gemm(X[:0], W, ids[:0])
    assert Y.shape == (0, 96)


def test_topk_gather_identity(cuda):
    """ids [T, topk] with X [T, H] == the reference applied to the expanded X."""
    T, topk, E = 333, 4, 10
    X, W = make(T, 256, 192, E, seed=8)
    ids = torch.topk(torch.randn(T, E, generator=torch.Generator().manual_seed(8)), topk).indices.to(cuda)
    Y2 = check_gemm(X, W, ids, topk)
    Y1 = K.grouped_gemm(X.repeat_interleave(topk, 0), W, ids.flatten())
    assert torch.equal(Y1, Y2)


def test_invalid_arguments_raise(cuda):
    X, W = make(4, 64, 32, 2)
    with pytest.raises(ValueError):
        K.grouped_gemm(X.float(), W.float(), torch.zeros(4, dtype=torch.int64, device=cuda))
    with pytest.raises(ValueError):
        K.grouped_gemm(X, W[:, :, :32], torch.zeros(4, dtype=torch.int64, device=cuda))
    with pytest.raises(ValueError):
        K.grouped_gemm(X, W, torch.zeros(5, dtype=torch.int64, device=cuda))


def test_large_tiles_ragged(cuda):
    """Problems big enough for the largest tiles, with H not a multiple of
    the k-tile, I not a multiple of the n-tile, one crowded expert and
    invalid ids."""
    T, topk, E, H, I = 8192, 2, 16, 1000, 1900
    X, W = make(T, H, I, E, seed=21)
    g = torch.Generator().manual_seed(21)
    ids = torch.randint(0, E, (T, topk), generator=g)
    ids[:2000, 0] = 3                                    # crowded expert
    ids[::97, 1] = torch.randint(E, E + 5, (ids[::97, 1].numel(),), generator=g)  # invalid
    Y = check_gemm(X, W, ids.to(cuda), topk)
    bad = ((ids < 0) | (ids >= E)).flatten().to(cuda)
    assert bad.any() and (Y[bad] == 0).all()
    # all rows on one expert
    check_gemm(X, W, torch.full((T, topk), 5, device=cuda), topk)


def test_config4_fusedmoe_test_shape(cuda):
    """T=4096, H=1024, I=256, E=8, top-2 from topk of N(0,1) logits -> 8192 rows."""
    g = torch.Generator().manual_seed(0)
    idx = torch.topk(torch.randn(4096, 8, generator=g), 2).indices
    X = torch.randn(4096, 1024, generator=g).bfloat16().to(cuda)
    W = (0.02 * torch.randn(8, 256, 1024, generator=g)).bfloat16().to(cuda)
    idx = idx.to(cuda)
    Y = check_gemm(X, W, idx, 2)
    Y1 = K.grouped_gemm(X.repeat_interleave(2, 0), W, idx.flatten())  # reference 1-D semantics
    assert torch.equal(Y, Y1)


def _c5_weights(cuda):
    gc = torch.Generator(device=cuda).manual_seed(0)
    W = torch.empty(256, 2048, 7168, dtype=torch.bfloat16, device=cuda)
    for e in range(0, 256, 32):
        W[e:e + 32] = (0.02 * torch.randn(32, 2048, 7168, generator=gc, device=cuda)).bfloat16()
    return W, gc


def _check_every_expert(Y, X, W, flat, x_row):
    """Compares every row of every non-empty expert with an fp32 matmul of
    that expert (x_row maps routed rows to X rows)."""
    counts = torch.bincount(flat, minlength=W.shape[0])
    checked = 0
    for e in torch.nonzero(counts).squeeze(1).tolist():
        rows = torch.nonzero(flat == e).squeeze(1)
        ref = X[x_row(rows)].float() @ W[e].float().T
        torch.testing.assert_close(Y[rows].float(), ref, rtol=RTOL, atol=ATOL)
        checked += rows.numel()
    assert checked == flat.numel()


def test_config5_deepseek_v3_shape(cuda):
    """T=4096, H=7168, I=2048, E=256, top-8 skewed routing (32768 rows, W 7.5 GB).
    Every row of every one of the 167 non-empty experts is checked."""
    g = torch.Generator().manual_seed(0)
    bias = 1.5 * torch.randn(256, generator=g)
    idx = torch.topk(torch.randn(4096, 256, generator=g) + bias, 8).indices.to(cuda)
    W, gc = _c5_weights(cuda)
    X = torch.randn(4096, 7168, generator=gc, device=cuda).bfloat16()
    Y = K.grouped_gemm(X, W, idx)
    torch.cuda.synchronize()
    flat = idx.flatten()
    assert int((torch.bincount(flat, minlength=256) > 0).sum()) == 167
    _check_every_expert(Y, X, W, flat, lambda rows: rows // 8)
    del W


def test_config5_uniform_routing(cuda):
    """The C5 shape under the reference benchmark's uniform routing
    (benchmarks/benchmark_grouped_gemm.py:104-109): 4096 * 8 / 256 = 128 rows
    per expert, expert_indices = arange(32768) % 256 over an X of 32768 rows
    (1-D ids, no gather), and its single-GPU expert-parallel shard
    (E_local = 32 experts, 4096 rows)."""
    W, gc = _c5_weights(cuda)
    R = 32768
    X = torch.randn(R, 7168, generator=gc, device=cuda).bfloat16()
    ids = torch.arange(R, device=cuda) % 256
    Y = K.grouped_gemm(X, W, ids)
    torch.cuda.synchronize()
    _check_every_expert(Y, X, W, ids, lambda rows: rows)
    # expert-parallel shard: the first 32 experts, 128 rows each
    Xs = X[:4096].contiguous()
    ids_s = torch.arange(4096, device=cuda) % 32
    Ws = W[:32]
    Ys = K.grouped_gemm(Xs, Ws, ids_s)
    torch.cuda.synchronize()
    _check_every_expert(Ys, Xs, Ws, ids_s, lambda rows: rows)
    del W


def test_reuse_routing_matches_full_call(cuda):
    """moe_grouped_gemm_routed on the routing tables of the previous call is
    bitwise the full call, for every tile configuration, with a different
    weight set on the same routing."""
    for T, topk, E, H, I in ((300, 2, 8, 256, 96), (4096, 2, 8, 1024, 256), (8192, 4, 64, 512, 512)):
        X, W = make(T, H, I, E, seed=T)
        W2 = (0.5 * W).contiguous()
        g = torch.Generator().manual_seed(T)
        ids = torch.randint(0, E + 1, (T, topk), generator=g).to(cuda)  # includes invalid ids
        Y = K.grouped_gemm(X, W, ids)
        Yr = K.grouped_gemm_reuse_routing(X, W, topk)
        assert torch.equal(Y, Yr)
        Y2 = K.grouped_gemm(X, W2, ids)
        assert torch.equal(K.grouped_gemm_reuse_routing(X, W2, topk), Y2)


# Routings of up to 8192 rows over at most 14 experts, with 16-byte aligned
# ids, take the self-routing launch (8 rows per thread up to 2048 rows, 32
# above), in which every workgroup derives its tile's rows from the ids; a
# view of the same ids 8 or 4 bytes off that alignment takes the routing
# sort and the GEMM.  Both must agree bitwise, and the tables the
# self-routing launch writes must serve a reusing call.  (8193 rows and 15
# experts are just outside.)
@pytest.mark.parametrize("R,E,idt,dtype", [(8192, 8, torch.int64, torch.bfloat16),
                                           (8192, 14, torch.int32, torch.float16),
                                           (8191, 14, torch.int64, torch.bfloat16),
                                           (8193, 8, torch.int64, torch.bfloat16),
                                           (4000, 3, torch.int32, torch.bfloat16),
                                           (2049, 1, torch.int64, torch.float16),
                                           (2048, 8, torch.int64, torch.bfloat16),
                                           (1000, 14, torch.int32, torch.float16),
                                           (100, 5, torch.int64, torch.bfloat16),
                                           (3001, 15, torch.int32, torch.bfloat16)])
def test_self_routing_matches_sorted_path(cuda, R, E, idt, dtype):
    X, W = make(R, 192, 160, E, seed=R + E, dtype=dtype)
    g = torch.Generator().manual_seed(R * 31 + E)
    ids = torch.randint(-1, E + 2, (R,), generator=g).to(idt)  # about 3 in E + 3 ids invalid
    ids[: R // 3] = E // 2                                        # one crowded expert
    buf = torch.empty(R + 1, dtype=idt, device=cuda)
    buf[1:] = ids.to(cuda)
    off = buf[1:]                       # not 16-byte aligned: routing sort + GEMM
    al = ids.to(cuda)                   # aligned: self-routing when R <= 8192 and E <= 14
    assert al.data_ptr() % 16 == 0 and off.data_ptr() % 16 != 0
    Ya = check_gemm(X, W, al)
    assert torch.equal(K.grouped_gemm_reuse_routing(X, W, 1), Ya)
    Yo = K.grouped_gemm(X, W, off)
    assert torch.equal(Yo, Ya)
    bad = ((al < 0) | (al >= E))
    assert (Ya[bad] == 0).all()
    assert (K.grouped_gemm(X, W, torch.full_like(al, E)) == 0).all()  # every row invalid


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_mixed_tile_heights(cuda, dtype):
    """Problems that take the tallest tiles mix them with short tiles: an
    expert of at most 128 rows gets one short tile (three-stage pipeline),
    larger ones tiles of 256 rows.  Skewed routing with experts of every
    size class, including exactly 128 and 129 rows, and invalid ids."""
    T, topk, E, H, I = 4096, 8, 96, 256, 1024
    g = torch.Generator().manual_seed(31)
    bias = 1.5 * torch.randn(E, generator=g)
    ids = torch.topk(torch.randn(T, E, generator=g) + bias, topk).indices
    flat = ids.flatten()
    flat[::211] = E + 7  # invalid
    # Force two experts to exactly 128 and 129 rows by re-routing rows of the largest expert.
    big = int(torch.bincount(flat[flat < E], minlength=E).argmax())
    for e, want in ((E - 1, 128), (E - 2, 129)):
        have = int((flat == e).sum())
        if have < want:
            src = torch.nonzero(flat == big).squeeze(1)[: want - have]
            flat[src] = e
        else:
            flat[torch.nonzero(flat == e).squeeze(1)[: have - want]] = big
    ids = flat.view(T, topk)
    counts = torch.bincount(flat[flat < E], minlength=E)
    assert int(counts[E - 1]) == 128 and int(counts[E - 2]) == 129
    assert (counts > 256).any() and ((counts > 0) & (counts <= 128)).any()
    X, W = make(T, H, I, E, seed=31, dtype=dtype)
    check_gemm(X, W, ids.to(cuda), topk)


# A few routed rows (decode: at most 64 rows, H >= 512) take the K-split
# launch: each tile's K range is split over several workgroups whose fp32
# partials the last one sums in a fixed order (rows <= 8, <= 16, <= 32 and
# <= 64 publish partials of different sizes).  The full call groups the rows
# itself (no sort launch) and writes the sort's tables, which the reusing
# call's table-driven split then reads.  Against the fp32 reference,
# bitwise reproducible from call to call, with invalid ids, fp16, [T, topk]
# ids, and the split's tables reused by a routed call.
@pytest.mark.parametrize("T,topk,H,I,E,dtype", [(1, 2, 4096, 1792, 8, torch.bfloat16),
                                                (8, 2, 2048, 1000, 8, torch.float16),
                                                (32, 2, 1024, 256, 4, torch.bfloat16),
                                                (12, 2, 1024, 384, 6, torch.bfloat16),
                                                (3, 1, 520, 130, 3, torch.bfloat16),
                                                (64, 1, 4096, 512, 2, torch.bfloat16)])
def test_k_split_small_problems(cuda, T, topk, H, I, E, dtype):
    X, W = make(T, H, I, E, seed=T * 7 + H, dtype=dtype)
    g = torch.Generator().manual_seed(T + I)
    ids = torch.randint(0, E, (T, topk), generator=g)
    ids[0, 0] = E + 1  # one invalid id: a zero row
    ids = ids.to(cuda)
    if dtype == torch.float16:
        ids = ids.int()  # int32 ids
    Y = check_gemm(X, W, ids, topk)
    assert (Y.view(T * topk, I)[0] == 0).all()
    for _ in range(3):
        assert torch.equal(K.grouped_gemm(X, W, ids), Y)
    assert torch.equal(K.grouped_gemm_reuse_routing(X, W, topk), Y)
