"""GPU parity of the routed-expert FFN pieces and of the whole FusedMoE.

Bars (floating point; the north-star GEMM tolerance rtol = atol = 1e-2):
  * grouped_gemm_swiglu vs a torch fp32 reference silu(X Wg^T) * (X Wu^T),
    over the three tile configurations, ragged shapes, [T, topk] ids,
    invalid ids (zero rows) and fp16.
  * moe_combine vs torch fp32.
  * fusedmoe_best: the routing it returns is Convention A of the float64
    oracle (every chosen expert within the fp32 logit error of the top-k,
    weights the all-expert softmax at the chosen experts), and the output
    equals the float64 oracle evaluated under that routing within
    rtol = atol = 2e-2 (bf16 intermediates h, y, as the reference's
    TileLang kernels keep them) — checked on small shapes against the
    numpy oracle and on larger ones against a torch reference that rounds
    at the same points.
"""
import math

import numpy as np
import pytest
import torch

from oracle import fusedmoe as ofm
from tilelang_moe_amd import kernels as K

pytestmark = pytest.mark.gpu


def rnd(*shape, g, dtype=torch.bfloat16, scale=None):
    t = torch.randn(*shape, generator=g, device="cuda")
    return (t / math.sqrt(shape[-1]) if scale is None else t * scale).to(dtype)


def swiglu_ref(X, Wg, Wu, ids, topk=1):
    ids = ids.reshape(-1).long()
    E, I, _ = Wg.shape
    Y = torch.zeros(ids.numel(), I, dtype=torch.float32, device=X.device)
    for e in torch.unique(ids).tolist():
        if not 0 <= e < E:
            continue
        rows = torch.nonzero(ids == e).squeeze(1)
        xr = X[rows // topk].float()
        g, u = xr @ Wg[e].float().T, xr @ Wu[e].float().T
        Y[rows] = g * torch.sigmoid(g) * u
    return Y


# Tile configurations: 64x128 (small), 128x256 ((16384, 2, 256, 384, 8)), 256x256 (8192, 2, 1000, 1900, 16).
# (4, 2, 1024, 256, 8): 8 rows, the K-split path.
@pytest.mark.parametrize("T,topk,H,I,E", [(1, 1, 64, 32, 1), (4, 2, 1024, 256, 8), (300, 2, 520, 200, 5),
                                          (4096, 2, 1024, 256, 8), (2048, 8, 512, 384, 64), (16384, 2, 256, 384, 8),
                                          (8192, 2, 1000, 1900, 16)])
def test_grouped_gemm_swiglu(cuda, T, topk, H, I, E):
    g = torch.Generator(device="cuda").manual_seed(T + I)
    X = rnd(T, H, g=g, scale=1.0)
    Wg, Wu = rnd(E, I, H, g=g), rnd(E, I, H, g=g)
    ids = torch.randint(0, E, (T, topk), device="cuda", generator=g)
    ids[::13, 0] = E + 3  # invalid: zero rows
    Y = K.grouped_gemm_swiglu(X, Wg, Wu, ids if topk > 1 else ids[:, 0])
    torch.cuda.synchronize()
    ref = swiglu_ref(X, Wg, Wu, ids, topk)
    torch.testing.assert_close(Y.float(), ref, rtol=1e-2, atol=1e-2)
    assert (Y[(ids.flatten() >= E)] == 0).all()


def test_grouped_gemm_swiglu_fp16(cuda):
    g = torch.Generator(device="cuda").manual_seed(3)
    X = rnd(500, 256, g=g, dtype=torch.float16, scale=1.0)
    Wg, Wu = rnd(6, 128, 256, g=g, dtype=torch.float16), rnd(6, 128, 256, g=g, dtype=torch.float16)
    ids = torch.randint(0, 6, (500,), device="cuda", generator=g).int()
    torch.testing.assert_close(K.grouped_gemm_swiglu(X, Wg, Wu, ids).float(), swiglu_ref(X, Wg, Wu, ids),
                               rtol=1e-2, atol=1e-2)


@pytest.mark.parametrize("T,k,D,shared", [(1, 1, 8, False), (37, 3, 100, True), (512, 8, 7168, True)])
def test_combine(cuda, T, k, D, shared):
    g = torch.Generator(device="cuda").manual_seed(T + D)
    Yr = rnd(T * k, D, g=g, scale=1.0)
    w = torch.rand(T, k, generator=g, device="cuda")
    S = rnd(T, D, g=g, scale=1.0) if shared else None
    out = K.moe_combine(Yr, w, S)
    ref = (Yr.float().view(T, k, D) * w[:, :, None]).sum(1) + (S.float() if shared else 0)
    torch.testing.assert_close(out.float(), ref, rtol=1e-2, atol=1e-2)


def _moe_weights(T, Dh, De, Ds, E, seed, dtype=torch.bfloat16):
    g = torch.Generator(device="cuda").manual_seed(seed)
    x = rnd(T, Dh, g=g, dtype=dtype, scale=1.0)
    w = dict(router_weight=rnd(E, Dh, g=g, dtype=dtype),
             shared_gate=rnd(Ds, Dh, g=g, dtype=dtype) if Ds else None,
             shared_up=rnd(Ds, Dh, g=g, dtype=dtype) if Ds else None,
             shared_down=rnd(Dh, Ds, g=g, dtype=dtype) if Ds else None,
             routed_gate=rnd(E, De, Dh, g=g, dtype=dtype), routed_up=rnd(E, De, Dh, g=g, dtype=dtype),
             routed_down=rnd(E, Dh, De, g=g, dtype=dtype))
    return x, w


def check_routing(x, router_weight, k, wts, ids):
    lg = (x.double() @ router_weight.double().T).cpu().numpy()
    bound = (1e-5 * (x.double().abs() @ router_weight.double().abs().T) + 1e-6).cpu().numpy().max(1)
    ids_np = ids.long().cpu().numpy()
    chosen = np.take_along_axis(lg, ids_np, 1)
    kth = np.sort(lg, 1)[:, ::-1][:, k - 1]
    assert (chosen.min(1) >= kth - 2 * bound).all()
    e = np.exp(lg - lg.max(1, keepdims=True))
    p = np.take_along_axis(e / e.sum(1, keepdims=True), ids_np, 1)
    np.testing.assert_allclose(wts.double().cpu().numpy(), p, rtol=1e-4, atol=1e-7)


# Ds == De: the shared expert rides in the routed grouped GEMMs as expert E;
# Ds == 2 De (two shared experts): separate shared GEMMs.
# (4, 1024, 512, 0, 8, 2) and (3, 1024, 512, 512, 8, 2): decode-size, the
# K-split GEMMs when no rows are appended.
@pytest.mark.parametrize("T,Dh,De,Ds,E,k", [(64, 256, 128, 128, 8, 2), (200, 512, 256, 0, 16, 4),
                                            (33, 1024, 512, 512, 4, 4), (48, 256, 128, 256, 8, 2),
                                            (4, 1024, 512, 0, 8, 2), (3, 1024, 512, 512, 8, 2)])
def test_fusedmoe_vs_numpy_oracle(cuda, T, Dh, De, Ds, E, k):
    x, w = _moe_weights(T, Dh, De, Ds, E, seed=T + E)
    out, wts, ids = K.fused_moe_routed(x, **w, n_experts_per_token=k, return_routing=True)
    torch.cuda.synchronize()
    check_routing(x, w["router_weight"], k, wts, ids)
    cpu = {n: (t.float().cpu().numpy() if t is not None else None) for n, t in w.items()}
    ref = ofm.fusedmoe(x.float().cpu().numpy(), **cpu, k=k,
                       routing=(wts.cpu().numpy(), ids.long().cpu().numpy()))
    np.testing.assert_allclose(out.float().cpu().numpy(), ref, rtol=2e-2, atol=2e-2)


def torch_moe_ref(x, w, k, wts, ids):
    """fp32 torch restatement of fusedmoe_pytorch under the given routing,
    rounding h and the expert outputs to bf16 where the kernels do."""
    bf = lambda t: t.to(x.dtype).float()  # noqa: E731

    def ffn(xs, g, u, d):
        a, b = xs @ g.float().T, xs @ u.float().T
        return bf(bf(a * torch.sigmoid(a) * b) @ d.float().T)

    xf = x.float()
    out = ffn(xf, w["shared_gate"], w["shared_up"], w["shared_down"]) if w["shared_gate"] is not None \
        else torch.zeros_like(xf)
    for e in torch.unique(ids).tolist():
        rows, slot = torch.nonzero(ids == e, as_tuple=True)
        out[rows] += wts[rows, slot][:, None] * ffn(xf[rows], w["routed_gate"][e], w["routed_up"][e],
                                                    w["routed_down"][e])
    return out


# (4096, 4096, 256, 256, 8, 2): the up GEMM takes 64-row tiles and the down
# GEMM 256-row tiles, so the down GEMM rebuilds the tile table from the up
# GEMM's routing.  (1024, ..., 8, 2) (Small-Test) and (1500, ..., 1): at most
# 2048 routed rows but more than 2048 with the shared expert's appended rows,
# sorted by the one-workgroup routing sort with the appended rows placed
# directly.
@pytest.mark.parametrize("T,Dh,De,Ds,E,k", [(2048, 2048, 1024, 1024, 8, 4), (4096, 1024, 512, 0, 64, 6),
                                            (4096, 4096, 256, 256, 8, 2), (1024, 2048, 512, 512, 8, 2),
                                            (1500, 512, 256, 256, 8, 1)])
def test_fusedmoe_large(cuda, T, Dh, De, Ds, E, k):
    x, w = _moe_weights(T, Dh, De, Ds, E, seed=T)
    out, wts, ids = K.fused_moe_routed(x, **w, n_experts_per_token=k, return_routing=True)
    torch.cuda.synchronize()
    check_routing(x, w["router_weight"], k, wts, ids)
    torch.testing.assert_close(out.float(), torch_moe_ref(x, w, k, wts, ids.long()), rtol=2e-2, atol=2e-2)


def test_fusedmoe_mixed_tile_tables(cuda):
    """A routing skewed enough that the up GEMM takes the mixed 256/128-row
    tile table (tall and short tiles interleaved, with holes) while the
    down GEMM, narrower, takes another tile height and rebuilds the table
    from the same routing."""
    T, Dh, De, Ds, E, k = 4096, 512, 1024, 1024, 64, 8
    x, w = _moe_weights(T, Dh, De, Ds, E, seed=7)
    g = torch.Generator(device="cuda").manual_seed(8)
    x[:, 0] = 4.0  # a constant input column turns router_weight[:, 0] into a per-expert bias
    w["router_weight"][:, 0] = (torch.randn(E, generator=g, device="cuda") * 2.0).to(x.dtype)
    out, wts, ids = K.fused_moe_routed(x, **w, n_experts_per_token=k, return_routing=True)
    torch.cuda.synchronize()
    counts = torch.bincount(ids.flatten().long(), minlength=E)
    assert (counts > 256).any() and ((counts > 0) & (counts <= 128)).any()
    check_routing(x, w["router_weight"], k, wts, ids)
    torch.testing.assert_close(out.float(), torch_moe_ref(x, w, k, wts, ids.long()), rtol=2e-2, atol=2e-2)


@pytest.mark.parametrize("T", [40, 600])  # split-H and unsplit router GEMM
def test_fusedmoe_more_than_256_experts(cuda, T):
    """E > 256: the router runs as router GEMM + TopK (the fused router
    selection stops at 256 experts)."""
    E, k = 288, 8
    x, w = _moe_weights(T, 512, 128, 128, E, seed=E + T)
    out, wts, ids = K.fused_moe_routed(x, **w, n_experts_per_token=k, return_routing=True)
    torch.cuda.synchronize()
    assert int(ids.max()) < E and int(ids.min()) >= 0
    check_routing(x, w["router_weight"], k, wts, ids)
    torch.testing.assert_close(out.float(), torch_moe_ref(x, w, k, wts, ids.long()), rtol=2e-2, atol=2e-2)


def test_reference_signatures(cuda):
    B, S, Dh, De, E, k = 2, 64, 256, 128, 8, 2
    x, w = _moe_weights(B * S, Dh, De, De, E, seed=5)
    x3 = x.view(B, S, Dh)
    args = (x3, w["router_weight"], w["shared_gate"], w["shared_up"], w["shared_down"], w["routed_gate"],
            w["routed_up"], w["routed_down"])
    out = K.fusedmoe_best(*args, k)
    assert out.shape == (B, S, Dh)
    assert torch.equal(out, K.fusedmoe(*args, k)) and torch.equal(out, K.fusedmoe_tilelang_streams(*args, k))
    m = K.FusedMoETileLang(Dh, De, E, 1, k, B, S, dtype=torch.bfloat16)
    assert torch.equal(m.forward(*args), out)
    flat = K.fused_moe_routed(x, **w, n_experts_per_token=k)
    assert torch.equal(flat.view(B, S, Dh), out)


def test_grouped_gemm_swiglu_mixed_tile_heights(cuda):
    """SwiGLU epilogue on a problem that takes the tallest tiles, with
    skewed routing so that small experts get short tiles."""
    T, topk, E, H, I = 4096, 8, 64, 512, 512
    g = torch.Generator().manual_seed(41)
    bias = 1.5 * torch.randn(E, generator=g)
    ids = torch.topk(torch.randn(T, E, generator=g) + bias, topk).indices.to(cuda)
    counts = torch.bincount(ids.flatten(), minlength=E)
    assert (counts > 256).any() and ((counts > 0) & (counts <= 128)).any()
    gd = torch.Generator(device="cuda").manual_seed(41)
    X = rnd(T, H, g=gd, scale=1.0)
    Wg, Wu = rnd(E, I, H, g=gd), rnd(E, I, H, g=gd)
    Y = K.grouped_gemm_swiglu(X, Wg, Wu, ids)
    torch.cuda.synchronize()
    torch.testing.assert_close(Y.float(), swiglu_ref(X, Wg, Wu, ids, topk), rtol=1e-2, atol=1e-2)
