"""moe_grouped_gemm_noalloc (its workspace in a static device array)
against moe_grouped_gemm (a caller workspace), both through the C ABI.

The two run the same kernels on the same routing, so their outputs must be
bit-identical.  Two calls in a row, the second smaller, check that what the
first call leaves in the shared array does not leak into the second."""
import pytest
import torch

from tilelang_moe_amd import _lib

pytestmark = pytest.mark.gpu

DT = {torch.bfloat16: _lib.MOE_BF16, torch.float16: _lib.MOE_F16}
IT = {torch.int32: _lib.MOE_I32, torch.int64: _lib.MOE_I64}


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _with_workspace(X, W, ids, topk):
    L = _lib.lib()
    T = X.shape[0]
    E, I, H = W.shape
    nbytes = L.moe_grouped_gemm_workspace_size(T, topk, E, I)
    ws = torch.zeros(nbytes, dtype=torch.uint8, device=X.device)
    Y = torch.full((T * topk, I), float("nan"), dtype=X.dtype, device=X.device)
    rc = L.moe_grouped_gemm(X.data_ptr(), W.data_ptr(), ids.data_ptr(), DT[X.dtype], IT[ids.dtype], T, topk, H,
                            I, E, Y.data_ptr(), ws.data_ptr(), nbytes, _stream())
    _lib.check(rc)
    return Y


def _noalloc(X, W, ids, topk):
    L = _lib.lib()
    T = X.shape[0]
    E, I, H = W.shape
    Y = torch.full((T * topk, I), float("nan"), dtype=X.dtype, device=X.device)
    rc = L.moe_grouped_gemm_noalloc(X.data_ptr(), W.data_ptr(), ids.data_ptr(), DT[X.dtype], IT[ids.dtype], T, topk,
                                    H, I, E, Y.data_ptr(), _stream())
    _lib.check(rc)
    return Y


def _case(T, topk, H, I, E, dtype, idt, seed, bad=0):
    g = torch.Generator(device="cuda").manual_seed(seed)
    X = torch.randn(T, H, device="cuda", generator=g).to(dtype)
    W = (0.05 * torch.randn(E, I, H, device="cuda", generator=g)).to(dtype)
    ids = torch.randint(0, E, (T, topk), device="cuda", generator=g)
    if bad:
        ids.view(-1)[:bad] = -1  # out-of-range ids give zero rows
        ids.view(-1)[bad:2 * bad] = E
    return X, W, ids.to(idt)


@pytest.mark.parametrize("order", ["noalloc_first", "workspace_first"])
def test_noalloc_matches_workspace_entry_point(order):
    # First call: 16384 routed rows over 64 experts (256x256 tiles, the
    # dynamic schedule and its counters); second: 600 rows over 8 experts;
    # third: 8 rows (the K split, its partials and per-tile counters).
    cases = [_case(2048, 8, 1024, 1024, 64, torch.bfloat16, torch.int64, 1, bad=37),
             _case(300, 2, 512, 384, 8, torch.float16, torch.int32, 2, bad=5),
             _case(4, 2, 2048, 512, 8, torch.bfloat16, torch.int64, 4, bad=2)]
    for X, W, ids, in cases:
        topk = ids.shape[1]
        if order == "noalloc_first":
            Yn = _noalloc(X, W, ids, topk)
            Yw = _with_workspace(X, W, ids, topk)
        else:
            Yw = _with_workspace(X, W, ids, topk)
            Yn = _noalloc(X, W, ids, topk)
        torch.cuda.synchronize()
        assert not torch.isnan(Yn.float()).any()
        assert torch.equal(Yn, Yw)
        assert (Yn[:4].float() == 0).all()  # rows with ids outside [0, E)


def test_noalloc_repeated_calls_and_graph_capture():
    X, W, ids = _case(512, 4, 256, 256, 16, torch.bfloat16, torch.int32, 3)
    ref = _with_workspace(X, W, ids, 4)
    for _ in range(3):
        assert torch.equal(_noalloc(X, W, ids, 4), ref)
    # Captured into a HIP graph: no allocation happens inside the call.
    s = torch.cuda.Stream()
    Y = torch.empty_like(ref)
    L = _lib.lib()
    with torch.cuda.stream(s):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            rc = L.moe_grouped_gemm_noalloc(X.data_ptr(), W.data_ptr(), ids.data_ptr(), _lib.MOE_BF16,
                                            _lib.MOE_I32, 512, 4, 256, 256, 16, Y.data_ptr(), s.cuda_stream)
    _lib.check(rc)
    for _ in range(3):
        Y.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(Y, ref)
        assert torch.equal(_noalloc(X, W, ids, 4), ref)  # eager calls between replays


def test_noalloc_largest_accepted_and_first_rejected_size():
    L = _lib.lib()
    E, I, H, topk = 256, 64, 64, 8
    # Smallest T whose workspace exceeds the fixed scratch.
    lo, hi = 1, 1 << 20
    while lo < hi:
        mid = (lo + hi) // 2
        if L.moe_grouped_gemm_workspace_size(mid, topk, E, I) > _lib.MOE_NOALLOC_SCRATCH_BYTES:
            hi = mid
        else:
            lo = mid + 1
    # Buffers for T = lo, so even a wrongly accepted call stays in bounds.
    X, W, ids = _case(lo, topk, H, I, E, torch.bfloat16, torch.int32, 4)
    Y = torch.empty(lo * topk, I, dtype=X.dtype, device=X.device)
    rc = L.moe_grouped_gemm_noalloc(X.data_ptr(), W.data_ptr(), ids.data_ptr(), _lib.MOE_BF16, _lib.MOE_I32, lo,
                                    topk, H, I, E, Y.data_ptr(), _stream())
    assert rc == _lib.MOE_EUNSUP
    assert b"scratch" in L.moe_last_error()
    # T = lo - 1 fits (about a million routed rows) and matches the workspace entry point.
    Xs, ids_s = X[:lo - 1], ids[:lo - 1]
    assert torch.equal(_noalloc(Xs, W, ids_s, topk), _with_workspace(Xs, W, ids_s, topk))
