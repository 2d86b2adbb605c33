"""Every entry point on a non-default stream and inside a replayed HIP graph.

The library is stream-ordered: it launches on torch's current stream, and
the Python layer keeps one zero-initialised workspace per (device, stream)
whose control block each call leaves zero (the split-row radix counters
live there).  Every kernel here is deterministic (fixed-order reductions,
an exact fixed-point softmax normaliser in the radix path), so results on a
side stream and from graph replays must equal the eager default-stream
results bit for bit.  The graph is replayed three times, with new inputs
copied into its static tensors and eager calls of the same operators
between replays, and every replay is checked against eager.
"""
import math

import pytest
import torch

from tilelang_moe_amd import kernels as K

pytestmark = pytest.mark.gpu


def _inputs(seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    d = {}
    d["radix"] = torch.randn(8, 32768, generator=g, device="cuda")               # one workgroup per row
    d["split"] = torch.randn(4, 65536, generator=g, device="cuda")               # split rows (workspace counters)
    d["small"] = torch.randn(256, 64, generator=g, device="cuda").bfloat16()      # bitonic
    d["sel"] = torch.randn(256, 256, generator=g, device="cuda").bfloat16()       # selection
    d["X"] = torch.randn(512, 1024, generator=g, device="cuda").bfloat16()
    d["W"] = (0.02 * torch.randn(8, 256, 1024, generator=g, device="cuda")).bfloat16()
    d["ids"] = torch.randint(0, 8, (512, 2), generator=g, device="cuda")       # 1024 rows: self-routing, 8 per thread
    d["ids8"] = torch.randint(0, 8, (512, 8), generator=g, device="cuda")      # 4096 rows: self-routing, 32 per thread
    d["Xr"] = torch.randn(256, 2048, generator=g, device="cuda").bfloat16()
    d["Wr"] = (torch.randn(2048, 64, generator=g, device="cuda") / math.sqrt(2048)).bfloat16()
    # A weight in the kernels' layout, made once (fixed across replays, as at load time).
    g_fixed = torch.Generator(device="cuda").manual_seed(99)
    W_fixed = (torch.randn(2048, 96, generator=g_fixed, device="cuda") / math.sqrt(2048)).bfloat16()
    d["Wt"] = K.prepare_router_weight(W_fixed)
    T, Dh, De, E = 128, 256, 128, 8
    d["x"] = torch.randn(T, Dh, generator=g, device="cuda").bfloat16()
    s = 1 / math.sqrt(Dh)
    d["moe"] = dict(router_weight=(s * torch.randn(E, Dh, generator=g, device="cuda")).bfloat16(),
                    shared_gate=(s * torch.randn(De, Dh, generator=g, device="cuda")).bfloat16(),
                    shared_up=(s * torch.randn(De, Dh, generator=g, device="cuda")).bfloat16(),
                    shared_down=(torch.randn(Dh, De, generator=g, device="cuda") / math.sqrt(De)).bfloat16(),
                    routed_gate=(s * torch.randn(E, De, Dh, generator=g, device="cuda")).bfloat16(),
                    routed_up=(s * torch.randn(E, De, Dh, generator=g, device="cuda")).bfloat16(),
                    routed_down=(torch.randn(E, Dh, De, generator=g, device="cuda") / math.sqrt(De)).bfloat16())
    return d


def _run_all(d):
    out = []
    out += K.topk_softmax(d["radix"], 2048)
    out += K.topk_softmax(d["split"], 512)
    out += K.topk_softmax(d["small"], 6)
    out += K.topk_softmax(d["sel"], 8)
    out.append(K.grouped_gemm(d["X"], d["W"], d["ids"]))
    out.append(K.grouped_gemm(d["X"], d["W"], d["ids8"]))
    out.append(K.grouped_gemm(d["X"][:4], d["W"], d["ids"][:4]))  # 8 rows: the K split (partials, counters)
    out += K.router_topk_softmax(d["Xr"], d["Wr"], 8)
    out += K.router_topk_softmax_prepared(d["Xr"], d["Wt"], 6)
    out.append(K.fused_moe_routed(d["x"], **d["moe"], n_experts_per_token=2))
    return out


def _assert_equal(got, want, what):
    assert len(got) == len(want)
    for i, (a, b) in enumerate(zip(got, want)):
        assert torch.equal(a, b), f"{what}: output {i} differs"


def test_side_stream_matches_default_stream(cuda):
    d = _inputs(1)
    want = _run_all(d)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        got = _run_all(d)
        got2 = _run_all(d)  # second call on the stream: its workspace counters were left zero
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    _assert_equal(got, want, "side stream")
    _assert_equal(got2, want, "side stream, second call")


def test_graph_replays_match_eager(cuda):
    d = _inputs(2)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        _run_all(d)  # warm up on the capture stream: its workspace exists before capture
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        static_out = _run_all(d)
    torch.cuda.synchronize()
    for rep in range(3):
        fresh = _inputs(10 + rep)
        for key, t in fresh.items():
            if key == "Wt":
                continue  # prepared once, never updated
            if key == "moe":
                for n, w in t.items():
                    d["moe"][n].copy_(w)
            else:
                d[key].copy_(t)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        want = _run_all(d)  # eager work between replays
        torch.cuda.synchronize()
        _assert_equal(static_out, want, f"replay {rep}")


def test_capture_as_first_call_on_a_fresh_stream(cuda):
    """A graph captured with no warm-up on its capture stream (torch's own
    capture stream, as in torch.cuda.graph(g) after a warm-up elsewhere):
    the call that needs a workspace makes it inside the capture (graph-pool
    memory, zero fill recorded in the graph), and every replay matches eager,
    with eager calls of the same shape between replays."""
    g = torch.Generator(device="cuda").manual_seed(5)
    split = torch.randn(4, 65536, generator=g, device="cuda")   # split rows: needs a workspace
    small = torch.randn(256, 64, generator=g, device="cuda").bfloat16()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static_out = list(K.topk_softmax(split, 512)) + list(K.topk_softmax(small, 6))
        static_out += list(K.topk_softmax(split, 512))  # a second captured call on the same buffer
    for rep in range(3):
        split.copy_(torch.randn(4, 65536, generator=g, device="cuda"))
        small.copy_(torch.randn(256, 64, generator=g, device="cuda").bfloat16())
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        want = list(K.topk_softmax(split, 512)) + list(K.topk_softmax(small, 6)) + list(K.topk_softmax(split, 512))
        torch.cuda.synchronize()
        _assert_equal(static_out, want, f"first-call capture, replay {rep}")


def test_graph_replay_after_workspace_growth(cuda):
    """A graph captured on stream s keeps using the workspace it captured
    after a larger eager call on s replaced that stream's workspace: the
    replaced buffer stays alive, so replays neither read freed memory nor
    race with tensors allocated since."""
    g = torch.Generator(device="cuda").manual_seed(6)
    x = torch.randn(4, 65536, generator=g, device="cuda")
    big = torch.randn(200, 65536, generator=g, device="cuda")
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        K.topk_softmax(x, 512)  # warm-up: the stream's workspace fits this call
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        static_out = K.topk_softmax(x, 512)
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        want_big = K.topk_softmax(big, 512)  # grows the stream's workspace
    torch.cuda.synchronize()
    junk = [torch.full((1 << 20,), 0x7F, dtype=torch.uint8, device="cuda") for _ in range(16)]
    for rep in range(3):
        x.copy_(torch.randn(4, 65536, generator=g, device="cuda"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        _assert_equal(static_out, K.topk_softmax(x, 512), f"replay {rep} after growth")
    with torch.cuda.stream(s):
        again = K.topk_softmax(big, 512)
    torch.cuda.synchronize()
    _assert_equal(again, want_big, "eager call on the grown workspace")
    del junk
