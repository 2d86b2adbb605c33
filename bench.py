#!/usr/bin/env python3
"""Benchmark of the MoE routed-expert hot path on one MI355X.

Headline: fused TopK+softmax, radix branch,
fp32 logits [64, 32768], K = 2048.  A step is one topk_softmax call on
inputs already resident in HBM; ``value`` is algorithmic HBM bytes per call
(logits read + fp32 scores + int32 indices written = 9,437,184 B) divided
by the measured time per call, in GB/s.

The other BASELINE configurations are measured after the headline and
reported under "secondary" (router C1/C3a/C3b in us and GB/s, grouped GEMM
C4/C5 in TFLOP/s with %MFMA and %HBM, the fused router GEMM + TopK +
softmax on the reference's router-fusion models).  ``cpu_baseline`` is the reference's
CPU PyTorch path (torch.topk + softmax, kernels/topk_softmax_baseline.py:39-66)
timed on this host's cores on the same C2 input.

    python bench.py [--gpus 1] [--steps 200] [--warmup 20] [--only c2|c5|...]
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

import torch

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
BF16_PEAK_TFLOPS = 2500.0      # MI355X dense bf16 MFMA, TFLOP/s


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--only", default="", help="comma list of c1,c2,c3a,c3b,c4,dec,c5,c5u,ep,router,moe (profiling runs)")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    p.add_argument("--copy-calibration", action="store_true",
                   help="only run a 1 GiB device-to-device copy (scale for rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    p.add_argument("--traffic", default=os.path.join(os.path.dirname(os.path.abspath(__file__)),
                                                     "profiles", "traffic_radix_topk_c2.json"),
                   help="rocprofv3 --pmc summary giving measured HBM bytes per radix launch")
    return p.parse_args()


def gpu_time_ms(fn, steps: int, warmup: int) -> float:
    """Average ms per call of fn over `steps` calls, HIP events on the stream
    the kernels are launched on (torch's current stream)."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(steps):
        fn()
    end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def graph_time_ms(fn, calls: int = 20, replays: int = 20) -> float:
    """Average ms per call with `calls` calls captured in one HIP graph and the
    graph replayed `replays` times: device time without Python/launch overhead."""
    for _ in range(3):
        fn()
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(calls):
            fn()
    # Untimed replays first: the first replays of a fresh graph run slower
    # (C5: 1.52, 1.48, then 1.45 ms per call, the eager rate).
    for _ in range(3):
        g.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(replays):
        g.replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / (calls * replays)


_FLUSH = None


def cold_time_ms(fn, reps: int = 50) -> float:
    """Median ms of one call with the caches cold: before each call a 512 MB
    buffer is written, which evicts the L2s (4 MB per XCD) and the 256 MB
    MALL; HIP events bracket the call alone."""
    global _FLUSH
    if _FLUSH is None:
        _FLUSH = torch.empty(512 << 20, dtype=torch.uint8, device="cuda")
    fn()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    times = []
    for _ in range(reps):
        _FLUSH.zero_()
        start.record()
        fn()
        end.record()
        torch.cuda.synchronize()
        times.append(start.elapsed_time(end))
    times.sort()
    return times[len(times) // 2]


def cpu_time_ms(fn, budget_s: float = 2.0) -> float:
    fn()
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < budget_s or n < 2:
        fn()
        n += 1
    return (time.perf_counter() - t0) / n * 1e3


def router_bytes(M, N, K, in_bytes):
    return M * N * in_bytes + M * K * 4 + M * K * 4


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor()


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(the router shards rows and the GEMM shards experts with no exchange "
              "inside the measured kernels); run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    assert torch.cuda.is_available(), "bench.py needs a GPU"
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from tilelang_moe_amd import kernels as K

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.copy_calibration:
        # A plain copy of known size: 1 GiB read + 1 GiB written per dispatch.
        src = torch.empty(1 << 30, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes": 1 << 30}))
        return
    only = set(filter(None, args.only.split(",")))
    want = (lambda c: not only or c in only)
    secondary = {}

    # ---------------- headline: C2 radix router ----------------
    g = torch.Generator().manual_seed(0)
    x2_cpu = torch.randn(64, 32768, generator=g)
    x2 = x2_cpu.to(dev)
    b2 = router_bytes(64, 32768, 2048, 4)
    ms2 = None
    ms2_cold = None
    if want("c2"):
        ms2 = gpu_time_ms(lambda: K.topk_softmax(x2, 2048), args.steps, args.warmup)
        ms2_cold = cold_time_ms(lambda: K.topk_softmax(x2, 2048))

    # ---------------- secondary router configs ----------------
    router_cfgs = {
        "c1": ("topk_softmax fp32 [320,128] K=6 (selection)", 320, 128, 6, False),
        "c3a": ("topk_softmax bf16 [4096,64] K=6 (bitonic)", 4096, 64, 6, True),
        "c3b": ("topk_softmax bf16 [4096,256] K=8 (selection)", 4096, 256, 8, True),
    }
    for name, (desc, M, N, Kk, bf16) in router_cfgs.items():
        if not want(name):
            continue
        xc = torch.randn(M, N, generator=torch.Generator().manual_seed(0))
        xc = xc.bfloat16() if bf16 else xc
        x = xc.to(dev)
        ms = gpu_time_ms(lambda: K.topk_softmax(x, Kk), args.steps, args.warmup)
        msg = graph_time_ms(lambda: K.topk_softmax(x, Kk))
        nb = router_bytes(M, N, Kk, 2 if bf16 else 4)
        entry = {"workload": desc, "algo": K.select_strategy(N, Kk), "us_eager": ms * 1e3,
                 "us": msg * 1e3, "GB_s": nb / msg / 1e6, "frac_hbm": nb / msg / 1e6 / HBM_PEAK_GBS,
                 "us_cold": cold_time_ms(lambda: K.topk_softmax(x, Kk)) * 1e3,
                 "timing": "us: HIP-graph replay (device time); us_eager: Python call loop; "
                           "us_cold: one call after an L2/MALL flush, median of 50"}
        if not args.no_cpu:
            from oracle import torch_baseline as tb
            entry["cpu_us"] = cpu_time_ms(lambda: tb.topk_softmax_fused(xc, Kk)) * 1e3
        secondary[name] = entry

    # ---------------- grouped GEMM configs ----------------
    # ms: the whole drop-in call (device routing sort + GEMM) by graph replay;
    # ms_gemm: the GEMM alone on the routing the call before computed
    # (grouped_gemm_reuse_routing), as the reference benchmark times its
    # kernels with the routing done outside the timed region
    # (benchmarks/benchmark_grouped_gemm.py:116-214).
    def gemm_entry(desc, X, W, idx, topk, cpu_calls=0, cold=False):
        T, H = X.shape
        E, I, _ = W.shape
        R = T * topk
        calls, replays = (5, 4) if R * H * I > 1e11 else (20, 20)
        # The large GEMMs run 15-20% slower for their first ~20 calls in a
        # process (measured per kernel with rocprofv3); the timed calls start
        # after that.
        for _ in range(24 if R * H * I > 1e11 else 3):
            K.grouped_gemm(X, W, idx)
        torch.cuda.synchronize()
        ms_eager = gpu_time_ms(lambda: K.grouped_gemm(X, W, idx), max(5, min(args.steps, 50)),
                               min(args.warmup, 5))
        ms = graph_time_ms(lambda: K.grouped_gemm(X, W, idx), calls=calls, replays=replays)
        K.grouped_gemm(X, W, idx)  # the routing tables the GEMM-only calls reuse
        ms_gemm = gpu_time_ms(lambda: K.grouped_gemm_reuse_routing(X, W, topk), max(5, min(args.steps, 50)),
                              min(args.warmup, 5))
        flops = 2.0 * R * H * I
        cnt = torch.bincount(idx.flatten(), minlength=E)
        e_nz = int((cnt > 0).sum())
        nbytes = e_nz * I * H * 2 + T * H * 2 + R * I * 2 + R * 4
        tf = flops / ms / 1e9
        entry = {"workload": desc, "ms": ms, "ms_eager": ms_eager, "ms_gemm": ms_gemm, "TFLOP_s": tf,
                 "frac_mfma": tf / BF16_PEAK_TFLOPS, "TFLOP_s_gemm": flops / ms_gemm / 1e9,
                 "GB_s": nbytes / ms / 1e6, "frac_hbm": nbytes / ms / 1e6 / HBM_PEAK_GBS,
                 "rows": R, "experts_nonempty": e_nz, "rows_max_expert": int(cnt.max()),
                 "timing": "ms: HIP-graph replay of the whole call (routing sort + GEMM); ms_gemm: GEMM alone "
                           "on reused routing tables, HIP events around back-to-back calls"}
        if cold:
            entry["ms_cold"] = cold_time_ms(lambda: K.grouped_gemm(X, W, idx))
            entry["timing"] += "; ms_cold: one call after an L2/MALL flush, median of 50"
        if cpu_calls and not args.no_cpu:
            from oracle import torch_baseline as tb
            Xc, Wc, ic = X.cpu(), W.cpu(), idx.cpu()
            Xr = Xc.repeat_interleave(topk, 0) if topk > 1 else Xc
            t_cpu = []
            for _ in range(cpu_calls):
                t0 = time.perf_counter()
                tb.grouped_gemm_loop(Xr, Wc, ic.flatten())
                t_cpu.append((time.perf_counter() - t0) * 1e3)
            t_cpu.sort()
            entry["cpu_ms"] = t_cpu[len(t_cpu) // 2]
            entry["cpu_calls"] = cpu_calls
            entry["cpu_threads"] = torch.get_num_threads()
            del Xc, Wc, Xr
        return entry

    def gemm_weights(E, I, H):
        gc = torch.Generator(device=dev).manual_seed(0)
        W = torch.empty(E, I, H, dtype=torch.bfloat16, device=dev)
        for e0 in range(0, E, 32):
            e1 = min(E, e0 + 32)
            W[e0:e1] = (0.02 * torch.randn(e1 - e0, I, H, generator=gc, device=dev)).bfloat16()
        return W, gc

    if want("c4"):
        gg = torch.Generator().manual_seed(0)
        idx = torch.topk(torch.randn(4096, 8, generator=gg), 2).indices.to(dev)
        W, gc = gemm_weights(8, 256, 1024)
        X = torch.randn(4096, 1024, generator=gc, device=dev).bfloat16()
        secondary["c4"] = gemm_entry("grouped_gemm bf16 T=4096 H=1024 I=256 E=8 top-2 (8192 rows)", X, W, idx, 2,
                                     cpu_calls=5, cold=True)
        del W, X
    if want("dec"):
        # Decode: one and eight tokens, top-2 of 8 experts (the K-split path).
        W, gc = gemm_weights(8, 1792, 4096)
        for T in (1, 8):
            idx = torch.topk(torch.randn(T, 8, generator=torch.Generator().manual_seed(T)), 2).indices.to(dev)
            X = torch.randn(T, 4096, generator=gc, device=dev).bfloat16()
            secondary[f"decode_t{T}"] = gemm_entry(
                f"grouped_gemm bf16 decode T={T} H=4096 I=1792 E=8 top-2 ({2 * T} rows, K split)", X, W, idx, 2)
        del W, X
    if want("c5") or want("c5u") or want("ep"):
        W, gc = gemm_weights(256, 2048, 7168)
        if want("c5"):
            gg = torch.Generator().manual_seed(0)
            bias = 1.5 * torch.randn(256, generator=gg)
            idx = torch.topk(torch.randn(4096, 256, generator=gg) + bias, 8).indices.to(dev)
            X = torch.randn(4096, 7168, generator=gc, device=dev).bfloat16()
            secondary["c5"] = gemm_entry("grouped_gemm bf16 T=4096 H=7168 I=2048 E=256 top-8 skewed (32768 rows)",
                                         X, W, idx, 8, cpu_calls=1)
        # The reference benchmark's routing (benchmarks/benchmark_grouped_gemm.py:104-109):
        # 4096 tokens * top-8 / 256 experts = 128 rows per expert, ids = arange % E_local
        # over an X of that many rows; E_local = 256 (all experts) and the single-GPU
        # expert-parallel shard E_local = 32.
        if want("c5u"):
            X = torch.randn(32768, 7168, device=dev).bfloat16()
            ids = torch.arange(32768, device=dev) % 256
            secondary["c5_uniform"] = gemm_entry(
                "grouped_gemm bf16 R=32768 H=7168 I=2048 E=256 uniform (arange % 256, 128 rows per expert)",
                X, W, ids, 1)
            # The vendor library on the same weights and FLOPs, for scale: hipBLASLt's
            # batched GEMM on the uniform case laid out per expert (no gather, no
            # routing), and one dense GEMM of 32768 rows against a single expert.
            Xb = X.view(256, 128, 7168)
            ms_bmm = gpu_time_ms(lambda: torch.bmm(Xb, W.transpose(1, 2)), 10, 3)
            ms_dense = gpu_time_ms(lambda: X @ W[0].T, 20, 5)
            fl = 2.0 * 32768 * 7168 * 2048
            secondary["c5_library"] = {
                "workload": "torch (hipBLASLt) bf16 at the C5 FLOPs: bmm [256,128,7168]x[256,7168,2048]; "
                            "dense [32768,7168]x[7168,2048]",
                "ms_bmm_uniform": ms_bmm, "TFLOP_s_bmm_uniform": fl / ms_bmm / 1e9,
                "ms_dense_one_expert": ms_dense, "TFLOP_s_dense_one_expert": fl / ms_dense / 1e9,
                "timing": "HIP events around back-to-back calls"}
            del Xb
        if want("ep"):
            X = torch.randn(4096, 7168, device=dev).bfloat16()
            ids = torch.arange(4096, device=dev) % 32
            secondary["ep_shard"] = gemm_entry(
                "grouped_gemm bf16 expert-parallel shard: E_local=32 of 256, R=4096 (128 per expert), H=7168 I=2048",
                X, W[:32], ids, 1)
        del W

    # ---------------- fused router GEMM + TopK + softmax ----------------
    # The reference's router-fusion benchmark models (benchmarks/benchmark_router_fusion.py:169-174)
    # at 256 and 16384 tokens: fused kernel vs the two-launch path (router_gemm + topk_softmax)
    # and torch (bf16 matmul + topk + softmax) on the same GPU.
    fused_cfgs = {"r_qwen2_t256": ("Qwen2-57B", 256, 3584, 64, 8),
                  "r_qwen3_t256": ("Qwen3-235B", 256, 4096, 128, 8),
                  "r_dsv2_t256": ("DeepSeek-V2", 256, 5120, 160, 6),
                  "r_dsv2_t16384": ("DeepSeek-V2", 16384, 5120, 160, 6)}
    for name, (model, T, H, E, Kk) in fused_cfgs.items():
        if not want(name) and not want("router"):
            continue
        gr = torch.Generator(device=dev).manual_seed(0)
        X = torch.randn(T, H, generator=gr, device=dev).bfloat16()
        W = torch.randn(H, E, generator=gr, device=dev).bfloat16()
        # The drop-in call re-derives the kernels' weight layout on every
        # replay of a captured graph (the weight may change between replays);
        # the prepared call takes that layout, made once, as a serving engine
        # would at load time.
        Wt = K.prepare_router_weight(W)
        us = graph_time_ms(lambda: K.router_topk_softmax(X, W, Kk)) * 1e3
        us_prep = graph_time_ms(lambda: K.router_topk_softmax_prepared(X, Wt, Kk)) * 1e3
        us_two = graph_time_ms(lambda: K.topk_softmax(K.router_gemm(X, W), Kk)) * 1e3

        def torch_router():
            v, i = torch.topk(X @ W, Kk, dim=-1)
            return torch.softmax(v.float(), dim=-1), i

        us_torch = gpu_time_ms(torch_router, 50, 5) * 1e3
        nb = T * H * 2 + H * E * 2 + T * Kk * 8
        fl = 2.0 * T * H * E
        secondary[name] = {"workload": f"fused router {model} T={T} H={H} E={E} K={Kk} bf16", "us": us,
                           "us_prepared": us_prep, "us_two_launch": us_two, "us_torch": us_torch,
                           "GB_s": nb / us_prep / 1e3, "frac_hbm": nb / us_prep / 1e3 / HBM_PEAK_GBS,
                           "TFLOP_s": fl / us_prep / 1e6,
                           "timing": "HIP-graph replay: us = router_topk_softmax(X, W) incl. the per-replay "
                                     "weight transpose, us_prepared = router_topk_softmax_prepared(X, Wt) "
                                     "(GB_s, TFLOP_s from it), us_two_launch = router_gemm + topk_softmax "
                                     "incl. the transpose; us_torch: eager torch on the GPU"}
        del X, W, Wt

    # ---------------- FusedMoE (routed + shared experts) ----------------
    # The reference's FusedMoE benchmark configs (benchmarks/benchmark_fusedmoe.py:29-50),
    # inputs as its generate_fusedmoe_inputs (randn / sqrt(fan_in)), bf16.
    moe_cfgs = {"moe_small": ("Small-Test", 1024, 2048, 512, 8, 1, 2),
                "moe_dsv3": ("DeepSeek-V3", 8192, 7168, 2048, 8, 1, 4)}
    for name, (model, T, Dh, De, E, NS, Kk) in moe_cfgs.items():
        if not want(name) and not want("moe"):
            continue
        gm = torch.Generator(device=dev).manual_seed(42)
        rn = lambda *shape: (torch.randn(*shape, generator=gm, device=dev) / shape[-1] ** 0.5).bfloat16()  # noqa: E731
        Ds = De * NS
        x = torch.randn(T, Dh, generator=gm, device=dev).bfloat16()
        mw = dict(router_weight=rn(E, Dh), shared_gate=rn(Ds, Dh), shared_up=rn(Ds, Dh), shared_down=rn(Dh, Ds),
                  routed_gate=rn(E, De, Dh), routed_up=rn(E, De, Dh), routed_down=rn(E, Dh, De))
        ms = graph_time_ms(lambda: K.fused_moe_routed(x, **mw, n_experts_per_token=Kk), calls=3, replays=5)
        from oracle import torch_baseline as tb
        ms_torch = gpu_time_ms(lambda: tb.fusedmoe_torch(x, *mw.values(), Kk), 5, 2)
        flops = 2.0 * 3 * (T * Kk * Dh * De + T * Dh * Ds) + 2.0 * T * Dh * E
        tf = flops / ms / 1e9
        secondary[name] = {"workload": f"FusedMoE {model} T={T} H={Dh} I={De} E={E} shared={NS} top-{Kk} bf16",
                           "ms": ms, "ms_torch": ms_torch, "TFLOP_s": tf, "frac_mfma": tf / BF16_PEAK_TFLOPS,
                           "timing": "ms: HIP-graph replay of the whole forward; ms_torch: eager torch "
                                     "fusedmoe_pytorch restatement on the GPU"}
        del x, mw

    # ---------------- CPU baseline (reference torch path) ----------------
    cpu = None
    if not args.no_cpu and ms2 is not None:
        from oracle import torch_baseline as tb
        threads = torch.get_num_threads()
        tb.topk_softmax_fused(x2_cpu, 2048)  # warm-up
        n, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < 10.0:
            tb.topk_softmax_fused(x2_cpu, 2048)
            n += 1
        cpu_ms = (time.perf_counter() - t0) / n * 1e3
        cpu = {"value": b2 / cpu_ms / 1e6, "unit": "GB/s", "cores": threads, "kind": "port",
               "sample": f"{n} calls of torch.topk+softmax on the C2 fp32 [64,32768] K=2048 input "
                         f"({cpu_ms:.3f} ms/call, {cpu_model()}, torch {torch.__version__})"}

    if ms2 is None:
        print(json.dumps({"secondary": secondary}))
        return

    achieved = b2 / ms2 / 1e6
    traffic = None
    if os.path.exists(args.traffic):
        try:
            traffic = json.load(open(args.traffic)).get("hbm_bytes_per_launch")
        except (OSError, ValueError):
            traffic = None
    out = {
        "metric": "router us + HBM GB/s; grouped-GEMM TFLOP/s (% bf16 MFMA peak), 1 MI355X",
        "value": achieved,
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms2,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded N(0,1) logits)",
        "config": {"workload": "topk_softmax radix, fp32 logits [64,32768], K=2048 (BASELINE configs[1])",
                   "M": 64, "N": 32768, "K": 2048, "us_per_call": ms2 * 1e3,
                   "us_per_call_cold": ms2_cold * 1e3,
                   "timing": "value, ms_per_step: HIP events around `steps` back-to-back calls on the "
                             "launching stream; us_per_call_cold: one call after writing 512 MB "
                             "(evicts L2 and MALL), median of 50"},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": traffic},
        "cpu_baseline": cpu,
        "secondary": secondary,
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
