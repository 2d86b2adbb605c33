"""CPU oracle for the MoE hot path — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this package, and only as the checker (or the timed CPU baseline);
the product package tilelang_moe_amd never imports it.

  oracle.router          numpy restatement of topk_softmax_fused with a fixed tie rule
  oracle.gemm            numpy restatement of grouped_gemm_loop and the routing sort
  oracle.router_gemm     float64 router logits X @ W and their top-K softmax
  oracle.torch_baseline  the reference's CPU torch path, for the timed baseline

Parity status: every function is pinned by tests/test_oracle.py (brute
force, torch on tie-free rows, closed forms); none is "parity unpinned".
"""
