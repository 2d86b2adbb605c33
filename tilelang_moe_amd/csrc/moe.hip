// Routed-expert FFN (FusedMoE) for gfx950, built from this library's
// kernels.  Replaces FusedMoETileLang.forward / fusedmoe_best
// (kernels/fusedmoe_tilelang.py:309-425, :605-690) and restates the
// semantics of fusedmoe_pytorch (kernels/fusedmoe_baseline.py:41-168):
//
//   logits = x . router_w^T                    moe_router_gemm (fp32)
//   w, idx = top-k of softmax(logits)          moe_topk_softmax_ex, Convention A
//   h      = silu(x Wg[e]^T) * (x Wu[e]^T)     SwiGLU grouped GEMM, per routed row
//   y      = h Wd[e]^T                         grouped GEMM
//   hs, ys = the same for the shared expert
//   out[t] = ys[t] + sum_j w[t,j] y[t k + j]   moe_combine_kernel (fp32, fixed order)
//
// When the shared expert is as wide as a routed one (Ds == De) it is
// expert E of the same grouped GEMMs: T more rows, one per token, appended
// after the T k routed rows, with their own weight pointers; the down GEMM
// reuses the up GEMM's routing tables.  A forward is then the router GEMM,
// the top-k, one routing sort, two grouped GEMMs and the combine.
//
// Every step is a stream-ordered kernel; there is no host synchronisation,
// no per-expert loop and no scatter_reduce (the combine reads each token's
// k rows in order, so the output is deterministic).  Intermediates h, y, hs,
// ys are kept in the input dtype, as the reference's TileLang kernels do
// (up_logits and output buffers, kernels/fusedmoe_tilelang.py:290-305).
#include "common.h"
#include "mfma_tile.h"
#include "moe_hip.h"

#include <algorithm>
#include <string>

namespace moe {

// out[t, c] = (S ? S[t, c] : 0) + sum_j w[t, j] * Yr[t * k + j, c], fp32 sums,
// 8 columns per thread with 16-byte loads when the row pitch allows.
template <typename T>
__global__ __launch_bounds__(256) void moe_combine_kernel(const uint16_t* __restrict__ Yr,
                                                          const uint16_t* __restrict__ S,
                                                          const float* __restrict__ w, int64_t Tn, int k,
                                                          int64_t D, uint16_t* __restrict__ out) {
  const int64_t t = blockIdx.y;
  const int64_t c0 = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 8;
  if (t >= Tn || c0 >= D) return;
  float acc[8];
  const bool full = c0 + 8 <= D && (D % 8 == 0);
  auto load8 = [&](const uint16_t* p, float* v) {
    if (full) {
      const uint4 q = *reinterpret_cast<const uint4*>(p);
      const uint32_t u[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        v[2 * i] = __uint_as_float(Elem<T>::bits(reinterpret_cast<const T*>(&u[i])));
        v[2 * i + 1] = __uint_as_float(Elem<T>::bits(reinterpret_cast<const T*>(&u[i]) + 1));
      }
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i)
        v[i] = c0 + i < D ? __uint_as_float(Elem<T>::bits(reinterpret_cast<const T*>(p) + i)) : 0.0f;
    }
  };
  if (S) {
    load8(S + t * D + c0, acc);
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = 0.0f;
  }
  for (int j = 0; j < k; ++j) {
    float v[8];
    load8(Yr + (t * k + j) * D + c0, v);
    const float wj = w[t * k + j];
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] += wj * v[i];
  }
#pragma unroll
  for (int i = 0; i < 8; ++i)
    if (c0 + i < D) out[t * D + c0 + i] = MfmaOp<T>::cvt(acc[i]);
}

__global__ void fill_i32_kernel(int32_t* p, int64_t n, int32_t v) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    p[i] = v;
}

struct MoeLayout {
  size_t scratch;  // shared by the sub-calls, after the control block
  size_t logits, w, idx, zeros, h, y, hs, ys, total;
};

static size_t up256(size_t v) { return (v + 255) & ~(size_t)255; }

// The shared expert rides in the routed grouped GEMMs as expert E.
static bool moe_merged_shared(int64_t De, int64_t Ds) { return Ds > 0 && Ds == De; }

static MoeLayout moe_layout(int64_t T, int64_t Dh, int64_t De, int64_t Ds, int64_t E, int64_t k) {
  MoeLayout L;
  const size_t ctl = kWsCtlBytes;
  const bool merged = moe_merged_shared(De, Ds);
  const int64_t rows = T * k + (merged ? T : 0);  // rows of h and y
  size_t scratch = 0;
  auto take = [&](size_t ws) { scratch = std::max(scratch, ws > ctl ? ws - ctl : 0); };
  take(moe_router_workspace_size(T, Dh, E));
  take(moe_topk_softmax_workspace_size(T, E, k, MOE_TOPK_AUTO));
  if (merged) {
    take(grouped_gemm_ws_bytes(rows, E + 1));
  } else {
    take(moe_grouped_gemm_workspace_size(T, k, E, std::max(De, Dh)));
    take(moe_grouped_gemm_workspace_size(T * k, 1, E, Dh));
    if (Ds > 0) take(moe_grouped_gemm_workspace_size(T, 1, 1, std::max(Ds, Dh)));
  }
  L.scratch = up256(scratch);
  size_t o = ctl + L.scratch;
  L.logits = o; o += up256((size_t)T * E * 4);
  L.w = o; o += up256((size_t)T * k * 4);
  L.idx = o; o += up256((size_t)T * k * 4);
  L.zeros = o; o += up256(merged ? 0 : (size_t)T * 4);
  L.h = o; o += up256((size_t)rows * De * 2);
  L.y = o; o += up256((size_t)rows * Dh * 2);
  L.hs = o; o += up256(merged ? 0 : (size_t)T * std::max<int64_t>(Ds, 0) * 2);
  L.ys = o; o += up256(merged ? 0 : (size_t)T * (Ds > 0 ? Dh : 0) * 2);
  L.total = o;
  return L;
}

}  // namespace moe

using namespace moe;

extern "C" size_t moe_fused_moe_workspace_size(int64_t T, int64_t Dh, int64_t De, int64_t Ds, int64_t E,
                                               int64_t k) {
  if (T < 1 || Dh < 1 || De < 1 || Ds < 0 || E < 1 || k < 1 || k > E) return kWsCtlBytes;
  return moe_layout(T, Dh, De, Ds, E, k).total;
}

extern "C" int moe_combine(const void* Yr, const void* S, const float* w, int dtype, int64_t T, int64_t k,
                           int64_t D, void* out, void* stream) {
  if (T < 0 || k < 0 || D < 1) return fail(MOE_EINVAL, "combine: need T >= 0, k >= 0, D >= 1");
  if (dtype != MOE_BF16 && dtype != MOE_F16) return fail(MOE_EINVAL, "combine: dtype must be bfloat16 or float16");
  if (T == 0) return MOE_OK;
  if (!out || (k > 0 && (!Yr || !w))) return fail(MOE_EINVAL, "combine: null pointer");
  if ((D % 8 == 0) && (((uintptr_t)Yr | (uintptr_t)S) & 15))
    return fail(MOE_EINVAL, "combine: Yr and S must be 16-byte aligned");
  if (T > 65535 * 1024LL) return fail(MOE_EUNSUP, "combine: too many tokens");
  const dim3 grid((unsigned)((D + 2047) / 2048), (unsigned)T);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == MOE_BF16)
    moe_combine_kernel<uint16_t><<<grid, 256, 0, st>>>(static_cast<const uint16_t*>(Yr),
                                                       static_cast<const uint16_t*>(S), w, T, (int)k, D,
                                                       static_cast<uint16_t*>(out));
  else
    moe_combine_kernel<Half16><<<grid, 256, 0, st>>>(static_cast<const uint16_t*>(Yr),
                                                     static_cast<const uint16_t*>(S), w, T, (int)k, D,
                                                     static_cast<uint16_t*>(out));
  return check_launch("moe_combine_kernel");
}

extern "C" int moe_fused_moe(const void* x, const void* router_w, const void* shared_gate, const void* shared_up,
                             const void* shared_down, const void* routed_gate, const void* routed_up,
                             const void* routed_down, int dtype, int64_t T, int64_t Dh, int64_t De, int64_t Ds,
                             int64_t E, int64_t k, void* out, float* topk_weights, void* topk_ids,
                             void* workspace, size_t ws_bytes, void* stream) {
  if (T < 0 || Dh < 1 || De < 1 || Ds < 0 || E < 1 || k < 1 || k > E)
    return fail(MOE_EINVAL, "fused_moe: need T >= 0, Dh, De >= 1, Ds >= 0, 1 <= k <= E");
  if (Dh % 8 || De % 8 || Ds % 8) return fail(MOE_EUNSUP, "fused_moe: Dh, De and Ds must be multiples of 8");
  if (dtype != MOE_BF16 && dtype != MOE_F16) return fail(MOE_EINVAL, "fused_moe: dtype must be bfloat16 or float16");
  if (T == 0) return MOE_OK;
  if (!x || !router_w || !routed_gate || !routed_up || !routed_down || !out ||
      (Ds > 0 && (!shared_gate || !shared_up || !shared_down)))
    return fail(MOE_EINVAL, "fused_moe: null pointer");
  const MoeLayout L = moe_layout(T, Dh, De, Ds, E, k);
  if (!workspace || ws_bytes < L.total)
    return fail(MOE_EINVAL, "fused_moe: workspace too small (" + std::to_string(ws_bytes) + " < " +
                                std::to_string(L.total) + ")");
  char* ws = static_cast<char*>(workspace);
  const size_t sub = kWsCtlBytes + L.scratch;  // control block + scratch, reused by each step in turn
  float* logits = reinterpret_cast<float*>(ws + L.logits);
  float* w = topk_weights ? topk_weights : reinterpret_cast<float*>(ws + L.w);
  int32_t* idx = topk_ids ? static_cast<int32_t*>(topk_ids) : reinterpret_cast<int32_t*>(ws + L.idx);
  int32_t* zeros = reinterpret_cast<int32_t*>(ws + L.zeros);
  void* h = ws + L.h;
  void* y = ws + L.y;
  void* hs = ws + L.hs;
  void* ys = ws + L.ys;
  hipStream_t st = static_cast<hipStream_t>(stream);
  int rc;
  // 1. Router (the reference takes router_weight as [E, Dh]: already the
  //    transposed layout the router GEMM reads).
  //    A split-H router GEMM leaves G partial rows per token: the selection
  //    kernel sums them and selects (Convention A) in one launch.
  if (E <= 256) {
    const float* part = nullptr;
    int G = 1;
    if ((rc = router_gemm_logits_or_partials(x, router_w, dtype, T, Dh, E, logits, &part, &G, ws, sub, st))) return rc;
    rc = G > 1 ? topk_select_partials(part, G, T, (int)E, (int)k, MOE_SCORES_ALL, w, idx, MOE_I32, st)
               : moe_topk_softmax_ex(logits, MOE_F32, T, E, E, k, w, idx, MOE_I32, MOE_TOPK_AUTO, MOE_SCORES_ALL, ws,
                                     sub, stream);
  } else {
    if ((rc = moe_router_gemm(x, router_w, dtype, T, Dh, E, logits, ws, sub, stream))) return rc;
    rc = moe_topk_softmax_ex(logits, MOE_F32, T, E, E, k, w, idx, MOE_I32, MOE_TOPK_AUTO, MOE_SCORES_ALL, ws, sub,
                             stream);
  }
  if (rc) return rc;
  if (moe_merged_shared(De, Ds)) {
    // 2. Routed experts and the shared one (expert E, rows T k .. T k + T - 1
    //    = tokens 0 .. T - 1): gate/up with the SwiGLU epilogue, then down
    //    over the same routing tables (h row r is the down GEMM's X row r).
    GemmExtra up;
    up.Wx = shared_gate;
    up.W2x = shared_up;
    up.Tx = T;
    int bm = 0;
    if ((rc = grouped_gemm_run(1, x, routed_gate, routed_up, idx, dtype, MOE_I32, T, k, Dh, De, E, up, h, ws, sub, st,
                               &bm)))
      return rc;
    GemmExtra down;
    down.Wx = shared_down;
    down.Tx = T;
    down.x_shift = T * k;
    down.reuse_bm = bm;
    if ((rc = grouped_gemm_run(0, h, routed_down, nullptr, idx, dtype, MOE_I32, T * k, 1, De, Dh, E, down, y, ws, sub,
                               st, nullptr)))
      return rc;
    // 3. Combine: the shared rows follow the routed ones in y.
    return moe_combine(y, static_cast<char*>(y) + (size_t)T * k * Dh * 2, w, dtype, T, k, Dh, out, stream);
  }
  // 2. Routed experts: gate/up with the SwiGLU epilogue, then down.
  if ((rc = moe_grouped_gemm_swiglu(x, routed_gate, routed_up, idx, dtype, MOE_I32, T, k, Dh, De, E, h, ws, sub,
                                    stream)))
    return rc;
  if ((rc = moe_grouped_gemm(h, routed_down, idx, dtype, MOE_I32, T * k, 1, De, Dh, E, y, ws, sub, stream))) return rc;
  // 3. Shared expert: one expert that every token takes.
  if (Ds > 0) {
    fill_i32_kernel<<<(unsigned)std::min<int64_t>((T + 255) / 256, 1024), 256, 0, st>>>(zeros, T, 0);
    if ((rc = check_launch("fill_i32_kernel"))) return rc;
    if ((rc = moe_grouped_gemm_swiglu(x, shared_gate, shared_up, zeros, dtype, MOE_I32, T, 1, Dh, Ds, 1, hs, ws, sub,
                                      stream)))
      return rc;
    if ((rc = moe_grouped_gemm(hs, shared_down, zeros, dtype, MOE_I32, T, 1, Ds, Dh, 1, ys, ws, sub, stream)))
      return rc;
  }
  // 4. Combine.
  return moe_combine(y, Ds > 0 ? ys : nullptr, w, dtype, T, k, Dh, out, stream);
}
