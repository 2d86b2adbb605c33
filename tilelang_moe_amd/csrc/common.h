// Shared helpers of the gfx950 MoE hot-path kernels: error reporting for the
// C ABI, order-preserving float keys and wave64 cross-lane primitives.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>
#include <string>

#include "../../include/moe_hip.h"

namespace moe {

// ---------------------------------------------------------------------------
// Host-side error state (thread-local, read through moe_last_error()).
// ---------------------------------------------------------------------------
void set_error(const std::string& msg);
int fail(int code, const std::string& msg);
int check_launch(const char* what);

#define MOE_HIP_CHECK(expr)                                                    \
  do {                                                                         \
    hipError_t _e = (expr);                                                    \
    if (_e != hipSuccess)                                                      \
      return ::moe::fail(MOE_EHIP, std::string(#expr) + ": " +                 \
                                       hipGetErrorString(_e));                 \
  } while (0)

// Raises a kernel's dynamic-LDS limit to `bytes` once per device, on the
// device of the launch stream `st` (made current for the call if it is not).
// `done` is the call site's static mask of devices already set (device d <
// 64 is bit d); concurrent first calls may both set the attribute, which is
// harmless.  Returns hipSuccess or the failing call's error.
inline hipError_t lds_cap_once(std::atomic<uint64_t>& done, const void* kernel, int bytes, hipStream_t st) {
  hipDevice_t dev = 0;
  hipError_t e = hipStreamGetDevice(st, &dev);
  if (e != hipSuccess) return e;
  const uint64_t bit = 1ull << (dev & 63);
  if (done.load(std::memory_order_acquire) & bit) return hipSuccess;
  int cur = 0;
  if ((e = hipGetDevice(&cur)) != hipSuccess) return e;
  if (cur != dev && (e = hipSetDevice(dev)) != hipSuccess) return e;
  e = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  if (cur != dev) {
    const hipError_t r = hipSetDevice(cur);
    if (e == hipSuccess) e = r;
  }
  if (e == hipSuccess) done.fetch_or(bit, std::memory_order_release);
  return e;
}

// Top-K + softmax of the rows sum_g part[g][M][N], g in order 0..G-1 (fp32
// partials of a split-H router GEMM), N <= 256; one wave per row.
// score_mode MOE_SCORES_TOPK (Convention B) or MOE_SCORES_ALL (A).
// Defined with the selection kernel (router.hip).
int topk_select_partials(const float* part, int G, int64_t M, int N, int K, int score_mode, float* scores,
                         void* indices, int idx_dtype, hipStream_t st);
// Router GEMM for the fused paths: the plan's split count G, and either the
// logits [T, E] (G == 1, written to `logits`) or G partial rows per token
// (G > 1, returned in *part, inside the workspace).  Defined with the
// router GEMM (router_gemm.hip).
int router_gemm_logits_or_partials(const void* X, const void* Wt, int dtype, int64_t T, int64_t H, int64_t E,
                                   float* logits, const float** part, int* G, void* workspace, size_t ws_bytes,
                                   hipStream_t st);

// Grouped GEMM with an appended expert and reusable routing tables, for
// the FusedMoE path (defined with the grouped GEMM, gemm.hip).  Rows
// T*topk .. T*topk + Tx - 1 form expert E, with weights Wx (and W2x for the
// SwiGLU epilogue) and X row r - T*topk + x_shift.  reuse_bm = 0 sorts the
// rows; reuse_bm = b > 0 reuses the routing tables an earlier call on the
// same workspace built for the same rows with tile height b (bm_used);
// reuse_bm < 0 reuses the tables of an earlier call of the same shape.
struct GemmExtra {
  const void* Wx = nullptr;
  const void* W2x = nullptr;
  int64_t Tx = 0;
  int64_t x_shift = 0;
  int reuse_bm = 0;
};
size_t grouped_gemm_ws_bytes(int64_t R, int64_t E);
int grouped_gemm_run(int epi, const void* X, const void* W, const void* W2, const void* expert_ids, int dtype,
                     int idx_dtype, int64_t T, int64_t topk, int64_t H, int64_t I, int64_t E, const GemmExtra& ex,
                     void* Y, void* workspace, size_t ws_bytes, hipStream_t stream, int* bm_used);

constexpr int kWave = 64;
// Every workspace starts with a control block of this size: the only bytes
// that must be zero before a call, and every call leaves them zero.  Scratch
// follows it and is overwritten freely, so one workspace can serve every
// entry point in turn on one stream.
constexpr size_t kWsCtlBytes = 4096;


// Workgroup barrier that orders LDS only.  __syncthreads() carries a
// workgroup fence over every address space, which waits for all of the
// wave's outstanding global loads (vmcnt(0)); this one waits for LDS
// traffic alone (lgkmcnt(0)), so row loads issued earlier stay in flight.
__device__ inline void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// ---------------------------------------------------------------------------
// Order-preserving 32-bit keys.  key(a) > key(b)  <=>  a > b, with -0.0 and
// +0.0 mapped to one key and every NaN mapped to the largest key (torch.topk
// ranks NaN above +inf).  Key 0 is never produced by a real value (the
// smallest, -inf, maps to 0x007FFFFF), so 0 is the padding key.
// ---------------------------------------------------------------------------
__host__ __device__ inline uint32_t key_of_bits(uint32_t u) {
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0xFFFFFFFFu;  // NaN
  if (u == 0x80000000u) u = 0u;                              // -0 -> +0
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Plain sign-flip key (3 ALU ops): equals key_of_bits except for NaN and
// -0.0, which callers detect and re-key.
__host__ __device__ inline uint32_t key_fast(uint32_t u) {
  return u ^ ((uint32_t)((int32_t)u >> 31) | 0x80000000u);
}
__host__ __device__ inline uint32_t bits_of_fast_key(uint32_t k) {
  return (k & 0x80000000u) ? (k ^ 0x80000000u) : ~k;
}

__host__ __device__ inline float value_of_key(uint32_t k) {
  uint32_t u = (k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k;
  union { uint32_t u; float f; } c;
  c.u = u;
  return c.f;
}

// Composite 64-bit sort key: value key in the high word, bitwise-NOT of the
// column index in the low word.  Descending order of the composite is
// "value descending, then index ascending"; every composite is unique.
__host__ __device__ inline uint64_t make_comp(uint32_t key, uint32_t idx) {
  return ((uint64_t)key << 32) | (uint32_t)(~idx);
}
__host__ __device__ inline uint32_t comp_key(uint64_t c) { return (uint32_t)(c >> 32); }
__host__ __device__ inline uint32_t comp_idx(uint64_t c) { return ~(uint32_t)c; }

// Element loads of the three logits dtypes, returned as fp32 bit patterns.
template <typename T> struct Elem;
template <> struct Elem<float> {
  static __device__ inline uint32_t bits(const float* p) { return __float_as_uint(*p); }
};
template <> struct Elem<uint16_t> {  // bfloat16 storage
  static __device__ inline uint32_t bits(const uint16_t* p) { return ((uint32_t)*p) << 16; }
};
struct Half16 { uint16_t v; };
template <> struct Elem<Half16> {
  static __device__ inline uint32_t bits(const Half16* p) {
    _Float16 h;
    __builtin_memcpy(&h, &p->v, 2);
    return __float_as_uint((float)h);
  }
};

// ---------------------------------------------------------------------------
// Wave64 cross-lane helpers.
// xor_lanes<M> returns x from lane (lane ^ M) without going through the LDS
// crossbar: DPP quad permutes for M = 1, 2, DPP row shifts for 4, a DPP row
// rotate for 8 and the gfx950 v_permlane16/32_swap for 16 and 32.  Scans and
// reductions are DPP row shifts / mirrors plus row broadcasts or readlanes.
// ---------------------------------------------------------------------------
__device__ inline uint32_t lane_id() { return __lane_id(); }

template <int CTRL, int ROW_MASK = 0xF, int BANK_MASK = 0xF>
__device__ inline uint32_t dpp(uint32_t old, uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp((int)old, (int)v, CTRL, ROW_MASK, BANK_MASK, false);
}
constexpr int kDppQuadXor1 = 0xB1;     // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;     // quad_perm [2,3,0,1]
constexpr int kDppRowShl4 = 0x104;     // lane n <- n+4 (within a 16-lane row)
constexpr int kDppRowShr1 = 0x111;     // lane n <- n-1
constexpr int kDppRowShr2 = 0x112;
constexpr int kDppRowShr4 = 0x114;
constexpr int kDppRowShr8 = 0x118;
constexpr int kDppRowRor8 = 0x128;     // lane n <- (n+8) mod 16 = n^8
constexpr int kDppRowMirror = 0x140;   // lane n <- 15-n
constexpr int kDppRowHalfMirror = 0x141;  // lane n <- 7-n (within 8)
constexpr int kDppRowBcast15 = 0x142;  // row r+1 <- lane 15 of row r
constexpr int kDppRowBcast31 = 0x143;  // rows 2,3 <- lane 31

template <int M>
__device__ inline uint32_t xor_lanes(uint32_t x) {
  if constexpr (M == 1) {
    return dpp<kDppQuadXor1>(x, x);
  } else if constexpr (M == 2) {
    return dpp<kDppQuadXor2>(x, x);
  } else if constexpr (M == 4) {
    const uint32_t up = dpp<kDppRowShl4>(x, x), dn = dpp<kDppRowShr4>(x, x);
    return (__lane_id() & 4) ? dn : up;
  } else if constexpr (M == 8) {
    return dpp<kDppRowRor8>(x, x);
  } else if constexpr (M == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(x, x, false, false);
    return ((__lane_id() >> 4) & 1) ? r[0] : r[1];
  } else {
    static_assert(M == 32, "xor_lanes: M must be a power of two below 64");
    const auto r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
    return (__lane_id() < 32) ? r[1] : r[0];
  }
}

template <int M>
__device__ inline uint64_t xor_lanes_u64(uint64_t v) {
  const uint32_t lo = xor_lanes<M>((uint32_t)v), hi = xor_lanes<M>((uint32_t)(v >> 32));
  return ((uint64_t)hi << 32) | lo;
}
template <int M>
__device__ inline float xor_lanes_f32(float v) {
  return __uint_as_float(xor_lanes<M>(__float_as_uint(v)));
}

// Runtime-mask variant (M a power of two < 64) for loops the compiler unrolls.
__device__ inline uint64_t xor_lanes_u64(uint64_t v, int m) {
  switch (m) {
    case 1: return xor_lanes_u64<1>(v);
    case 2: return xor_lanes_u64<2>(v);
    case 4: return xor_lanes_u64<4>(v);
    case 8: return xor_lanes_u64<8>(v);
    case 16: return xor_lanes_u64<16>(v);
    default: return xor_lanes_u64<32>(v);
  }
}
__device__ inline float xor_lanes_f32(float v, int m) {
  const uint32_t u = __float_as_uint(v);
  uint32_t r;
  switch (m) {
    case 1: r = xor_lanes<1>(u); break;
    case 2: r = xor_lanes<2>(u); break;
    case 4: r = xor_lanes<4>(u); break;
    case 8: r = xor_lanes<8>(u); break;
    case 16: r = xor_lanes<16>(u); break;
    default: r = xor_lanes<32>(u); break;
  }
  return __uint_as_float(r);
}

// Inclusive prefix sum over the 64 lanes.
__device__ inline uint32_t wave_incl_scan(uint32_t x) {
  x += dpp<kDppRowShr1>(0u, x);
  x += dpp<kDppRowShr2>(0u, x);
  x += dpp<kDppRowShr4>(0u, x);
  x += dpp<kDppRowShr8>(0u, x);
  x += dpp<kDppRowBcast15, 0xA>(0u, x);
  x += dpp<kDppRowBcast31, 0xC>(0u, x);
  return x;
}

// All-lane reductions.
__device__ inline uint32_t wave_max_u32(uint32_t x) {
  x = max(x, dpp<kDppQuadXor1>(x, x));
  x = max(x, dpp<kDppQuadXor2>(x, x));
  x = max(x, dpp<kDppRowHalfMirror>(x, x));
  x = max(x, dpp<kDppRowMirror>(x, x));
  const uint32_t a = __builtin_amdgcn_readlane(x, 0), b = __builtin_amdgcn_readlane(x, 16);
  const uint32_t c = __builtin_amdgcn_readlane(x, 32), d = __builtin_amdgcn_readlane(x, 48);
  return max(max(a, b), max(c, d));
}

__device__ inline float wave_sum_f32(float v) {
  uint32_t x = __float_as_uint(v);
  x = __float_as_uint(__uint_as_float(x) + __uint_as_float(dpp<kDppQuadXor1>(x, x)));
  x = __float_as_uint(__uint_as_float(x) + __uint_as_float(dpp<kDppQuadXor2>(x, x)));
  x = __float_as_uint(__uint_as_float(x) + __uint_as_float(dpp<kDppRowHalfMirror>(x, x)));
  x = __float_as_uint(__uint_as_float(x) + __uint_as_float(dpp<kDppRowMirror>(x, x)));
  const float a = __uint_as_float(__builtin_amdgcn_readlane(x, 0));
  const float b = __uint_as_float(__builtin_amdgcn_readlane(x, 16));
  const float c = __uint_as_float(__builtin_amdgcn_readlane(x, 32));
  const float d = __uint_as_float(__builtin_amdgcn_readlane(x, 48));
  return (a + b) + (c + d);
}

__device__ inline uint64_t umax64(uint64_t a, uint64_t b) { return a > b ? a : b; }
__device__ inline uint64_t umin64(uint64_t a, uint64_t b) { return a < b ? a : b; }

__device__ inline uint64_t readlane_u64(uint64_t v, int l) {
  const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)v, l);
  const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)(v >> 32), l);
  return ((uint64_t)hi << 32) | lo;
}

__device__ inline uint64_t wave_max_u64(uint64_t x) {
  x = umax64(x, xor_lanes_u64<1>(x));
  x = umax64(x, xor_lanes_u64<2>(x));
  x = umax64(x, xor_lanes_u64<4>(x));
  x = umax64(x, xor_lanes_u64<8>(x));
  const uint64_t a = readlane_u64(x, 0), b = readlane_u64(x, 16);
  const uint64_t c = readlane_u64(x, 32), d = readlane_u64(x, 48);
  return umax64(umax64(a, b), umax64(c, d));
}

__device__ inline uint32_t xor_lanes_u32(uint32_t x, int m) {
  return __float_as_uint(xor_lanes_f32(__uint_as_float(x), m));
}

// 32-bit composites of bfloat16 values: the order-preserving key of a
// bfloat16 value is 16 bits wide (the key of its fp32 widening shifted
// right by 16: the dropped bits are constant for a given sign), so key and
// column (< 65536) pack into one unique 32-bit composite
// (key16 << 16) | (0xFFFF - column): larger means a larger value, then a
// lower column; 0 is below every real composite.
__device__ inline uint32_t comp16_of(uint32_t bits16, int col) {
  return ((key_of_bits(bits16 << 16) >> 16) << 16) | (0xFFFFu - (uint32_t)col);
}
__device__ inline float value_of_comp16(uint32_t c) {
  const uint32_t k16 = c >> 16;
  return value_of_key((k16 << 16) | ((k16 & 0x8000u) ? 0u : 0xFFFFu));
}

// ---------------------------------------------------------------------------
// Segment helpers: a segment is one 16-lane DPP row of the wave.
// ---------------------------------------------------------------------------
__device__ inline uint32_t seg16_shfl(uint32_t v, int src) {
  return (uint32_t)__builtin_amdgcn_ds_bpermute(((int)(__lane_id() & ~15u) + src) << 2, (int)v);
}
__device__ inline uint64_t seg16_shfl_u64(uint64_t v, int src) {
  return ((uint64_t)seg16_shfl((uint32_t)(v >> 32), src) << 32) | seg16_shfl((uint32_t)v, src);
}
__device__ inline uint32_t seg16_incl_scan(uint32_t x) {
  x += dpp<kDppRowShr1>(0u, x);
  x += dpp<kDppRowShr2>(0u, x);
  x += dpp<kDppRowShr4>(0u, x);
  x += dpp<kDppRowShr8>(0u, x);
  return x;
}
__device__ inline uint32_t seg16_sum(uint32_t x) {
  x += xor_lanes<1>(x);
  x += xor_lanes<2>(x);
  x += xor_lanes<4>(x);
  x += xor_lanes<8>(x);
  return x;
}
// Descending bitonic sort of one value per lane over the segment.
template <typename V>
__device__ inline V seg16_sort_desc(V v) {
  const int pos = __lane_id() & 15;
#pragma unroll
  for (int k2 = 2; k2 <= 16; k2 <<= 1) {
#pragma unroll
    for (int j = k2 >> 1; j > 0; j >>= 1) {
      V o;
      if constexpr (sizeof(V) == 8) o = xor_lanes_u64(v, j);
      else o = (V)__float_as_uint(xor_lanes_f32(__uint_as_float((uint32_t)v), j));
      const bool desc = (pos & k2) == 0, lower = (pos & j) == 0;
      v = (desc == lower) ? (v > o ? v : o) : (v < o ? v : o);
    }
  }
  return v;
}

// Top-K (K <= 16) of one row held by a segment: lane pos holds keys key[i]
// of columns col(pos, i) (key 0 = no element).  The K-th largest of the 16
// lane maxima, tau, is a lower bound of the row's K-th largest key (K
// lanes hold a key >= tau), so every winner is among the keys >= tau.
// Those are compacted into the segment's 16 LDS slots and sorted as
// composites (key desc, column asc); lane r < K returns winner r in `out`.
// Returns false, leaving `out` alone, when K > 16 or more than 16 keys are
// >= tau (segment-uniform).
template <int EPL, typename ColFn>
__device__ inline bool seg16_topk_filtered(const uint32_t (&key)[EPL], int K, uint64_t* scratch, uint64_t& out,
                                           ColFn col) {
  if (K > 16) return false;
  const int pos = __lane_id() & 15;
  uint32_t m = key[0];
#pragma unroll
  for (int i = 1; i < EPL; ++i) m = max(m, key[i]);
  const uint32_t tau = max(seg16_shfl(seg16_sort_desc(m), K - 1), 1u);
  uint32_t cnt = 0;
#pragma unroll
  for (int i = 0; i < EPL; ++i) cnt += key[i] >= tau;
  const uint32_t total = seg16_sum(cnt);
  if (total > 16) return false;
  uint32_t p = seg16_incl_scan(cnt) - cnt;
#pragma unroll
  for (int i = 0; i < EPL; ++i)
    if (key[i] >= tau) scratch[p++] = make_comp(key[i], (uint32_t)col(pos, i));
  __builtin_amdgcn_wave_barrier();  // LDS ops of one wave complete in order
  const uint64_t c = seg16_sort_desc<uint64_t>(pos < (int)total ? scratch[pos] : 0);
  __builtin_amdgcn_wave_barrier();  // the slots are reused by the next row
  out = pos < K ? c : 0;
  return true;
}

}  // namespace moe
