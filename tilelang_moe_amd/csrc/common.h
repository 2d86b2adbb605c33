// Shared helpers of the gfx950 MoE hot-path kernels: error reporting for the
// C ABI, order-preserving float keys and wave64 cross-lane primitives.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
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

constexpr int kWave = 64;

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
// ---------------------------------------------------------------------------
__device__ inline uint32_t lane_id() { return __lane_id(); }

__device__ inline uint64_t shfl_xor_u64(uint64_t v, int mask) {
  uint32_t lo = (uint32_t)v, hi = (uint32_t)(v >> 32);
  lo = __shfl_xor(lo, mask, kWave);
  hi = __shfl_xor(hi, mask, kWave);
  return ((uint64_t)hi << 32) | lo;
}

__device__ inline uint64_t shfl_u64(uint64_t v, int src) {
  uint32_t lo = (uint32_t)v, hi = (uint32_t)(v >> 32);
  lo = __shfl(lo, src, kWave);
  hi = __shfl(hi, src, kWave);
  return ((uint64_t)hi << 32) | lo;
}

__device__ inline uint64_t umax64(uint64_t a, uint64_t b) { return a > b ? a : b; }
__device__ inline uint64_t umin64(uint64_t a, uint64_t b) { return a < b ? a : b; }

}  // namespace moe
