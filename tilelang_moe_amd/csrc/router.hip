// Fused TopK + softmax router kernels for gfx950.
//
// Three algorithms, selected by row length N (moe_topk_select_algo):
//   bitonic   N <= 64     one wave64 sorts 64/S rows of S = pow2 >= N lanes
//                         with a register bitonic network (no LDS, no barrier)
//   selection N <= 1024   one wave64 per row, K rounds of a wave argmax over
//                         the row held in VGPRs (lane l owns l, l+64, ...)
//   radix     any N       one workgroup per row, three histogram passes over
//                         11/11/10-bit digits of the order-preserving key,
//                         then an LDS bitonic sort of the K winners
// Every kernel ends with the Convention-B softmax of the reference baseline
// (kernels/topk_softmax_baseline.py:39-66): scores = exp(v - v0) / sum, over
// the K selected values in descending order.
#include "common.h"

#include <algorithm>
#include <type_traits>

namespace moe {

// ---------------------------------------------------------------------------
// Output helper.
// ---------------------------------------------------------------------------
template <typename IdxT>
__device__ inline void store_out(float* scores, IdxT* indices, int64_t off, float s,
                                 uint32_t idx) {
  if (scores) scores[off] = s;
  indices[off] = (IdxT)idx;
}

// ===========================================================================
// 1. Wave64 bitonic network, N <= 64.
//    Replaces _make_topk_softmax_bitonic_kernel (kernels/topk_softmax_tilelang.py:463-538),
//    which sorts a padded row in shared memory with a barrier per stage.
//    Here a segment of S lanes (S = next pow2 >= N) holds one row, so a wave
//    sorts 64/S rows at once and every compare-exchange is a lane shuffle.
// ===========================================================================
//    bfloat16 rows sort 32-bit composites (comp16_of) instead of 64-bit ones.
template <typename T, int S, typename IdxT>
__global__ __launch_bounds__(256) void topk_bitonic_kernel(const T* __restrict__ logits,
                                                           int64_t M, int N, int64_t ld,
                                                           int K, float* __restrict__ scores,
                                                           IdxT* __restrict__ indices) {
  constexpr int RPW = kWave / S;  // rows per wave
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int pos = lane & (S - 1);
  const int64_t row = ((int64_t)blockIdx.x * (blockDim.x / kWave) + wave) * RPW + lane / S;

  if constexpr (std::is_same<T, uint16_t>::value) {
    uint32_t c = (row < M && pos < N) ? comp16_of(logits[row * ld + pos], pos) : 0u;
#pragma unroll
    for (int k = 2; k <= S; k <<= 1) {
#pragma unroll
      for (int j = k >> 1; j > 0; j >>= 1) {
        const uint32_t o = xor_lanes_u32(c, j);
        const bool desc = (pos & k) == 0;
        const bool lower = (pos & j) == 0;
        c = (desc == lower) ? max(c, o) : min(c, o);
      }
    }
    uint32_t cmax = c;  // the segment head holds the largest
#pragma unroll
    for (int j = 1; j < S; j <<= 1) cmax = max(cmax, xor_lanes_u32(cmax, j));
    const float vmax = value_of_comp16(cmax);
    const float e = pos < K ? expf(value_of_comp16(c) - vmax) : 0.0f;
    float sum = e;
#pragma unroll
    for (int j = 1; j < S; j <<= 1) sum += xor_lanes_f32(sum, j);
    if (row < M && pos < K) store_out(scores, indices, row * K + pos, e / sum, 0xFFFFu - (c & 0xFFFFu));
    return;
  }

  uint64_t c = 0;  // padding composite sorts last
  if (row < M && pos < N) c = make_comp(key_of_bits(Elem<T>::bits(logits + row * ld + pos)), pos);

#pragma unroll
  for (int k = 2; k <= S; k <<= 1) {
#pragma unroll
    for (int j = k >> 1; j > 0; j >>= 1) {
      const uint64_t o = xor_lanes_u64(c, j);
      const bool desc = (pos & k) == 0;
      const bool lower = (pos & j) == 0;
      c = (desc == lower) ? umax64(c, o) : umin64(c, o);
    }
  }

  // Softmax over positions [0, K) of each segment.
  const float v = value_of_key(comp_key(c));
  uint32_t kmax = comp_key(c);  // segment head holds the largest key
#pragma unroll
  for (int j = 1; j < S; j <<= 1) {
    const uint64_t o = xor_lanes_u64((uint64_t)kmax, j);
    kmax = max(kmax, (uint32_t)o);
  }
  const float vmax = value_of_key(kmax);
  float e = pos < K ? expf(v - vmax) : 0.0f;
  float sum = e;
#pragma unroll
  for (int j = 1; j < S; j <<= 1) sum += xor_lanes_f32(sum, j);
  if (row < M && pos < K) store_out(scores, indices, row * K + pos, e / sum, comp_idx(c));
}

// ===========================================================================
// 2. Selection, one wave64 per row.
//    Replaces topk_softmax_selection_kernel (kernels/topk_softmax_tilelang.py:312-449):
//    K rounds of "argmax, ties to the lower index, then exclude the winner".
//    The reference does a per-thread scan plus an LDS tree with 8 barriers
//    per round and rescans its already-selected list; here the row lives in
//    VGPRs (EPL composites per lane), a round is a 6-step xor butterfly on
//    unique 64-bit composites and the winner is cleared in place.
//    The K winners are staged in LDS for the softmax epilogue.
// ===========================================================================
// With PSUM (fp32 rows only) the row is the sum, in order g = 0..G-1, of the
// G partial rows logits + g * gstride (split-H router GEMM partials), and
// all_scores selects Convention A: exp(v - max) / sum over the whole row
// (NaN everywhere if the row holds a NaN, as torch.softmax).
template <typename T, int EPL, typename IdxT, bool PSUM = false>
__global__ __launch_bounds__(256) void topk_select_kernel(const T* __restrict__ logits,
                                                          int64_t M, int N, int64_t ld,
                                                          int K, float* __restrict__ scores,
                                                          IdxT* __restrict__ indices, int G = 1,
                                                          int64_t gstride = 0, bool all_scores = false) {
  extern __shared__ uint64_t win_all[];  // [waves][K]
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int64_t row = (int64_t)blockIdx.x * (blockDim.x / kWave) + wave;
  const bool live = row < M;  // wave-uniform
  uint64_t* win = win_all + (size_t)wave * K;
  const T* x = logits + (live ? row : 0) * ld;

  uint64_t c[EPL];
  if constexpr (PSUM) {
    static_assert(sizeof(T) == 4, "partial sums are fp32");
    float v[EPL];
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
      const int idx = lane + kWave * i;
      v[i] = (live && idx < N) ? x[idx] : 0.0f;
    }
    // Eight partial rows in flight at a time, added in split order.
    for (int g0 = 1; g0 < G; g0 += 8) {
      float p[8][EPL];
#pragma unroll
      for (int q = 0; q < 8; ++q)
#pragma unroll
        for (int i = 0; i < EPL; ++i) {
          const int idx = lane + kWave * i;
          p[q][i] = (live && idx < N && g0 + q < G) ? x[(size_t)(g0 + q) * gstride + idx] : 0.0f;
        }
#pragma unroll
      for (int q = 0; q < 8; ++q)
#pragma unroll
        for (int i = 0; i < EPL; ++i)
          if (g0 + q < G) v[i] += p[q][i];
    }
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
      const int idx = lane + kWave * i;
      c[i] = (live && idx < N) ? make_comp(key_of_bits(__float_as_uint(v[i])), idx) : 0;
    }
    if (all_scores) {
      // Convention A: the normaliser over all N values, taken against the
      // row maximum (the first winner; a NaN maximum makes every score NaN).
      uint64_t best = c[0];
#pragma unroll
      for (int i = 1; i < EPL; ++i) best = umax64(best, c[i]);
      const float m = value_of_key(comp_key(wave_max_u64(best)));
      float sa = 0.0f;
#pragma unroll
      for (int i = 0; i < EPL; ++i)
        if (lane + kWave * i < N) sa += expf(v[i] - m);
      sa = wave_sum_f32(sa);
      for (int r = 0; r < K; ++r) {
        uint64_t b = c[0];
#pragma unroll
        for (int i = 1; i < EPL; ++i) b = umax64(b, c[i]);
        b = wave_max_u64(b);
#pragma unroll
        for (int i = 0; i < EPL; ++i) c[i] = (c[i] == b) ? 0 : c[i];
        if (lane == 0) win[r] = b;
      }
      __syncthreads();
      if (!live) return;
      for (int r = lane; r < K; r += kWave) {
        const uint64_t w = win[r];
        store_out(scores, indices, row * K + r, expf(value_of_key(comp_key(w)) - m) / sa, comp_idx(w));
      }
      return;
    }
  } else {
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
      const int idx = lane + kWave * i;
      c[i] = (live && idx < N) ? make_comp(key_of_bits(Elem<T>::bits(x + idx)), idx) : 0;
    }
  }

  for (int r = 0; r < K; ++r) {
    uint64_t best = c[0];
#pragma unroll
    for (int i = 1; i < EPL; ++i) best = umax64(best, c[i]);
    best = wave_max_u64(best);
#pragma unroll
    for (int i = 0; i < EPL; ++i) c[i] = (c[i] == best) ? 0 : c[i];
    if (lane == 0) win[r] = best;
  }
  __syncthreads();
  if (!live) return;

  const float vmax = value_of_key(comp_key(win[0]));
  float sum = 0.0f;
  for (int r = lane; r < K; r += kWave) sum += expf(value_of_key(comp_key(win[r])) - vmax);
  sum = wave_sum_f32(sum);
  for (int r = lane; r < K; r += kWave) {
    const uint64_t w = win[r];
    store_out(scores, indices, row * K + r, expf(value_of_key(comp_key(w)) - vmax) / sum,
              comp_idx(w));
  }
}

// ===========================================================================
// 2c. Selection for bfloat16 rows: the order-preserving key of a bfloat16
//     value is 16 bits wide (the key of its fp32 widening shifted right by
//     16: the dropped bits are constant for a given sign), so the key and
//     the column (N <= 65536) pack into one unique 32-bit composite
//     (key16 << 16) | (0xFFFF - column): a larger composite is a larger
//     value, then a lower column, as everywhere.  A round of the selection is
//     then a 32-bit wave max (DPP max steps) instead of 64-bit
//     compare-and-select butterflies.  Same results as topk_select_kernel.
// ===========================================================================

template <int EPL, typename IdxT, bool VEC4 = false>
__global__ __launch_bounds__(256) void topk_select16_kernel(const uint16_t* __restrict__ logits, int64_t M, int N,
                                                            int64_t ld, int K, float* __restrict__ scores,
                                                            IdxT* __restrict__ indices) {
  extern __shared__ uint32_t win16_all[];  // [waves][K]
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int64_t row = (int64_t)blockIdx.x * (blockDim.x / kWave) + wave;
  const bool live = row < M;  // wave-uniform
  uint32_t* win = win16_all + (size_t)wave * K;
  const uint16_t* x = logits + (live ? row : 0) * ld;
  uint32_t c[EPL];
  if constexpr (VEC4) {
    // Four consecutive columns per lane and 8-byte load (N % 4 == 0, rows
    // 8-byte aligned): lane l holds columns 4 (l + 64 j) .. + 3.
#pragma unroll
    for (int j = 0; j < EPL / 4; ++j) {
      const int col = 4 * (lane + kWave * j);
      uint64_t v = 0;
      if (live && col < N) v = *reinterpret_cast<const uint64_t*>(x + col);
#pragma unroll
      for (int t = 0; t < 4; ++t)
        c[4 * j + t] = (live && col < N) ? comp16_of((uint16_t)(v >> (16 * t)), col + t) : 0u;
    }
  } else {
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
      const int idx = lane + kWave * i;
      c[i] = (live && idx < N) ? comp16_of(x[idx], idx) : 0u;  // 0: below every real composite
    }
  }
  for (int r = 0; r < K; ++r) {
    uint32_t best = c[0];
#pragma unroll
    for (int i = 1; i < EPL; ++i) best = max(best, c[i]);
    best = wave_max_u32(best);
#pragma unroll
    for (int i = 0; i < EPL; ++i) c[i] = c[i] == best ? 0u : c[i];
    if (lane == 0) win[r] = best;
  }
  __syncthreads();
  if (!live) return;
  const float vmax = value_of_comp16(win[0]);
  float sum = 0.0f;
  for (int r = lane; r < K; r += kWave) sum += expf(value_of_comp16(win[r]) - vmax);
  sum = wave_sum_f32(sum);
  for (int r = lane; r < K; r += kWave) {
    const uint32_t w = win[r];
    store_out(scores, indices, row * K + r, expf(value_of_comp16(w) - vmax) / sum, 0xFFFFu - (w & 0xFFFFu));
  }
}

// ===========================================================================
// 3. Radix select.
//    Replaces tl_topk_radix_kernel (kernels/topk_softmax_tilelang.py:54-202)
//    plus the torch gather + softmax that follows it (:1128-1131).
//    One 1024-thread workgroup per row.  Digits: bits 31..21, 20..10, 9..0 of
//    the 32-bit key.  Pass p builds a 2048-bin LDS histogram of digit p over
//    the elements whose higher digits equal the threshold prefix found so
//    far, and picks the bin that holds the K-th largest; a pass stops the
//    search early when that whole bin is taken.  The K winners are then put
//    in descending order in LDS and the softmax is applied in the same kernel.
//
//    topk_radix_reg_kernel (N <= 64K, K <= 8192) reads the row from HBM once
//    with 16-byte loads and keeps its keys in VGPRs for every pass.  Its
//    ordering step is a counting sort of the winners on (key - base) >> s
//    (base = smallest possible winner key, s chosen so the winners span at
//    most 4096 buckets) followed by an insertion sort inside each bucket;
//    rows whose winners crowd one bucket (> 32) fall back to a bitonic sort.
//    topk_radix_kernel handles any N and K <= 16384 by re-reading the row
//    from L2 in every pass.
// ===========================================================================
constexpr int kRadixThreads = 1024;
constexpr int kRadixBins = 2048;
constexpr int kBucketFixMax = 32;

__device__ inline uint32_t block_excl_scan_1024(uint32_t v, uint32_t* wsum, uint32_t* total) {
  // Exclusive prefix sum over a 1024-thread block; wsum needs 16 slots.
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const uint32_t incl = wave_incl_scan(v);
  if (lane == kWave - 1) wsum[wave] = incl;
  __syncthreads();
  uint32_t base = 0, tot = 0;
#pragma unroll
  for (int w = 0; w < kRadixThreads / kWave; ++w) {
    const uint32_t s = wsum[w];
    base += (w < wave) ? s : 0;
    tot += s;
  }
  if (total) *total = tot;
  __syncthreads();
  return base + incl - v;
}

// Threshold search shared by both radix kernels: after pass p the caller
// has filled hist[] with digit p over keys whose decided digits equal prefix.
struct RadixState {
  uint32_t prefix, fixed, need, eq_count;
  bool all_taken;
};

__device__ inline void radix_pick_bin(RadixState& st, const uint32_t* hist, int sh, uint32_t dm,
                                      uint32_t* wsum, uint32_t* s_pick) {
  const int tid = threadIdx.x;
  // Bins in descending order: thread t owns bins 2047-2t and 2046-2t.
  const int b0 = kRadixBins - 1 - 2 * tid, b1 = b0 - 1;
  const uint32_t h0 = hist[b0], h1 = hist[b1];
  const uint32_t above0 = block_excl_scan_1024(h0 + h1, wsum, nullptr);
  const uint32_t above1 = above0 + h0;
  if (above0 < st.need && st.need <= above0 + h0) { s_pick[0] = b0; s_pick[1] = above0; }
  if (above1 < st.need && st.need <= above1 + h1) { s_pick[0] = b1; s_pick[1] = above1; }
  __syncthreads();
  const uint32_t bin = s_pick[0];
  st.need -= s_pick[1];
  st.prefix |= bin << sh;
  st.fixed |= dm << sh;
  st.eq_count = hist[bin];
  st.all_taken = st.eq_count == st.need;
  __syncthreads();
}

// Same contract as radix_pick_bin with one barrier: the caller has
// completed hist[] (barrier passed); wave 0 alone scans the 2048 bins in
// descending order, each lane summing a block of 32, and publishes the bin
// holding the need-th largest.  hist must be 16-byte aligned (uint4 reads).
__device__ inline void radix_pick_bin_w0(RadixState& st, const uint32_t* hist, int sh, uint32_t dm,
                                         uint32_t* s_pick) {
  if (threadIdx.x < kWave) {
    // Level 1: lane l sums the 32 bins kRadixBins-32(l+1) .. kRadixBins-32l-1.
    const int lane = threadIdx.x;
    const int lo = kRadixBins - 32 * (lane + 1);
    const uint4* h4 = reinterpret_cast<const uint4*>(hist + lo);
    uint32_t sum = 0;
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const uint4 t = h4[q];
      sum += (t.x + t.y) + (t.z + t.w);
    }
    const uint32_t incl = wave_incl_scan(sum);
    const uint32_t above = incl - sum;
    const uint64_t hit = __ballot(above < st.need && st.need <= incl);
    const int L1 = __ffsll((long long)hit) - 1;
    const uint32_t above1 = __builtin_amdgcn_readlane(above, L1);
    // Level 2: the 32 bins of block L1, one per lane, in descending order.
    const int lo1 = kRadixBins - 32 * (L1 + 1);
    const uint32_t v = lane < 32 ? hist[lo1 + 31 - lane] : 0u;
    const uint32_t incl2 = wave_incl_scan(v);
    const uint32_t a2 = above1 + incl2 - v;
    const uint64_t hit2 = __ballot(lane < 32 && a2 < st.need && st.need <= a2 + v);
    const int L2 = __ffsll((long long)hit2) - 1;
    if (lane == L2) {
      s_pick[0] = (uint32_t)(lo1 + 31 - lane);
      s_pick[1] = a2;
      s_pick[2] = v;
    }
  }
  lds_barrier();
  const uint32_t bin = s_pick[0];
  st.need -= s_pick[1];
  st.prefix |= bin << sh;
  st.fixed |= dm << sh;
  st.eq_count = s_pick[2];
  st.all_taken = st.eq_count == st.need;
}

__device__ inline int next_pow2_dev(int v) {
  int p = 1;
  while (p < v) p <<= 1;
  return p;
}

// Descending bitonic sort of n (power of two) composites in LDS.
__device__ inline void lds_bitonic_desc(uint64_t* buf, int n) {
  const int tid = threadIdx.x;
  for (int k = 2; k <= n; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int p = tid; p < n / 2; p += kRadixThreads) {
        const int i = 2 * p - (p & (j - 1));
        const int l = i + j;
        const uint64_t a = buf[i], b = buf[l];
        const bool desc = (i & k) == 0;
        if (desc ? (a < b) : (a > b)) { buf[i] = b; buf[l] = a; }
      }
      __syncthreads();
    }
  }
}

// x * 2^48 rounded down, exactly, for x in [0, 1] (0 for NaN or x < 2^-48).
__device__ inline uint64_t fixed48(float x) {
  const uint32_t b = __float_as_uint(x);
  const int e = (int)(b >> 23);                      // biased exponent (x >= 0)
  const uint64_t m = (uint64_t)((b & 0x7FFFFFu) | 0x800000u);  // x = m 2^(e - 150)
  const int sh = e - 102;                            // x 2^48 = m 2^sh, sh <= 25
  if (e == 0 || e > 127) return 0;
  return sh >= 0 ? m << sh : (sh > -24 ? m >> -sh : 0);
}

__device__ inline uint64_t wave_sum_u64(uint64_t v) {
  v += xor_lanes_u64<1>(v);
  v += xor_lanes_u64<2>(v);
  v += xor_lanes_u64<4>(v);
  v += xor_lanes_u64<8>(v);
  v += xor_lanes_u64<16>(v);
  v += xor_lanes_u64<32>(v);
  return v;
}

// Softmax over buf[0..K) (descending) and the coalesced store of one row.
// The normaliser is the same exact fixed-point sum as in order_and_store
// (every exp in [0, 1] rounded down to a multiple of 2^-48, added as
// uint64), so a row gets the same scores whichever path ordered it.
// s_sum needs kRadixThreads / 64 entries.
template <typename IdxT>
__device__ inline void radix_epilogue(const uint64_t* buf, int K, int64_t row, uint64_t* s_sum,
                                      float* scores, IdxT* indices) {
  const int tid = threadIdx.x;
  const float vmax = value_of_key(comp_key(buf[0]));
  uint64_t q = 0;
  bool nan = false;
  for (int r = tid; r < K; r += kRadixThreads) {
    const float ex = expf(value_of_key(comp_key(buf[r])) - vmax);
    q += fixed48(ex);
    nan |= ex != ex;
  }
  q = wave_sum_u64(q);
  if ((tid & (kWave - 1)) == 0) s_sum[tid / kWave] = __ballot(nan) ? ~0ull : q;
  __syncthreads();
  uint64_t total = 0;
  bool any_nan = false;
#pragma unroll
  for (int w = 0; w < kRadixThreads / kWave; ++w) {
    const uint64_t v = s_sum[w];
    any_nan |= v == ~0ull;
    total += v;
  }
  const float sum = any_nan ? __builtin_nanf("") : (float)((double)total * 0x1p-48);
  for (int r = tid; r < K; r += kRadixThreads) {
    const uint64_t w = buf[r];
    store_out(scores, indices, row * K + r, expf(value_of_key(comp_key(w)) - vmax) / sum, comp_idx(w));
  }
}

// 16-byte row loads: VEC elements of T per load.
template <typename T, int VEC> struct VecLoad;
template <typename T> struct VecLoad<T, 1> {
  static __device__ inline void load(const T* p, uint32_t* bits) { bits[0] = Elem<T>::bits(p); }
};
template <> struct VecLoad<float, 4> {
  static __device__ inline void load(const float* p, uint32_t* bits) {
    const uint4 v = *reinterpret_cast<const uint4*>(p);
    bits[0] = v.x; bits[1] = v.y; bits[2] = v.z; bits[3] = v.w;
  }
};
template <> struct VecLoad<uint16_t, 8> {
  static __device__ inline void load(const uint16_t* p, uint32_t* bits) {
    const uint4 v = *reinterpret_cast<const uint4*>(p);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) { bits[2 * i] = w[i] << 16; bits[2 * i + 1] = w[i] & 0xFFFF0000u; }
  }
};
template <> struct VecLoad<Half16, 8> {
  static __device__ inline void load(const Half16* p, uint32_t* bits) {
    const uint4 v = *reinterpret_cast<const uint4*>(p);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      _Float16 lo, hi;
      const uint16_t l16 = (uint16_t)(w[i] & 0xFFFFu), h16 = (uint16_t)(w[i] >> 16);
      __builtin_memcpy(&lo, &l16, 2);
      __builtin_memcpy(&hi, &h16, 2);
      bits[2 * i] = __float_as_uint((float)lo);
      bits[2 * i + 1] = __float_as_uint((float)hi);
    }
  }
};

// ===========================================================================
// 2b. Segment selection, N <= 128 and K <= 16 (e.g. the DeepSeek-V2
//     router shape, 128 experts, top-6).  One 16-lane DPP row per
//     row of the input, so a wave (one workgroup) takes four rows.
//     Lane pos holds columns pos*EPL .. pos*EPL + EPL - 1 (16-byte loads when
//     the rows are full and aligned).  The K-th largest of the 16 lane maxima
//     bounds the row's K-th largest key from below, so the winners are among
//     the few keys at or above it: they are compacted and sorted with a
//     16-lane bitonic network (seg16_topk_filtered), with K rounds of a
//     segment max as the fallback on heavy ties.  Same tie rule and results
//     as topk_select_kernel; no block barrier at all.
// ===========================================================================
constexpr int kSegThreads = 64;  // one wave, four rows: many small workgroups hide the chain's latency

template <typename T, int EPL, typename IdxT, bool VECLOAD>
__global__ __launch_bounds__(kSegThreads) void topk_seg_kernel(const T* __restrict__ logits, int64_t M, int N,
                                                               int64_t ld, int K, float* __restrict__ scores,
                                                               IdxT* __restrict__ indices) {
  __shared__ uint64_t scratch[kSegThreads];  // 16 slots per segment
  const int tid = threadIdx.x, pos = tid & 15;
  const int64_t row = (int64_t)blockIdx.x * (kSegThreads / 16) + tid / 16;
  const bool live = row < M;  // segment-uniform
  const T* x = logits + (live ? row : 0) * ld + pos * EPL;
  uint32_t key[EPL];
  if constexpr (VECLOAD) {
    constexpr int VEC = 16 / sizeof(T);
    static_assert(EPL % VEC == 0, "whole vectors per lane");
#pragma unroll
    for (int j = 0; j < EPL / VEC; ++j) VecLoad<T, VEC>::load(x + j * VEC, key + j * VEC);
#pragma unroll
    for (int i = 0; i < EPL; ++i) key[i] = key_of_bits(key[i]);
  } else {
#pragma unroll
    for (int i = 0; i < EPL; ++i)
      key[i] = (live && pos * EPL + i < N) ? key_of_bits(Elem<T>::bits(x + i)) : 0u;
  }
  uint64_t win = 0;
  if (!seg16_topk_filtered<EPL>(key, K, scratch + (tid & ~15), win, [](int p, int i) { return p * EPL + i; })) {
    // K rounds of a segment max; lane r keeps winner r.
    uint64_t c[EPL];
#pragma unroll
    for (int i = 0; i < EPL; ++i) c[i] = key[i] ? make_comp(key[i], (uint32_t)(pos * EPL + i)) : 0;
    for (int r = 0; r < K; ++r) {
      uint64_t best = c[0];
#pragma unroll
      for (int i = 1; i < EPL; ++i) best = umax64(best, c[i]);
      best = umax64(best, xor_lanes_u64<1>(best));
      best = umax64(best, xor_lanes_u64<2>(best));
      best = umax64(best, xor_lanes_u64<4>(best));
      best = umax64(best, xor_lanes_u64<8>(best));
#pragma unroll
      for (int i = 0; i < EPL; ++i) c[i] = c[i] == best ? 0 : c[i];
      if (r == pos) win = best;
    }
  }
  // Softmax over the K winners (Convention B); lane 0 holds the maximum.
  const float vmax = value_of_key(comp_key(seg16_shfl_u64(win, 0)));
  const float e = pos < K ? expf(value_of_key(comp_key(win)) - vmax) : 0.0f;
  float sum = e;
  sum += xor_lanes_f32<1>(sum);
  sum += xor_lanes_f32<2>(sum);
  sum += xor_lanes_f32<4>(sum);
  sum += xor_lanes_f32<8>(sum);
  if (live && pos < K) store_out(scores, indices, row * K + pos, e / sum, comp_idx(win));
}

// ---------------------------------------------------------------------------
// Pieces shared by the radix kernels.
//
// Selection.  A sample of 1024 keys spread over the whole row gives a lower
// bound L on the K-th largest key: a radix pass over the sample finds the
// bin holding its m-th largest key, m = mu + 4 sigma + 2 with
// mu = 1024 K / N, and L is that bin's lower edge (one more pass narrows
// the bin when it would admit too many candidates).  Every key >= L is a
// candidate.  If the bound admits fewer than K or more than kCandCap
// candidates (a skewed row), exact radix passes over all keys find the
// threshold key T instead and exactly K candidates are taken (keys above T,
// then the lowest-column copies of T).
//
// Ordering.  Candidates are counted into kOrdBuckets buckets of
// (key - base) >> s (base = smallest candidate key), the counts are
// scanned, candidates are scattered bucket by bucket, and a candidate's rank
// is its bucket start plus the number of larger composites in its bucket.
// The thread that ranks a winner (rank < K) also computes its exp and,
// after one block reduction, stores its score and index.  A bucket holding
// more than kBucketFixMax candidates switches to an LDS bitonic sort.
// ---------------------------------------------------------------------------
constexpr int kCandCap = 8192;
constexpr int kOrdPad = 4;  // slack entries after tmp[] for the rank loop's unconditional loads
// Dynamic LDS of the register-row kernels: cand[kCandCap], tmp[kCandCap + kOrdPad].
constexpr size_t kRadixDynLds = (2 * kCandCap + kOrdPad) * sizeof(uint64_t);
constexpr int kOrdBuckets = 2048;
constexpr int kSample = kRadixThreads;

// Lower bound L (>= 1) on the K-th largest key of a row of N keys from one
// sample key per thread.  Deterministic: every workgroup that passes the
// same samples gets the same L.  hist needs kRadixBins entries.
__device__ inline uint32_t sample_bound(uint32_t samp, int K, int N, uint32_t* hist, uint32_t* s_pick) {
  const float mu = (float)kSample * (float)K / (float)N;
  const float sd = sqrtf(mu * (1.0f - (float)K / (float)N));
  const int m_rank = (int)ceilf(mu + 4.0f * sd + 2.0f);
  if (m_rank >= kSample) return 1u;  // no useful bound: every real key
  const int tid = threadIdx.x;
  for (int b = tid; b < kRadixBins; b += kRadixThreads) hist[b] = 0;
  lds_barrier();
  atomicAdd(&hist[samp >> 21], 1u);
  lds_barrier();
  RadixState ss{0u, 0u, (uint32_t)m_rank, 0u, false};
  radix_pick_bin_w0(ss, hist, 21, 0x7FFu, s_pick);
  // Samples at or above the bin's lower edge estimate the candidate count.
  const uint32_t at_or_above = (uint32_t)m_rank - ss.need + ss.eq_count;
  if (!ss.all_taken && (float)at_or_above * ((float)N / kSample) > 0.5f * kCandCap) {
    for (int b = tid; b < kRadixBins; b += kRadixThreads) hist[b] = 0;
    lds_barrier();
    const bool in = (samp & ss.fixed) == ss.prefix;
    if (in) atomicAdd(&hist[(samp >> 10) & 0x7FFu], 1u);
    lds_barrier();
    radix_pick_bin_w0(ss, hist, 10, 0x7FFu, s_pick);
  }
  return max(ss.prefix, 1u);
}

// Clears what order_and_store expects zeroed (the bucket counts and the
// crowding flag).  Callers run it before the barrier that publishes cand[].
__device__ inline void order_prepare(uint32_t* hist, uint32_t* s_flag) {
  for (int b = threadIdx.x; b < kOrdBuckets; b += kRadixThreads) hist[b] = 0;
  if (threadIdx.x == 0) *s_flag = 0;
}

// Orders the C candidates in cand[] (LDS, distinct composites, the K largest
// among them are the row's winners), applies the softmax and stores row
// `row`.  Thread t owns candidates t + 1024 u, u < U (U * 1024 >= C), and
// keeps them, their buckets and their ranks in registers from the first
// step to the last, so every step issues its U LDS accesses together.
// hist[] and *s_flag must be zero (order_prepare) and published by a
// barrier; tmp needs kCandCap + kOrdPad entries, hist and bstart kOrdBuckets + 1.
template <int U, typename IdxT>
__device__ __attribute__((always_inline)) inline void order_and_store_u(uint64_t* cand, int C, uint32_t base, uint32_t rmax, int K,
                                         int64_t row, uint64_t* tmp, uint32_t* hist, uint32_t* bstart,
                                         uint32_t* wsum, uint32_t* s_flag, uint64_t* s_red,
                                         float* scores, IdxT* indices, uint64_t* s_sum64) {
  uint32_t* s_cw = s_flag + 1;  // candidates in the buckets that can win (s_flag[2])
  constexpr int BPT = kOrdBuckets / kRadixThreads;
  const int tid = threadIdx.x, lane = tid & (kWave - 1);
  int sh = 0;
  while (((rmax - base) >> sh) >= (uint32_t)kOrdBuckets) ++sh;
  auto bucket = [&](uint64_t v) { return kOrdBuckets - 1 - (int)((comp_key(v) - base) >> sh); };
  uint64_t v[U];
  int bk[U];
  bool in[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int p = tid + kRadixThreads * u;
    in[u] = p < C;
    v[u] = in[u] ? cand[p] : 0ull;
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    bk[u] = bucket(v[u]);
    if (in[u]) atomicAdd(&hist[bk[u]], 1u);
  }
  __syncthreads();
  {
    uint32_t h[BPT], hs = 0, hmax = 0;
#pragma unroll
    for (int q = 0; q < BPT; ++q) {
      h[q] = hist[tid * BPT + q];
      hs += h[q];
      hmax = max(hmax, h[q]);
    }
    uint32_t run = block_excl_scan_1024(hs, wsum, nullptr);
#pragma unroll
    for (int q = 0; q < BPT; ++q) {
      bstart[tid * BPT + q] = run;
      hist[tid * BPT + q] = run;  // cursor
      // The bucket holding rank K - 1 ends the candidates that can win.
      if (run < (uint32_t)K && (uint32_t)K <= run + h[q]) *s_cw = run + h[q];
      run += h[q];
    }
    if (tid == 0) bstart[kOrdBuckets] = (uint32_t)C;
    if (__ballot(hmax > (uint32_t)kBucketFixMax) && lane == 0) *s_flag = 1;
  }
  __syncthreads();
  if (*s_flag) {
    // Crowded bucket: sort all candidates instead (cand[] is intact).
    const int Cpad = next_pow2_dev(C);
    for (int p = C + tid; p < Cpad; p += kRadixThreads) cand[p] = 0;
    __syncthreads();
    lds_bitonic_desc(cand, Cpad);
    radix_epilogue(cand, K, row, s_red, scores, indices);
    return;
  }
  // Only buckets that start below rank K can hold winners: the others are
  // neither placed nor ranked.
  const int Cw = (int)*s_cw;
#pragma unroll
  for (int u = 0; u < U; ++u)
    if (in[u] && (int)bstart[bk[u]] < K) tmp[atomicAdd(&hist[bk[u]], 1u)] = v[u];
  __syncthreads();
  // Rank = bucket start + larger composites in the bucket (buckets hold at
  // most kBucketFixMax candidates).  Thread t now ranks the candidates at
  // sorted positions t + 1024 u < Cw, so the lanes of a wave share buckets.
  int beg[U], len[U], rk[U], lmax = 0;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    in[u] = tid + kRadixThreads * u < Cw;
    v[u] = in[u] ? tmp[tid + kRadixThreads * u] : 0ull;
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int b = bucket(v[u]);
    beg[u] = in[u] ? (int)bstart[b] : 0;
    len[u] = in[u] ? (int)bstart[b + 1] - beg[u] : 0;
    rk[u] = beg[u];
    lmax = max(lmax, len[u]);
  }
  // Four in-bucket loads per candidate are in flight before any compare;
  // they are unconditional (tmp has kOrdPad entries of slack past kCandCap)
  // so that adjacent pairs issue as one ds_read2_b64, and the compare masks
  // the entries past the bucket.
  for (int j = 0; j < lmax; j += 4) {
    uint64_t t[U][4];
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int q = 0; q < 4; ++q) t[u][q] = tmp[beg[u] + j + q];
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int q = 0; q < 4; ++q) rk[u] += (j + q < len[u]) & (t[u][q] > v[u]);
  }
  // The normaliser is summed exactly, in fixed point, so the scores are
  // bitwise reproducible whatever (atomic) order the candidates reached
  // threads in: every winner's exp lies in [0, 1] and is converted to
  // round-down multiples of 2^-48 (error <= K 2^-48 relative to a sum >= 1)
  // and added as uint64, which is associative.  A NaN exp (a NaN or +inf
  // in the row) makes every score NaN, as in torch.softmax.
  // Each winner's exp and column are staged in cand[] at its rank (cand[] is
  // no longer read), so the row is stored with coalesced writes.
  const float vmax = value_of_key(rmax);
  uint64_t qsum = 0;
  bool nan = false;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    if (in[u] && rk[u] < K) {
      const float ex = expf(value_of_key(comp_key(v[u])) - vmax);
      qsum += fixed48(ex);
      nan |= ex != ex;
      cand[rk[u]] = ((uint64_t)__float_as_uint(ex) << 32) | comp_idx(v[u]);
    }
  }
  qsum = wave_sum_u64(qsum);
  if (lane == 0) s_sum64[tid / kWave] = __ballot(nan) ? ~0ull : qsum;
  __syncthreads();
  uint64_t total = 0;
  bool any_nan = false;
#pragma unroll
  for (int w = 0; w < kRadixThreads / kWave; ++w) {
    const uint64_t q = s_sum64[w];
    any_nan |= q == ~0ull;
    total += q;
  }
  const float sum = any_nan ? __builtin_nanf("") : (float)((double)total * 0x1p-48);
  for (int r = tid; r < K; r += kRadixThreads) {
    const uint64_t e = cand[r];
    store_out(scores, indices, row * K + r, __uint_as_float((uint32_t)(e >> 32)) / sum, (uint32_t)e);
  }
}

template <typename IdxT>
__device__ __attribute__((always_inline)) inline void order_and_store(uint64_t* cand, int C, uint32_t base, uint32_t rmax, int K,
                                       int64_t row, uint64_t* tmp, uint32_t* hist, uint32_t* bstart,
                                       uint32_t* wsum, uint32_t* s_flag, uint64_t* s_red,
                                       float* scores, IdxT* indices, uint64_t* s_sum64) {
  static_assert(kCandCap == 8 * kRadixThreads, "order_and_store covers 8 candidates per thread");
  const int units = (C + kRadixThreads - 1) / kRadixThreads;
#define MOE_ORDER_U(n) \
  order_and_store_u<n, IdxT>(cand, C, base, rmax, K, row, tmp, hist, bstart, wsum, s_flag, s_red, scores, indices, s_sum64)
  if (units <= 1) MOE_ORDER_U(1);
  else if (units == 2) MOE_ORDER_U(2);
  else if (units == 3) MOE_ORDER_U(3);
  else if (units == 4) MOE_ORDER_U(4);
  else if (units <= 6) MOE_ORDER_U(6);
  else MOE_ORDER_U(8);
#undef MOE_ORDER_U
}

// Row slice [c0, end) of thread tid: columns c0 + VEC*(tid + 1024*j) + c,
// j < KPT/VEC, c < VEC.  Loading is split in two so that work needing only
// the row's sample (the bound) runs while these loads are in flight:
// issue_row_loads starts every vector load and touches none of them (vectors
// outside the range read the row start instead, always in bounds, so there
// is no branch between the loads); keys_from_bits later turns the raw bits
// into keys in place, 0 (padding) outside the range.  Keys use the plain
// sign flip; `special` reports NaN or -0.0, for which the caller re-keys
// with key_of_bits.
template <typename T, int VEC, int KPT, bool FULL = false>
__device__ inline void issue_row_loads(const T* __restrict__ x, int c0, int end, uint32_t* bits) {
  constexpr int NV = KPT / VEC;
  const int tid = threadIdx.x;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int c = c0 + VEC * (tid + kRadixThreads * j);
    VecLoad<T, VEC>::load(x + (FULL || c + VEC <= end ? c : 0), bits + j * VEC);
  }
}

template <typename T, int VEC, int KPT, bool FULL = false>
__device__ inline void keys_from_bits(const T* __restrict__ x, int c0, int end, uint32_t* key, bool& special) {
  constexpr int NV = KPT / VEC;
  const int tid = threadIdx.x;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int c = c0 + VEC * (tid + kRadixThreads * j);
#pragma unroll
    for (int i = 0; i < VEC; ++i) {
      const uint32_t b = key[j * VEC + i];
      special |= __builtin_amdgcn_classf(__uint_as_float(b), 0x23);  // NaN or -0
      key[j * VEC + i] = FULL || c + VEC <= end ? key_fast(b) : 0u;
    }
  }
  // A vector straddling `end` (end - c0 not a multiple of VEC).
  if (!FULL && (end - c0) % VEC != 0) {
    const int jt = ((end - c0) / VEC) / kRadixThreads, tt = ((end - c0) / VEC) % kRadixThreads;
    if (tid == tt && jt < NV) {
#pragma unroll
      for (int j = 0; j < NV; ++j)
        if (j == jt)
#pragma unroll
          for (int i = 0; i < VEC; ++i) {
            const int c = c0 + VEC * (tid + kRadixThreads * j) + i;
            if (c < end) {
              const uint32_t b = Elem<T>::bits(x + c);
              special |= __builtin_amdgcn_classf(__uint_as_float(b), 0x23);
              key[j * VEC + i] = key_fast(b);
            }
          }
    }
  }
}

// Column of key slot i of thread tid in a slice starting at c0.
template <int VEC>
__device__ inline uint32_t slot_col(int c0, int i) {
  return (uint32_t)(c0 + VEC * ((int)threadIdx.x + kRadixThreads * (i / VEC)) + (i % VEC));
}

template <int KPT>
__device__ inline void rekey_if_special(uint32_t* key, bool special) {
  // key_fast equals key_of_bits except for NaN and -0.0, so a thread that
  // holds neither keeps its keys: no block-wide decision is needed.
  if (special) {
#pragma unroll
    for (int i = 0; i < KPT; ++i) key[i] = key[i] ? key_of_bits(bits_of_fast_key(key[i])) : 0u;  // 0 = padding
  }
}

// Sample key of thread tid for a row of N columns (exact key; identical in
// every workgroup of the row): 64 runs of 16 consecutive columns, run j
// starting at column floor(j*N/64).  A wave's 64 lanes then touch four
// 64-byte runs (fp32) instead of 64 separate lines, so the sample takes
// little of the CU's load bandwidth while the row loads are in flight
// (C2: 15.15 against 15.43 us per call; runs of 4 gave 15.19).
constexpr int kSampleRun = 16;
template <typename T>
__device__ inline uint32_t sample_key(const T* __restrict__ x, int N) {
  const int j = (int)threadIdx.x / kSampleRun;
  const int c = min(N - 1, (int)(((int64_t)j * N) / (kSample / kSampleRun)) + (int)threadIdx.x % kSampleRun);
  return key_of_bits(Elem<T>::bits(x + c));
}

// Whole-row exact path for one workgroup, re-reading the row from L2 in
// every pass: radix passes find the threshold, then the winners are
// bitonic-sorted in LDS.  sbuf needs Kpad entries.
template <typename T, typename IdxT>
__device__ inline void radix_row_global(const T* __restrict__ x, int64_t N, int K, int Kpad, int64_t row,
                                        uint64_t* sbuf, uint32_t* hist, uint32_t* wsum, uint32_t* s_pick,
                                        uint32_t* s_slot, uint64_t* s_red, float* scores, IdxT* indices) {
  const int tid = threadIdx.x;
  RadixState st{0u, 0u, (uint32_t)K, 0u, false};
  const int shifts[3] = {21, 10, 0};
  const uint32_t dmask[3] = {0x7FFu, 0x7FFu, 0x3FFu};
  for (int pass = 0; pass < 3 && !st.all_taken; ++pass) {
    for (int b = tid; b < kRadixBins; b += kRadixThreads) hist[b] = 0;
    __syncthreads();
    for (int64_t i = tid; i < N; i += kRadixThreads) {
      const uint32_t key = key_of_bits(Elem<T>::bits(x + i));
      if ((key & st.fixed) == st.prefix) atomicAdd(&hist[(key >> shifts[pass]) & dmask[pass]], 1u);
    }
    __syncthreads();
    radix_pick_bin(st, hist, shifts[pass], dmask[pass], wsum, s_pick);
  }
  // Selection rule: key > thr, or key == thr among the first `need` by index.
  // When a whole bin is taken, every key with the decided digits == prefix
  // qualifies: express that as "masked key >= prefix".
  if (tid == 0) *s_slot = 0;
  __syncthreads();
  const bool ties_partial = !st.all_taken && st.eq_count > st.need;
  for (int64_t i = tid; i < N; i += kRadixThreads) {
    const uint32_t key = key_of_bits(Elem<T>::bits(x + i));
    const uint32_t mk = key & st.fixed;
    const bool take = ties_partial ? (mk > st.prefix) : (mk >= st.prefix);
    if (take) {
      const uint32_t s = atomicAdd(s_slot, 1u);
      if (s < (uint32_t)Kpad) sbuf[s] = make_comp(key, (uint32_t)i);
    }
  }
  if (ties_partial) {
    // The threshold key T = prefix occurs eq_count > need times: take the
    // `need` lowest indices.  Thread t scans a contiguous index range so the
    // block prefix sum of per-thread counts orders the copies by index.
    const int64_t chunk = (N + kRadixThreads - 1) / kRadixThreads;
    const int64_t lo = std::min<int64_t>(N, tid * chunk), hi = std::min<int64_t>(N, lo + chunk);
    uint32_t cnt = 0;
    for (int64_t i = lo; i < hi; ++i) cnt += key_of_bits(Elem<T>::bits(x + i)) == st.prefix;
    uint32_t before = block_excl_scan_1024(cnt, wsum, nullptr);
    for (int64_t i = lo; i < hi && before < st.need; ++i) {
      const uint32_t key = key_of_bits(Elem<T>::bits(x + i));
      if (key == st.prefix) {
        const uint32_t s = atomicAdd(s_slot, 1u);
        if (s < (uint32_t)Kpad) sbuf[s] = make_comp(key, (uint32_t)i);
        ++before;
      }
    }
  }
  __syncthreads();
  for (int i = K + tid; i < Kpad; i += kRadixThreads) sbuf[i] = 0;
  __syncthreads();
  lds_bitonic_desc(sbuf, Kpad);
  radix_epilogue(sbuf, K, row, s_red, scores, indices);
}

// ===========================================================================
// 3a. One workgroup per row, row in VGPRs (N <= 32K with 16-byte rows).
//     Thread t holds KPT keys: vector j covers columns VEC*(t + 1024*j) ..
//     +VEC-1, so column order is (j, t, c).  Candidate extraction: each
//     thread marks its candidate slots in a bitmask, a block prefix sum of
//     the popcounts gives every candidate its LDS slot, and the extraction
//     loop runs only as many times as the wave's largest popcount, re-reading
//     each candidate's column from L2 (the row was just read) instead of
//     indexing the VGPR array dynamically.
// ===========================================================================
template <typename T, typename IdxT, int VEC, int KPT, bool FULL>
__global__ __launch_bounds__(kRadixThreads) void topk_radix_reg_kernel(
    const T* __restrict__ logits, int64_t M, int N, int64_t ld, int K, int Kpad,
    float* __restrict__ scores, IdxT* __restrict__ indices) {
  static_assert(KPT <= 32, "candidate bitmask is 32 bits");
  constexpr int NV = KPT / VEC;
  extern __shared__ uint64_t dyn[];
  uint64_t* cand = dyn;              // [kCandCap] in extraction order
  uint64_t* tmp = dyn + kCandCap;    // [kCandCap + kOrdPad] grouped by bucket
  __shared__ __align__(16) uint32_t hist[kRadixBins + 1];
  __shared__ uint32_t bstart[kOrdBuckets + 1];
  __shared__ uint32_t wsum[kRadixThreads / kWave];
  __shared__ uint32_t s_pick[3];
  __shared__ uint32_t s_max, s_flag[2];  // crowding flag, winner-bucket count
  __shared__ uint64_t s_sum64[kRadixThreads / kWave];
  __shared__ uint64_t s_red[kRadixThreads / kWave];

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int64_t row = blockIdx.x;
  const T* x = logits + row * ld;

  // The sample load goes first so that the bound waits for it alone while
  // the row loads are still in flight.
  const uint32_t samp = sample_key(x, N);
  uint32_t key[KPT];
  issue_row_loads<T, VEC, KPT, FULL>(x, 0, N, key);
  if (tid == 0) s_max = 0;
  const uint32_t L = sample_bound(samp, K, N, hist, s_pick);  // has barriers
  bool special = false;
  keys_from_bits<T, VEC, KPT, FULL>(x, 0, N, key, special);
  rekey_if_special<KPT>(key, special);
  uint32_t kmax = 0;
#pragma unroll
  for (int i = 0; i < KPT; ++i) kmax = max(kmax, key[i]);
  kmax = wave_max_u32(kmax);
  if (lane == 0) atomicMax(&s_max, kmax);

  // ---- candidate count: keys >= L, else exact mode (which builds a mask) ----
  uint32_t mask = 0, own = 0;
#pragma unroll
  for (int i = 0; i < KPT; ++i) own += key[i] >= L;
  uint32_t C;
  uint32_t cpos = block_excl_scan_1024(own, wsum, &C);
  uint32_t base = L;
  const bool exact = C < (uint32_t)K || C > (uint32_t)kCandCap;  // workgroup-uniform
  if (exact) {
    // Exact threshold: radix passes over every key.  This rare path
    // re-reads the row from L2 one vector at a time so that it adds no
    // register pressure to the common path.
    auto load_vec = [&](int j, uint32_t* kv) {
      const int c0 = VEC * (tid + kRadixThreads * j);
      uint32_t bits[VEC];
      if (c0 + VEC <= N) {
        VecLoad<T, VEC>::load(x + c0, bits);
#pragma unroll
        for (int c = 0; c < VEC; ++c) kv[c] = key_of_bits(bits[c]);
      } else {
#pragma unroll
        for (int c = 0; c < VEC; ++c) kv[c] = (c0 + c < N) ? key_of_bits(Elem<T>::bits(x + c0 + c)) : 0u;
      }
    };
    RadixState st{0u, 0u, (uint32_t)K, 0u, false};
    for (int p = 0; p < 3 && !st.all_taken; ++p) {
      const int shp = p == 0 ? 21 : (p == 1 ? 10 : 0);
      const uint32_t dmp = p == 2 ? 0x3FFu : 0x7FFu;
      for (int b = tid; b < kRadixBins; b += kRadixThreads) hist[b] = 0;
      __syncthreads();
      for (int j = 0; j < NV; ++j) {
        uint32_t kv[VEC];
        load_vec(j, kv);
#pragma unroll
        for (int c = 0; c < VEC; ++c)
          if (kv[c] && (kv[c] & st.fixed) == st.prefix) atomicAdd(&hist[(kv[c] >> shp) & dmp], 1u);
      }
      __syncthreads();
      radix_pick_bin_w0(st, hist, shp, dmp, s_pick);
    }
    const bool ties_partial = !st.all_taken && st.eq_count > st.need;
    mask = 0;
    uint32_t before = 0;  // copies of T taken in earlier columns (j, t, c)
    for (int j = 0; j < NV; ++j) {
      uint32_t kv[VEC];
      load_vec(j, kv);
      uint32_t e = 0;
#pragma unroll
      for (int c = 0; c < VEC; ++c) {
        const bool above = ties_partial ? (kv[c] > st.prefix)
                                        : (kv[c] != 0u && (kv[c] & st.fixed) >= st.prefix);
        mask |= (uint32_t)above << (j * VEC + c);
        e += ties_partial && kv[c] == st.prefix;
      }
      if (ties_partial) {
        uint32_t etot;
        uint32_t r = before + block_excl_scan_1024(e, wsum, &etot);
#pragma unroll
        for (int c = 0; c < VEC; ++c) {
          if (kv[c] == st.prefix) {
            if (r < st.need) mask |= 1u << (j * VEC + c);
            ++r;
          }
        }
        before += etot;
      }
    }
    cpos = block_excl_scan_1024((uint32_t)__popc(mask), wsum, &C);  // C == K
    base = st.prefix;
  }
  const uint32_t rmax = s_max;  // complete: the scans above hold barriers

  // ---- extraction from the key registers (fully unrolled, no indexing) ----
  // On the common path a slot is a candidate exactly when its key is at
  // least L, so the test is the compare itself rather than a bit of the
  // mask, and the slot is written through a running LDS pointer.
  uint64_t* cp = cand + cpos;
  if (!exact) {
    // An opaque copy of L, so that the compiler recomputes each compare (one
    // VALU op) instead of keeping the 32 compare masks of the candidate count
    // alive in scalar registers, which spill.
    uint32_t Lx;
    asm volatile("s_mov_b32 %0, %1" : "=s"(Lx) : "s"(L));
#pragma unroll
    for (int i = 0; i < KPT; ++i)
      if (key[i] >= Lx) *cp++ = make_comp(key[i], slot_col<VEC>(0, i));
  } else {
#pragma unroll
    for (int i = 0; i < KPT; ++i)
      if ((mask >> i) & 1u) *cp++ = make_comp(key[i], slot_col<VEC>(0, i));
  }
  order_prepare(hist, s_flag);
  __syncthreads();
  order_and_store(cand, (int)C, base, rmax, K, row, tmp, hist, bstart, wsum, s_flag, s_red, scores, indices,
                  s_sum64);
}

// ===========================================================================
// 3b. G workgroups per row (few rows, long rows: e.g. 64 rows of 32K).
//     Workgroup g loads columns [g*slice, (g+1)*slice) into VGPRs.  All G
//     workgroups compute the same bound L from the same row-wide sample,
//     compact their candidates (keys >= L) into the row's global candidate
//     buffer (one atomic per workgroup reserves the space) and publish their
//     slice maximum.  The last workgroup to finish (agent-scope release /
//     exchange through agent-scope atomic stores and loads and a per-row
//     counter; no workgroup waits for another)
//     orders the candidates, applies the softmax, stores the row and resets
//     the row's counters to zero for the next call.  If the bound admitted
//     fewer than K or more than kCandCap candidates, that last workgroup runs
//     the exact whole-row path instead.
//     The G workgroups of a row are numbered so that they land on one XCD
//     (workgroup b runs on XCD b % 8), which keeps the row's slices in one
//     L2 for the last workgroup's re-reads; correctness does not depend on it.
// ===========================================================================
struct SplitRowCtl {
  uint32_t count;   // candidates published
  uint32_t done;    // workgroups finished
  uint32_t rmax;    // row maximum key
  uint32_t pad;
};

template <typename T, typename IdxT, int VEC, int KPT>
__global__ __launch_bounds__(kRadixThreads) void topk_radix_split_kernel(
    const T* __restrict__ logits, int64_t M, int N, int64_t ld, int K, int Kpad, int G, int slice,
    float* __restrict__ scores, IdxT* __restrict__ indices, SplitRowCtl* __restrict__ ctl,
    uint64_t* __restrict__ gcand) {
  static_assert(KPT <= 32, "candidate bitmask is 32 bits");
  extern __shared__ uint64_t dyn[];
  uint64_t* cand = dyn;              // [kCandCap]
  uint64_t* tmp = dyn + kCandCap;    // [kCandCap + kOrdPad]
  __shared__ __align__(16) uint32_t hist[kRadixBins + 1];
  __shared__ uint32_t bstart[kOrdBuckets + 1];
  __shared__ uint32_t wsum[kRadixThreads / kWave];
  __shared__ uint32_t s_pick[3];
  __shared__ uint32_t s_max, s_base, s_last, s_flag[2];  // s_flag: crowding flag, winner-bucket count
  __shared__ uint64_t s_sum64[kRadixThreads / kWave];
  __shared__ uint64_t s_red[kRadixThreads / kWave];

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int q = blockIdx.x >> 3;
  const int g = q % G;
  const int64_t row = (int64_t)(q / G) * 8 + (blockIdx.x & 7);
  if (row >= M) return;  // whole workgroup
  const T* x = logits + row * ld;
  SplitRowCtl* rc = ctl + row;
  uint64_t* rcand = gcand + row * kCandCap;
  const int c0 = g * slice;
  const int end = min(N, c0 + slice);

  const uint32_t samp = sample_key(x, N);
  uint32_t key[KPT];
  issue_row_loads<T, VEC, KPT>(x, c0, end, key);
  if (tid == 0) s_max = 0;
  const uint32_t L = sample_bound(samp, K, N, hist, s_pick);  // has barriers
  bool special = false;
  keys_from_bits<T, VEC, KPT>(x, c0, end, key, special);
  rekey_if_special<KPT>(key, special);
  uint32_t kmax = 0;
#pragma unroll
  for (int i = 0; i < KPT; ++i) kmax = max(kmax, key[i]);
  kmax = wave_max_u32(kmax);
  if (lane == 0) atomicMax(&s_max, kmax);

  uint32_t mask = 0;
#pragma unroll
  for (int i = 0; i < KPT; ++i) mask |= (uint32_t)(key[i] >= L) << i;
  uint32_t cnt;
  uint32_t cpos = block_excl_scan_1024((uint32_t)__popc(mask), wsum, &cnt);
  if (tid == 0) {
    s_base = atomicAdd(&rc->count, cnt);
    atomicMax(&rc->rmax, s_max);
  }
  __syncthreads();
  cpos += s_base;
#pragma unroll
  for (int i = 0; i < KPT; ++i) {
    if ((mask >> i) & 1u) {
      if (cpos < (uint32_t)kCandCap)
        __hip_atomic_store(rcand + cpos, make_comp(key[i], slot_col<VEC>(c0, i)), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
      ++cpos;
    }
  }
  // Publish, then count in.  The candidates went out as agent-scope atomic
  // stores, which write through the XCD's L2, so waiting for this
  // workgroup's stores to complete is the whole release: no L2 writeback
  // (an agent-scope release fence writes back the entire L2 of the XCD,
  // which costs tens of microseconds when every workgroup issues one).
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (tid == 0) s_last = __hip_atomic_fetch_add(&rc->done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (uint32_t)(G - 1);
  __syncthreads();
  if (!s_last) return;

  // ---- last workgroup of the row ----
  const uint32_t C = __hip_atomic_load(&rc->count, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const uint32_t rmax = __hip_atomic_load(&rc->rmax, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  if (tid == 0) {  // leave the row's counters zeroed for the next call
    __hip_atomic_store(&rc->count, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(&rc->done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(&rc->rmax, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (C < (uint32_t)K || C > (uint32_t)kCandCap) {
    radix_row_global<T, IdxT>(x, N, K, Kpad, row, cand, hist, wsum, s_pick, s_flag, s_red, scores, indices);
    return;
  }
  // Agent-scope atomic loads read past this XCD's L2 copy, so they see every
  // workgroup's candidates.
  for (uint32_t p = tid; p < C; p += kRadixThreads)
    cand[p] = __hip_atomic_load(rcand + p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  order_prepare(hist, s_flag);
  __syncthreads();
  order_and_store(cand, (int)C, L, rmax, K, row, tmp, hist, bstart, wsum, s_flag, s_red, scores, indices,
                  s_sum64);
}

// ===========================================================================
// 3c. Any N: one workgroup per row re-reads the row from L2 in every pass.
// ===========================================================================
template <typename T, typename IdxT>
__global__ __launch_bounds__(kRadixThreads) void topk_radix_kernel(
    const T* __restrict__ logits, int64_t M, int64_t N, int64_t ld, int K, int Kpad,
    float* __restrict__ scores, IdxT* __restrict__ indices) {
  extern __shared__ uint64_t sbuf[];  // [Kpad] winner composites
  __shared__ __align__(16) uint32_t hist[kRadixBins];
  __shared__ uint32_t wsum[kRadixThreads / kWave];
  __shared__ uint32_t s_pick[2], s_slot;
  __shared__ uint64_t s_red[kRadixThreads / kWave];
  const int64_t row = blockIdx.x;
  radix_row_global<T, IdxT>(logits + row * ld, N, K, Kpad, row, sbuf, hist, wsum, s_pick, &s_slot, s_red,
                            scores, indices);
}

// ===========================================================================
// Host launchers.
// ===========================================================================
constexpr int kBitonicMaxN = 64;
constexpr int kSelectMaxN = 1024;
constexpr int kRadixMaxK = 16384;

static int next_pow2(int64_t v) {
  int p = 1;
  while (p < v) p <<= 1;
  return p;
}

template <typename T, typename IdxT, int S>
static void launch_bitonic_s(const T* x, int64_t M, int N, int64_t ld, int K, float* s, IdxT* id,
                             hipStream_t st) {
  const int rows_per_block = (256 / kWave) * (kWave / S);
  const int64_t grid = (M + rows_per_block - 1) / rows_per_block;
  topk_bitonic_kernel<T, S, IdxT><<<dim3((unsigned)grid), dim3(256), 0, st>>>(x, M, N, ld, K, s, id);
}

template <typename T, typename IdxT>
static int launch_bitonic(const T* x, int64_t M, int N, int64_t ld, int K, float* s, IdxT* id,
                          hipStream_t st) {
  switch (next_pow2(N)) {
    case 1: launch_bitonic_s<T, IdxT, 1>(x, M, N, ld, K, s, id, st); break;
    case 2: launch_bitonic_s<T, IdxT, 2>(x, M, N, ld, K, s, id, st); break;
    case 4: launch_bitonic_s<T, IdxT, 4>(x, M, N, ld, K, s, id, st); break;
    case 8: launch_bitonic_s<T, IdxT, 8>(x, M, N, ld, K, s, id, st); break;
    case 16: launch_bitonic_s<T, IdxT, 16>(x, M, N, ld, K, s, id, st); break;
    case 32: launch_bitonic_s<T, IdxT, 32>(x, M, N, ld, K, s, id, st); break;
    case 64: launch_bitonic_s<T, IdxT, 64>(x, M, N, ld, K, s, id, st); break;
    default: return fail(MOE_EUNSUP, "bitonic router supports N <= 64");
  }
  return check_launch("topk_bitonic_kernel");
}

template <typename T, typename IdxT, int EPL>
static void launch_select_e(const T* x, int64_t M, int N, int64_t ld, int K, float* s, IdxT* id,
                            hipStream_t st) {
  const int waves = 4;
  const int64_t grid = (M + waves - 1) / waves;
  const size_t lds = (size_t)waves * K * sizeof(uint64_t);
  topk_select_kernel<T, EPL, IdxT><<<dim3((unsigned)grid), dim3(waves * kWave), lds, st>>>(
      x, M, N, ld, K, s, id);
}

template <typename IdxT, int EPL>
static void launch_select_psum_e(const float* part, int G, int64_t M, int N, int K, bool all, float* s, IdxT* id,
                                 hipStream_t st) {
  const int waves = 4;
  const int64_t grid = (M + waves - 1) / waves;
  const size_t lds = (size_t)waves * K * sizeof(uint64_t);
  topk_select_kernel<float, EPL, IdxT, true><<<dim3((unsigned)grid), dim3(waves * kWave), lds, st>>>(
      part, M, N, N, K, s, id, G, M * N, all);
}

template <typename IdxT>
static int launch_select_psum(const float* part, int G, int64_t M, int N, int K, bool all, float* s, IdxT* id,
                              hipStream_t st) {
  const int epl = (N + kWave - 1) / kWave;
  if (epl <= 1) launch_select_psum_e<IdxT, 1>(part, G, M, N, K, all, s, id, st);
  else if (epl <= 2) launch_select_psum_e<IdxT, 2>(part, G, M, N, K, all, s, id, st);
  else if (epl <= 4) launch_select_psum_e<IdxT, 4>(part, G, M, N, K, all, s, id, st);
  else return fail(MOE_EUNSUP, "partial-sum selection supports N <= 256");
  return check_launch("topk_select_kernel");
}

int topk_select_partials(const float* part, int G, int64_t M, int N, int K, int score_mode, float* scores,
                         void* indices, int idx_dtype, hipStream_t st) {
  if (M == 0) return MOE_OK;
  if (K > N || G < 1) return fail(MOE_EINVAL, "topk_select_partials: need K <= N and G >= 1");
  const bool all = score_mode == MOE_SCORES_ALL;
  if (idx_dtype == MOE_I64)
    return launch_select_psum(part, G, M, N, K, all, scores, static_cast<int64_t*>(indices), st);
  return launch_select_psum(part, G, M, N, K, all, scores, static_cast<int32_t*>(indices), st);
}

template <typename T, typename IdxT, int EPL>
static int launch_seg_e(const T* x, int64_t M, int N, int64_t ld, int K, float* s, IdxT* id, hipStream_t st) {
  constexpr int VEC = 16 / sizeof(T);
  const bool vec = EPL % VEC == 0 && N == 16 * EPL && ((uintptr_t)x % 16) == 0 &&
                   ((ld * (int64_t)sizeof(T)) % 16) == 0;
  constexpr int RPB = kSegThreads / 16;  // rows per workgroup
  const unsigned grid = (unsigned)((M + RPB - 1) / RPB);
  if constexpr (EPL % VEC == 0) {
    if (vec) {
      topk_seg_kernel<T, EPL, IdxT, true><<<grid, kSegThreads, 0, st>>>(x, M, N, ld, K, s, id);
      return check_launch("topk_seg_kernel");
    }
  }
  topk_seg_kernel<T, EPL, IdxT, false><<<grid, kSegThreads, 0, st>>>(x, M, N, ld, K, s, id);
  return check_launch("topk_seg_kernel");
}

template <typename IdxT, int EPL>
static void launch_select16_e(const uint16_t* x, int64_t M, int N, int64_t ld, int K, float* s, IdxT* id,
                              hipStream_t st) {
  const int waves = 4;
  const int64_t grid = (M + waves - 1) / waves;
  if constexpr (EPL % 4 == 0) {
    if (N % 4 == 0 && ld % 4 == 0 && ((uintptr_t)x & 7) == 0) {
      topk_select16_kernel<EPL, IdxT, true><<<dim3((unsigned)grid), dim3(waves * kWave), (size_t)waves * K * 4, st>>>(
          x, M, N, ld, K, s, id);
      return;
    }
  }
  topk_select16_kernel<EPL, IdxT><<<dim3((unsigned)grid), dim3(waves * kWave), (size_t)waves * K * 4, st>>>(
      x, M, N, ld, K, s, id);
}

template <typename T, typename IdxT>
static int launch_select(const T* x, int64_t M, int N, int64_t ld, int K, float* s, IdxT* id,
                         hipStream_t st) {
  // Rows of up to 128 with K <= 16 take the segment kernel (measured: fp32
  // [320,128] K=6 2.9 us against 3.9 us); at N = 256 (16 keys per lane)
  // the one-wave-per-row kernel below is as fast or faster.
  if (K <= 16 && N <= 128 && M <= (int64_t)INT32_MAX) {
    if (N <= 64) return launch_seg_e<T, IdxT, 4>(x, M, N, ld, K, s, id, st);
    return launch_seg_e<T, IdxT, 8>(x, M, N, ld, K, s, id, st);
  }
  if constexpr (std::is_same<T, uint16_t>::value) {  // bfloat16: 32-bit composites
    const int epl = (N + kWave - 1) / kWave;
    if (epl <= 1) launch_select16_e<IdxT, 1>(x, M, N, ld, K, s, id, st);
    else if (epl <= 2) launch_select16_e<IdxT, 2>(x, M, N, ld, K, s, id, st);
    else if (epl <= 4) launch_select16_e<IdxT, 4>(x, M, N, ld, K, s, id, st);
    else if (epl <= 8) launch_select16_e<IdxT, 8>(x, M, N, ld, K, s, id, st);
    else if (epl <= 16) launch_select16_e<IdxT, 16>(x, M, N, ld, K, s, id, st);
    else return fail(MOE_EUNSUP, "selection router supports N <= 1024");
    return check_launch("topk_select16_kernel");
  }
  const int epl = (N + kWave - 1) / kWave;
  if (epl <= 1) launch_select_e<T, IdxT, 1>(x, M, N, ld, K, s, id, st);
  else if (epl <= 2) launch_select_e<T, IdxT, 2>(x, M, N, ld, K, s, id, st);
  else if (epl <= 4) launch_select_e<T, IdxT, 4>(x, M, N, ld, K, s, id, st);
  else if (epl <= 8) launch_select_e<T, IdxT, 8>(x, M, N, ld, K, s, id, st);
  else if (epl <= 16) launch_select_e<T, IdxT, 16>(x, M, N, ld, K, s, id, st);
  else return fail(MOE_EUNSUP, "selection router supports N <= 1024");
  return check_launch("topk_select_kernel");
}

// ===========================================================================
// 4. Convention-A scores: softmax over the whole row, read at the K winners.
//    Replaces topk_softmax_separate (kernels/topk_softmax_baseline.py:15-36):
//    scores = softmax(logits) then topk.  The winners (and their order) are
//    those of the top-K kernels; this pass rewrites their scores as
//    exp(x[idx] - m) / sum_j exp(x[j] - m) over all N columns, m the row
//    maximum.  One wave per row keeps a running (maximum, sum) per lane over
//    the row, merges the lanes, then rescales.  A row holding a NaN gets NaN
//    scores (as torch.softmax).
// ===========================================================================
template <typename T, typename IdxT>
__global__ __launch_bounds__(256) void topk_scores_all_kernel(const T* __restrict__ logits, int64_t M, int N,
                                                              int64_t ld, int K, float* __restrict__ scores,
                                                              const IdxT* __restrict__ indices) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t row = (int64_t)blockIdx.x * (blockDim.x / kWave) + threadIdx.x / kWave;
  if (row >= M) return;  // wave-uniform
  const T* x = logits + row * ld;
  float m = -__builtin_inff(), sum = 0.0f;
  bool nan = false;
  for (int c = lane; c < N; c += kWave) {
    const float v = __uint_as_float(Elem<T>::bits(x + c));
    nan |= v != v;
    if (v > m) {
      sum = sum * expf(m - v) + 1.0f;
      m = v;
    } else {
      sum += expf(v - m);
    }
  }
  // Merge the lanes' (m, sum); lanes that saw only -inf carry sum 0 at -inf.
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const float m2 = xor_lanes_f32(m, o), s2 = xor_lanes_f32(sum, o);
    const float mm = fmaxf(m, m2);
    sum = (m == -__builtin_inff() ? 0.0f : sum * expf(m - mm)) + (m2 == -__builtin_inff() ? 0.0f : s2 * expf(m2 - mm));
    m = mm;
  }
  nan = __ballot(nan) != 0;
  for (int j = lane; j < K; j += kWave) {
    const float v = __uint_as_float(Elem<T>::bits(x + (int64_t)indices[row * K + j]));
    scores[row * K + j] = nan ? __builtin_nanf("") : expf(v - m) / sum;
  }
}

template <typename T, typename IdxT>
static int launch_scores_all(const void* logits, int64_t M, int64_t N, int64_t ld, int64_t K, float* s,
                             const void* idx, hipStream_t st) {
  const int64_t grid = (M + 3) / 4;
  topk_scores_all_kernel<T, IdxT><<<dim3((unsigned)grid), 256, 0, st>>>(
      static_cast<const T*>(logits), M, (int)N, ld, (int)K, s, static_cast<const IdxT*>(idx));
  return check_launch("topk_scores_all_kernel");
}

constexpr int kRadixRegMaxK = 8192;

template <typename T, typename IdxT, int VEC, int KPT>
static int launch_radix_reg(const T* x, int64_t M, int N, int64_t ld, int K, float* s, IdxT* id,
                            hipStream_t st) {
  const int Kpad = next_pow2(K);
  // Rows of exactly KPT keys per thread need no range checks.
  auto go = [&](auto full) {
    constexpr bool F = decltype(full)::value;
    static std::atomic<uint64_t> lds_cap_set{0};
    MOE_HIP_CHECK(lds_cap_once(lds_cap_set, (const void*)topk_radix_reg_kernel<T, IdxT, VEC, KPT, F>,
                                (int)(kRadixDynLds), st));
    topk_radix_reg_kernel<T, IdxT, VEC, KPT, F><<<dim3((unsigned)M), dim3(kRadixThreads), kRadixDynLds, st>>>(
        x, M, N, ld, K, Kpad, s, id);
    return check_launch("topk_radix_reg_kernel");
  };
  if (VEC > 1 && N == KPT * kRadixThreads) return go(std::true_type{});
  return go(std::false_type{});
}

constexpr int kRadixRegMaxKPT = 32;  // keys per thread held in VGPRs

template <typename T, typename IdxT, int VEC, int KPT>
static int launch_radix_reg_v(const T* x, int64_t M, int N, int64_t ld, int K, float* s, IdxT* id,
                              hipStream_t st) {
  const int per = (N + kRadixThreads - 1) / kRadixThreads;
  if (per <= KPT) return launch_radix_reg<T, IdxT, VEC, KPT>(x, M, N, ld, K, s, id, st);
  // Unaligned rows (VEC == 1) stop at 16 keys per thread: 32 would spill.
  if constexpr (2 * KPT <= kRadixRegMaxKPT && (VEC > 1 || 2 * KPT <= 16))
    return launch_radix_reg_v<T, IdxT, VEC, 2 * KPT>(x, M, N, ld, K, s, id, st);
  return fail(MOE_EUNSUP, "radix row too long for the register kernel");
}

// Split-row plan: G workgroups per row when rows are few and long, so that
// about one workgroup per CU is busy.  G == 1: no split.
static int num_cus() {
  static int cus = 0;
  if (!cus) {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0)
      cus = n;
    else
      cus = 256;
  }
  return cus;
}

// Rows whose counters fit in the workspace control block.
constexpr int64_t kSplitMaxRows = kWsCtlBytes / sizeof(SplitRowCtl);
constexpr int kSplitMaxG = 64;


// Rows too long for one workgroup's registers are split over G workgroups
// (G a power of two, slice <= 1024 * kRadixRegMaxKPT keys).  Rows that fit
// stay whole: a row is latency-bound, and for them the candidate exchange
// costs about what the shorter slices save.  G grows further (to slices of
// 8192 keys) while the grid stays within one workgroup per CU (each
// workgroup takes 128 KB of LDS).
static int split_groups(int64_t M, int64_t N, int64_t K) {
  if (K > kRadixRegMaxK || M < 1 || M > kSplitMaxRows) return 1;
  const int64_t cap = (int64_t)kRadixThreads * kRadixRegMaxKPT;
  if (N <= cap) return 1;
  int G = 1;
  while ((int64_t)G * cap < N) G *= 2;
  if (G > kSplitMaxG) return 1;
  while (G < kSplitMaxG && N / (2 * G) >= 8192 && M * 2 * G <= (int64_t)num_cus()) G *= 2;
  return G;
}

static size_t split_ws_bytes(int64_t M) {
  return kWsCtlBytes + (size_t)M * kCandCap * sizeof(uint64_t);
}

template <typename T, typename IdxT, int VEC, int KPT>
static int launch_radix_split(const T* x, int64_t M, int N, int64_t ld, int K, int G, int slice, float* s,
                              IdxT* id, void* ws, hipStream_t st) {
  static std::atomic<uint64_t> lds_cap_set{0};
  MOE_HIP_CHECK(lds_cap_once(lds_cap_set, (const void*)topk_radix_split_kernel<T, IdxT, VEC, KPT>,
                              (int)(kRadixDynLds), st));
  SplitRowCtl* ctl = static_cast<SplitRowCtl*>(ws);
  uint64_t* gcand = reinterpret_cast<uint64_t*>(static_cast<char*>(ws) + kWsCtlBytes);
  const int64_t grid = (M + 7) / 8 * 8 * G;
  topk_radix_split_kernel<T, IdxT, VEC, KPT><<<dim3((unsigned)grid), dim3(kRadixThreads),
                                                kRadixDynLds, st>>>(
      x, M, N, ld, K, next_pow2(K), G, slice, s, id, ctl, gcand);
  return check_launch("topk_radix_split_kernel");
}

template <typename T, typename IdxT, int VEC, int KPT>
static int launch_radix_split_v(const T* x, int64_t M, int N, int64_t ld, int K, int G, int slice, float* s,
                                IdxT* id, void* ws, hipStream_t st) {
  if (slice / kRadixThreads <= KPT) return launch_radix_split<T, IdxT, VEC, KPT>(x, M, N, ld, K, G, slice, s, id, ws, st);
  if constexpr (2 * KPT <= kRadixRegMaxKPT)
    return launch_radix_split_v<T, IdxT, VEC, 2 * KPT>(x, M, N, ld, K, G, slice, s, id, ws, st);
  return fail(MOE_EUNSUP, "radix slice too long");
}

template <typename T, typename IdxT>
static int launch_radix(const T* x, int64_t M, int64_t N, int64_t ld, int K, float* s, IdxT* id,
                        void* ws, size_t ws_bytes, hipStream_t st) {
  constexpr int VEC = 16 / sizeof(T);
  const bool vec_ok = ((uintptr_t)x % 16 == 0) && ((ld * (int64_t)sizeof(T)) % 16 == 0);
  const int G = split_groups(M, N, K);
  if (G > 1 && vec_ok && ws && ws_bytes >= split_ws_bytes(M)) {
    const int64_t unit = (int64_t)VEC * kRadixThreads;
    const int64_t slice = ((N + G - 1) / G + unit - 1) / unit * unit;
    if (slice <= (int64_t)kRadixThreads * kRadixRegMaxKPT)
      return launch_radix_split_v<T, IdxT, VEC, VEC>(x, M, (int)N, ld, K, G, (int)slice, s, id, ws, st);
  }
  if (K <= kRadixRegMaxK && N <= (int64_t)kRadixThreads * (vec_ok ? kRadixRegMaxKPT : 16)) {
    if (vec_ok) return launch_radix_reg_v<T, IdxT, VEC, VEC>(x, M, (int)N, ld, K, s, id, st);
    return launch_radix_reg_v<T, IdxT, 1, 1>(x, M, (int)N, ld, K, s, id, st);
  }
  const int Kpad = next_pow2(K);
  const size_t lds = (size_t)Kpad * sizeof(uint64_t);
  static std::atomic<uint64_t> lds_cap_set{0};  // raise the dynamic-LDS cap once per device
  MOE_HIP_CHECK(lds_cap_once(lds_cap_set, (const void*)topk_radix_kernel<T, IdxT>,
                              (int)(kRadixMaxK * sizeof(uint64_t)), st));
  topk_radix_kernel<T, IdxT><<<dim3((unsigned)M), dim3(kRadixThreads), lds, st>>>(x, M, N, ld, K,
                                                                               Kpad, s, id);
  return check_launch("topk_radix_kernel");
}

template <typename T, typename IdxT>
static int dispatch_topk(const void* logits, int64_t M, int64_t N, int64_t ld, int64_t K,
                         float* scores, void* indices, int algo, void* ws, size_t ws_bytes,
                         hipStream_t st) {
  const T* x = static_cast<const T*>(logits);
  IdxT* id = static_cast<IdxT*>(indices);
  switch (algo) {
    case MOE_TOPK_BITONIC: return launch_bitonic<T, IdxT>(x, M, (int)N, ld, (int)K, scores, id, st);
    case MOE_TOPK_SELECTION: return launch_select<T, IdxT>(x, M, (int)N, ld, (int)K, scores, id, st);
    case MOE_TOPK_RADIX: return launch_radix<T, IdxT>(x, M, N, ld, (int)K, scores, id, ws, ws_bytes, st);
    default: return fail(MOE_EINVAL, "unknown top-k algorithm");
  }
}

}  // namespace moe

using namespace moe;

extern "C" int moe_topk_select_algo(int64_t N, int64_t K) {
  (void)K;
  if (N <= kBitonicMaxN) return MOE_TOPK_BITONIC;
  if (N <= 512) return MOE_TOPK_SELECTION;
  return MOE_TOPK_RADIX;
}

extern "C" size_t moe_topk_softmax_workspace_size(int64_t M, int64_t N, int64_t K, int algo) {
  if (M < 1 || N < 1 || K < 1 || K > N) return 0;
  if (algo == MOE_TOPK_AUTO) algo = moe_topk_select_algo(N, K);
  if (algo != MOE_TOPK_RADIX || split_groups(M, N, K) <= 1) return 0;
  return split_ws_bytes(M);
}

extern "C" int moe_topk_softmax(const void* logits, int logits_dtype, int64_t M, int64_t N,
                                int64_t ld, int64_t K, float* scores, void* indices,
                                int idx_dtype, int algo, void* workspace, size_t ws_bytes,
                                void* stream) {
  return moe_topk_softmax_ex(logits, logits_dtype, M, N, ld, K, scores, indices, idx_dtype, algo,
                             MOE_SCORES_TOPK, workspace, ws_bytes, stream);
}

extern "C" int moe_topk_softmax_ex(const void* logits, int logits_dtype, int64_t M, int64_t N,
                                   int64_t ld, int64_t K, float* scores, void* indices,
                                   int idx_dtype, int algo, int score_mode, void* workspace,
                                   size_t ws_bytes, void* stream) {
  if (score_mode != MOE_SCORES_TOPK && score_mode != MOE_SCORES_ALL && score_mode != MOE_SCORES_TOPK_RENORM)
    return fail(MOE_EINVAL, "topk_softmax: unknown score mode");
  if (score_mode == MOE_SCORES_ALL && !scores) return fail(MOE_EINVAL, "topk_softmax: score mode ALL needs scores");
  if (M < 0 || N < 1 || K < 1 || K > N)
    return fail(MOE_EINVAL, "topk_softmax: need M >= 0, N >= 1 and 1 <= K <= N (got M=" +
                                std::to_string(M) + ", N=" + std::to_string(N) +
                                ", K=" + std::to_string(K) + ")");
  if (ld < N) return fail(MOE_EINVAL, "topk_softmax: row stride ld must be >= N");
  if (N > INT32_MAX || M * ld > ((int64_t)1 << 40))
    return fail(MOE_EUNSUP, "topk_softmax: matrix too large");
  if (!indices || (M > 0 && !logits)) return fail(MOE_EINVAL, "topk_softmax: null pointer");
  if (idx_dtype != MOE_I32 && idx_dtype != MOE_I64)
    return fail(MOE_EINVAL, "topk_softmax: indices must be int32 or int64");
  if (algo == MOE_TOPK_AUTO) algo = moe_topk_select_algo(N, K);
  if (algo == MOE_TOPK_BITONIC && N > kBitonicMaxN)
    return fail(MOE_EUNSUP, "topk_softmax: bitonic algorithm supports N <= 64");
  if (algo == MOE_TOPK_SELECTION && N > kSelectMaxN)
    return fail(MOE_EUNSUP, "topk_softmax: selection algorithm supports N <= 1024");
  if (algo == MOE_TOPK_RADIX && K > kRadixMaxK)
    return fail(MOE_EUNSUP, "topk_softmax: radix algorithm supports K <= 16384");
  if (M == 0) return MOE_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool i64 = idx_dtype == MOE_I64;
  int rc;
  switch (logits_dtype) {
    case MOE_F32:
      rc = i64 ? dispatch_topk<float, int64_t>(logits, M, N, ld, K, scores, indices, algo, workspace, ws_bytes, st)
               : dispatch_topk<float, int32_t>(logits, M, N, ld, K, scores, indices, algo, workspace, ws_bytes, st);
      if (rc == MOE_OK && score_mode == MOE_SCORES_ALL)
        rc = i64 ? launch_scores_all<float, int64_t>(logits, M, N, ld, K, scores, indices, st)
                 : launch_scores_all<float, int32_t>(logits, M, N, ld, K, scores, indices, st);
      return rc;
    case MOE_BF16:
      rc = i64 ? dispatch_topk<uint16_t, int64_t>(logits, M, N, ld, K, scores, indices, algo, workspace, ws_bytes, st)
               : dispatch_topk<uint16_t, int32_t>(logits, M, N, ld, K, scores, indices, algo, workspace, ws_bytes, st);
      if (rc == MOE_OK && score_mode == MOE_SCORES_ALL)
        rc = i64 ? launch_scores_all<uint16_t, int64_t>(logits, M, N, ld, K, scores, indices, st)
                 : launch_scores_all<uint16_t, int32_t>(logits, M, N, ld, K, scores, indices, st);
      return rc;
    case MOE_F16:
      rc = i64 ? dispatch_topk<Half16, int64_t>(logits, M, N, ld, K, scores, indices, algo, workspace, ws_bytes, st)
               : dispatch_topk<Half16, int32_t>(logits, M, N, ld, K, scores, indices, algo, workspace, ws_bytes, st);
      if (rc == MOE_OK && score_mode == MOE_SCORES_ALL)
        rc = i64 ? launch_scores_all<Half16, int64_t>(logits, M, N, ld, K, scores, indices, st)
                 : launch_scores_all<Half16, int32_t>(logits, M, N, ld, K, scores, indices, st);
      return rc;
    default:
      return fail(MOE_EINVAL, "topk_softmax: logits must be float32, bfloat16 or float16");
  }
}
