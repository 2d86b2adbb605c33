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
template <typename T, int EPL, typename IdxT>
__global__ __launch_bounds__(256) void topk_select_kernel(const T* __restrict__ logits,
                                                          int64_t M, int N, int64_t ld,
                                                          int K, float* __restrict__ scores,
                                                          IdxT* __restrict__ indices) {
  extern __shared__ uint64_t win_all[];  // [waves][K]
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int64_t row = (int64_t)blockIdx.x * (blockDim.x / kWave) + wave;
  const bool live = row < M;  // wave-uniform
  uint64_t* win = win_all + (size_t)wave * K;
  const T* x = logits + (live ? row : 0) * ld;

  uint64_t c[EPL];
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    const int idx = lane + kWave * i;
    c[i] = (live && idx < N) ? make_comp(key_of_bits(Elem<T>::bits(x + idx)), idx) : 0;
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
constexpr int kBuckets = 4096;
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
// holding the need-th largest.
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
  __syncthreads();
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

// Softmax over buf[0..K) (descending) and the coalesced store of one row.
template <typename IdxT>
__device__ inline void radix_epilogue(const uint64_t* buf, int K, int64_t row, float* s_red,
                                      float* scores, IdxT* indices) {
  const int tid = threadIdx.x;
  const float vmax = value_of_key(comp_key(buf[0]));
  float part = 0.0f;
  for (int r = tid; r < K; r += kRadixThreads) part += expf(value_of_key(comp_key(buf[r])) - vmax);
  part = wave_sum_f32(part);
  if ((tid & (kWave - 1)) == 0) s_red[tid / kWave] = part;
  __syncthreads();
  float sum = 0.0f;
#pragma unroll
  for (int w = 0; w < kRadixThreads / kWave; ++w) sum += s_red[w];
  for (int r = tid; r < K; r += kRadixThreads) {
    const uint64_t w = buf[r];
    store_out(scores, indices, row * K + r, expf(value_of_key(comp_key(w)) - vmax) / sum,
              comp_idx(w));
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

// Row in VGPRs.  Thread t holds KPT keys: vector j (j < KPT/VEC) covers
// columns VEC*(t + 1024*j) .. +VEC-1, so column order is (j, t, c).
//
// Selection.  A sample of one key per thread, spread over the whole row,
// gives a lower bound L on the K-th largest key: two radix passes over the
// sample find the bin of its m-th largest key, m = mu + 4 sigma + 2 with
// mu = 1024 K / N, and L is that bin's lower edge.  Every key >= L is a
// candidate.  If that yields fewer than K or more than kCandCap candidates
// (a skewed row), the exact radix passes over all keys find the threshold
// key T and the candidates become exactly the K winners (keys above T plus
// the lowest-column copies of T).
//
// Extraction.  Each thread marks its candidate slots in a bitmask; a block
// prefix sum of the popcounts gives every candidate its LDS slot, and the
// extraction loop runs only as many times as the wave's largest popcount,
// re-reading each candidate's column from L2 (the row was just read) rather
// than indexing the VGPR array dynamically.  The same loop counts the
// candidates into kOrdBuckets buckets of (key - base) >> s.
//
// Ordering.  Bucket counts are scanned, candidates are scattered bucket by
// bucket, and each candidate's rank is its bucket start plus the number of
// larger composites in its bucket.  The thread that ranks a winner (rank <
// K) also computes its exp and, after one block reduction, stores its score
// and index.  A bucket holding more than kBucketFixMax candidates switches
// the row to an LDS bitonic sort.
constexpr int kCandCap = 8192;
constexpr int kOrdBuckets = 2048;
constexpr int kSample = kRadixThreads;

// Histogram insert with one LDS atomic per distinct bin per wave: lanes
// holding the same bin are found by intersecting the ballots of its bits.
__device__ inline void wave_aggregated_add(uint32_t* hist, uint32_t bin, bool valid, int nbits) {
  uint64_t match = __ballot(valid);
  for (int b = 0; b < nbits; ++b) {
    const uint64_t bal = __ballot((bin >> b) & 1u);
    match &= ((bin >> b) & 1u) ? bal : ~bal;
  }
  const uint32_t lane = __lane_id();
  if (valid && (uint32_t)(__ffsll((long long)match) - 1) == lane) atomicAdd(&hist[bin], (uint32_t)__popcll(match));
}

template <typename T, typename IdxT, int VEC, int KPT>
__global__ __launch_bounds__(kRadixThreads) void topk_radix_reg_kernel(
    const T* __restrict__ logits, int64_t M, int N, int64_t ld, int K, int Kpad,
    float* __restrict__ scores, IdxT* __restrict__ indices) {
  static_assert(KPT <= 32, "candidate bitmask is 32 bits");
  constexpr int NV = KPT / VEC;
  constexpr int CPT = kCandCap / kRadixThreads;  // candidates per thread, max
  extern __shared__ uint64_t dyn[];
  uint64_t* cand = dyn;              // [kCandCap] in extraction order
  uint64_t* tmp = dyn + kCandCap;    // [kCandCap] grouped by bucket
  __shared__ uint32_t hist[kRadixBins];  // radix digits; bucket counts and cursors
  __shared__ uint32_t bstart[kOrdBuckets + 1];
  __shared__ uint32_t wsum[kRadixThreads / kWave];
  __shared__ uint32_t s_pick[3];
  __shared__ uint32_t s_max, s_hmax;
  __shared__ float s_red[kRadixThreads / kWave];
  static_assert(kOrdBuckets <= kRadixBins, "bucket counts live in hist[]");

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int64_t row = blockIdx.x;
  const T* x = logits + row * ld;

  MOE_PHASE(0);
  // ---- load the row once; key 0 marks columns past N ----
  // Keys are first formed with the plain sign flip; rows holding a NaN or a
  // -0.0 (flagged by v_cmp_class) are re-keyed with key_of_bits below.
  uint32_t key[KPT];
  bool special = false;
  {
    // All vector loads are issued before any is used: out-of-row vectors
    // read the row's first vector instead (always in bounds) and are
    // discarded, so there is no branch, and no wait, between the loads.
    uint32_t bits[KPT];
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int c0 = VEC * (tid + kRadixThreads * j);
      VecLoad<T, VEC>::load(x + (c0 + VEC <= N ? c0 : 0), bits + j * VEC);
    }
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int c0 = VEC * (tid + kRadixThreads * j);
#pragma unroll
      for (int c = 0; c < VEC; ++c) {
        const uint32_t b = bits[j * VEC + c];
        special |= __builtin_amdgcn_classf(__uint_as_float(b), 0x23);  // NaN or -0
        key[j * VEC + c] = c0 + VEC <= N ? key_fast(b) : 0u;
      }
    }
    // A vector straddling the row end (N not a multiple of VEC).
    const int jt = (N / VEC) / kRadixThreads, tt = (N / VEC) % kRadixThreads;
    if (N % VEC != 0 && tid == tt && jt < NV) {
#pragma unroll
      for (int j = 0; j < NV; ++j)
        if (j == jt)
#pragma unroll
          for (int c = 0; c < VEC; ++c)
            if (VEC * (tid + kRadixThreads * j) + c < N) {
              const uint32_t b = Elem<T>::bits(x + VEC * (tid + kRadixThreads * j) + c);
              special |= __builtin_amdgcn_classf(__uint_as_float(b), 0x23);
              key[j * VEC + c] = key_fast(b);
            }
    }
  }
  MOE_PHASE(1);

  // ---- row maximum; sample bound L ----
  if (__syncthreads_or(special)) {
#pragma unroll
    for (int i = 0; i < KPT; ++i) key[i] = key[i] ? key_of_bits(bits_of_fast_key(key[i])) : 0u;  // 0 = padding
  }
  uint32_t kmax = 0;
#pragma unroll
  for (int i = 0; i < KPT; ++i) kmax = max(kmax, key[i]);
  kmax = wave_max_u32(kmax);
  // Sample key: slot q, one per wave (wave-uniform, so a scalar branch),
  // spread so that the 16 waves cover every vector j.
  uint32_t samp = 0;
  {
    const int q = __builtin_amdgcn_readfirstlane((tid / kWave) * KPT / (kRadixThreads / kWave));
#pragma unroll
    for (int i = 0; i < KPT; ++i)
      if (q == i) samp = key[i];
  }
  if (tid == 0) s_max = 0;
  for (int b = tid; b < kRadixBins; b += kRadixThreads) hist[b] = 0;
  __syncthreads();
  if (lane == 0) atomicMax(&s_max, kmax);
  const float mu = (float)kSample * (float)K / (float)N;
  const float sd = sqrtf(mu * (1.0f - (float)K / (float)N));
  const int m_rank = (int)ceilf(mu + 4.0f * sd + 2.0f);
  uint32_t L = 1u;  // 1: every real key (0 is padding)
  if (m_rank < kSample) {
    RadixState ss{0u, 0u, (uint32_t)m_rank, 0u, false};
    wave_aggregated_add(hist, samp >> 21, true, 11);
    __syncthreads();
    radix_pick_bin_w0(ss, hist, 21, 0x7FFu, s_pick);
    MOE_PHASE(2);
    if (!ss.all_taken) {
      for (int b = tid; b < kRadixBins; b += kRadixThreads) hist[b] = 0;
      __syncthreads();
      const bool in = (samp & ss.fixed) == ss.prefix;
      if (__ballot(in)) wave_aggregated_add(hist, (samp >> 10) & 0x7FFu, in, 11);
      __syncthreads();
      radix_pick_bin_w0(ss, hist, 10, 0x7FFu, s_pick);
    }
    L = max(ss.prefix, 1u);  // lower edge of the bin of the m-th largest sample
  }
  MOE_PHASE(3);
  const uint32_t rmax = s_max;

  // ---- candidate mask: sample mode (key >= L), else exact mode ----
  uint32_t mask = 0;
#pragma unroll
  for (int i = 0; i < KPT; ++i) mask |= (uint32_t)(key[i] >= L) << i;
  uint32_t C;
  uint32_t cpos = block_excl_scan_1024((uint32_t)__popc(mask), wsum, &C);
  uint32_t base = L;
  if (C < (uint32_t)K || C > (uint32_t)kCandCap) {
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
  int sh = 0;
  while (((rmax - base) >> sh) >= (uint32_t)kOrdBuckets) ++sh;
  for (int b = tid; b < kOrdBuckets; b += kRadixThreads) hist[b] = 0;
  if (tid == 0) s_hmax = 0;
  __syncthreads();
  MOE_PHASE(4);

  // ---- extraction: candidate columns re-read from L2, bucket counts ----
  {
    constexpr int BATCH = 4;  // loads in flight per lane
    const uint32_t rounds = wave_max_u32((uint32_t)__popc(mask));
    for (uint32_t it = 0; it < rounds; it += BATCH) {
      int col[BATCH];
      uint32_t bits[BATCH];
#pragma unroll
      for (int u = 0; u < BATCH; ++u) {
        col[u] = -1;
        if (mask) {
          const int i = __ffs(mask) - 1;
          mask &= mask - 1;
          col[u] = VEC * (tid + kRadixThreads * (i / VEC)) + (i % VEC);
        }
      }
#pragma unroll
      for (int u = 0; u < BATCH; ++u) bits[u] = Elem<T>::bits(x + (col[u] >= 0 ? col[u] : 0));
#pragma unroll
      for (int u = 0; u < BATCH; ++u) {
        if (col[u] >= 0) {
          const uint32_t k = key_of_bits(bits[u]);
          cand[cpos++] = make_comp(k, (uint32_t)col[u]);
          atomicAdd(&hist[kOrdBuckets - 1 - ((k - base) >> sh)], 1u);
        }
      }
    }
  }
  __syncthreads();
  {
    constexpr int BPT = kOrdBuckets / kRadixThreads;
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
      run += h[q];
    }
    if (tid == 0) bstart[kOrdBuckets] = C;
    hmax = wave_max_u32(hmax);
    if (lane == 0) atomicMax(&s_hmax, hmax);
  }
  __syncthreads();
  MOE_PHASE(5);
  for (uint32_t p = tid; p < C; p += kRadixThreads) {
    const uint64_t v = cand[p];
    const uint32_t pos = atomicAdd(&hist[kOrdBuckets - 1 - ((comp_key(v) - base) >> sh)], 1u);
    tmp[pos] = v;
  }
  __syncthreads();
  MOE_PHASE(6);
  const float vmax = value_of_key(rmax);

  if (s_hmax > (uint32_t)kBucketFixMax) {
    // Crowded bucket: sort all candidates (C <= kCandCap) instead.
    const int Cpad = next_pow2_dev((int)C);
    for (int p = (int)C + tid; p < Cpad; p += kRadixThreads) tmp[p] = 0;
    __syncthreads();
    lds_bitonic_desc(tmp, Cpad);
    radix_epilogue(tmp, K, row, s_red, scores, indices);
    MOE_PHASE(7);
    MOE_PHASE(8);
    return;
  }

  // ---- rank within bucket, exp, block sum, store ----
  int rk[CPT];
  float ex[CPT];
  uint32_t ix[CPT];
  float part = 0.0f;
#pragma unroll
  for (int u = 0; u < CPT; ++u) {
    const uint32_t p = tid + kRadixThreads * u;
    rk[u] = K;
    if (p < C) {
      const uint64_t v = tmp[p];
      const int rb = kOrdBuckets - 1 - (int)((comp_key(v) - base) >> sh);
      const int beg = (int)bstart[rb], end = (int)bstart[rb + 1];
      int r = beg;
      for (int q = beg; q < end; ++q) r += tmp[q] > v;
      rk[u] = r;
      ix[u] = comp_idx(v);
      ex[u] = expf(value_of_key(comp_key(v)) - vmax);
      if (r < K) part += ex[u];
    }
  }
  MOE_PHASE(7);
  part = wave_sum_f32(part);
  if (lane == 0) s_red[tid / kWave] = part;
  __syncthreads();
  float sum = 0.0f;
#pragma unroll
  for (int w = 0; w < kRadixThreads / kWave; ++w) sum += s_red[w];
#pragma unroll
  for (int u = 0; u < CPT; ++u)
    if (rk[u] < K) store_out(scores, indices, row * K + rk[u], ex[u] / sum, ix[u]);
  MOE_PHASE(8);
}

// Any N: the row is re-read from global memory (L2) in every pass.
template <typename T, typename IdxT>
__global__ __launch_bounds__(kRadixThreads) void topk_radix_kernel(
    const T* __restrict__ logits, int64_t M, int64_t N, int64_t ld, int K, int Kpad,
    float* __restrict__ scores, IdxT* __restrict__ indices) {
  extern __shared__ uint64_t sbuf[];  // [Kpad] winner composites
  __shared__ uint32_t hist[kRadixBins];
  __shared__ uint32_t wsum[kRadixThreads / kWave];
  __shared__ uint32_t s_pick[2], s_slot;
  __shared__ float s_red[kRadixThreads / kWave];

  const int tid = threadIdx.x;
  const int64_t row = blockIdx.x;
  const T* x = logits + row * ld;

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
  if (tid == 0) s_slot = 0;
  __syncthreads();
  const bool ties_partial = !st.all_taken && st.eq_count > st.need;
  for (int64_t i = tid; i < N; i += kRadixThreads) {
    const uint32_t key = key_of_bits(Elem<T>::bits(x + i));
    const uint32_t mk = key & st.fixed;
    const bool take = ties_partial ? (mk > st.prefix) : (mk >= st.prefix);
    if (take) {
      const uint32_t s = atomicAdd(&s_slot, 1u);
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
        const uint32_t s = atomicAdd(&s_slot, 1u);
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

template <typename T, typename IdxT>
static int launch_select(const T* x, int64_t M, int N, int64_t ld, int K, float* s, IdxT* id,
                         hipStream_t st) {
  const int epl = (N + kWave - 1) / kWave;
  if (epl <= 1) launch_select_e<T, IdxT, 1>(x, M, N, ld, K, s, id, st);
  else if (epl <= 2) launch_select_e<T, IdxT, 2>(x, M, N, ld, K, s, id, st);
  else if (epl <= 4) launch_select_e<T, IdxT, 4>(x, M, N, ld, K, s, id, st);
  else if (epl <= 8) launch_select_e<T, IdxT, 8>(x, M, N, ld, K, s, id, st);
  else if (epl <= 16) launch_select_e<T, IdxT, 16>(x, M, N, ld, K, s, id, st);
  else return fail(MOE_EUNSUP, "selection router supports N <= 1024");
  return check_launch("topk_select_kernel");
}

constexpr int kRadixRegMaxK = 8192;

template <typename T, typename IdxT, int VEC, int KPT>
static int launch_radix_reg(const T* x, int64_t M, int N, int64_t ld, int K, float* s, IdxT* id,
                            hipStream_t st) {
  const int Kpad = next_pow2(K);
  static bool attr_set = false;
  if (!attr_set) {
    MOE_HIP_CHECK(hipFuncSetAttribute((const void*)topk_radix_reg_kernel<T, IdxT, VEC, KPT>,
                                      hipFuncAttributeMaxDynamicSharedMemorySize,
                                      (int)(2 * kCandCap * sizeof(uint64_t))));
    attr_set = true;
  }
  topk_radix_reg_kernel<T, IdxT, VEC, KPT><<<dim3((unsigned)M), dim3(kRadixThreads),
                                              2 * kCandCap * sizeof(uint64_t), st>>>(x, M, N, ld, K, Kpad,
                                                                                     s, id);
  return check_launch("topk_radix_reg_kernel");
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

template <typename T, typename IdxT>
static int launch_radix(const T* x, int64_t M, int64_t N, int64_t ld, int K, float* s, IdxT* id,
                        hipStream_t st) {
  constexpr int VEC = 16 / sizeof(T);
  const bool vec_ok = ((uintptr_t)x % 16 == 0) && ((ld * (int64_t)sizeof(T)) % 16 == 0);
  if (K <= kRadixRegMaxK && N <= (int64_t)kRadixThreads * (vec_ok ? kRadixRegMaxKPT : 16)) {
    if (vec_ok) return launch_radix_reg_v<T, IdxT, VEC, VEC>(x, M, (int)N, ld, K, s, id, st);
    return launch_radix_reg_v<T, IdxT, 1, 1>(x, M, (int)N, ld, K, s, id, st);
  }
  const int Kpad = next_pow2(K);
  const size_t lds = (size_t)Kpad * sizeof(uint64_t);
  static bool attr_set = false;  // raise the dynamic-LDS cap once per process
  if (!attr_set) {
    MOE_HIP_CHECK(hipFuncSetAttribute((const void*)topk_radix_kernel<T, IdxT>,
                                      hipFuncAttributeMaxDynamicSharedMemorySize,
                                      (int)(kRadixMaxK * sizeof(uint64_t))));
    attr_set = true;
  }
  topk_radix_kernel<T, IdxT><<<dim3((unsigned)M), dim3(kRadixThreads), lds, st>>>(x, M, N, ld, K,
                                                                               Kpad, s, id);
  return check_launch("topk_radix_kernel");
}

template <typename T, typename IdxT>
static int dispatch_topk(const void* logits, int64_t M, int64_t N, int64_t ld, int64_t K,
                         float* scores, void* indices, int algo, hipStream_t st) {
  const T* x = static_cast<const T*>(logits);
  IdxT* id = static_cast<IdxT*>(indices);
  switch (algo) {
    case MOE_TOPK_BITONIC: return launch_bitonic<T, IdxT>(x, M, (int)N, ld, (int)K, scores, id, st);
    case MOE_TOPK_SELECTION: return launch_select<T, IdxT>(x, M, (int)N, ld, (int)K, scores, id, st);
    case MOE_TOPK_RADIX: return launch_radix<T, IdxT>(x, M, N, ld, (int)K, scores, id, st);
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
  (void)M; (void)N; (void)K; (void)algo;
  return 0;
}

extern "C" int moe_topk_softmax(const void* logits, int logits_dtype, int64_t M, int64_t N,
                                int64_t ld, int64_t K, float* scores, void* indices,
                                int idx_dtype, int algo, void* workspace, size_t ws_bytes,
                                void* stream) {
  (void)workspace; (void)ws_bytes;
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
  switch (logits_dtype) {
    case MOE_F32:
      return i64 ? dispatch_topk<float, int64_t>(logits, M, N, ld, K, scores, indices, algo, st)
                 : dispatch_topk<float, int32_t>(logits, M, N, ld, K, scores, indices, algo, st);
    case MOE_BF16:
      return i64 ? dispatch_topk<uint16_t, int64_t>(logits, M, N, ld, K, scores, indices, algo, st)
                 : dispatch_topk<uint16_t, int32_t>(logits, M, N, ld, K, scores, indices, algo, st);
    case MOE_F16:
      return i64 ? dispatch_topk<Half16, int64_t>(logits, M, N, ld, K, scores, indices, algo, st)
                 : dispatch_topk<Half16, int32_t>(logits, M, N, ld, K, scores, indices, algo, st);
    default:
      return fail(MOE_EINVAL, "topk_softmax: logits must be float32, bfloat16 or float16");
  }
}
