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
      const uint64_t o = shfl_xor_u64(c, j);
      const bool desc = (pos & k) == 0;
      const bool lower = (pos & j) == 0;
      c = (desc == lower) ? umax64(c, o) : umin64(c, o);
    }
  }

  // Softmax over positions [0, K) of each segment.
  const float v = value_of_key(comp_key(c));
  const float vmax = __shfl(v, lane & ~(S - 1), kWave);
  float e = pos < K ? expf(v - vmax) : 0.0f;
  float sum = e;
#pragma unroll
  for (int j = 1; j < S; j <<= 1) sum += __shfl_xor(sum, j, kWave);
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
#pragma unroll
    for (int m = kWave / 2; m >= 1; m >>= 1) best = umax64(best, shfl_xor_u64(best, m));
#pragma unroll
    for (int i = 0; i < EPL; ++i) c[i] = (c[i] == best) ? 0 : c[i];
    if (lane == 0) win[r] = best;
  }
  __syncthreads();
  if (!live) return;

  const float vmax = value_of_key(comp_key(win[0]));
  float sum = 0.0f;
  for (int r = lane; r < K; r += kWave) sum += expf(value_of_key(comp_key(win[r])) - vmax);
#pragma unroll
  for (int m = 1; m < kWave; m <<= 1) sum += __shfl_xor(sum, m, kWave);
  for (int r = lane; r < K; r += kWave) {
    const uint64_t w = win[r];
    store_out(scores, indices, row * K + r, expf(value_of_key(comp_key(w)) - vmax) / sum,
              comp_idx(w));
  }
}

// ===========================================================================
// 3. Radix select, one 1024-thread workgroup per row.
//    Replaces tl_topk_radix_kernel (kernels/topk_softmax_tilelang.py:54-202)
//    plus the torch gather + softmax that follows it (:1128-1131).
//    Digits: bits 31..21, 20..10, 9..0 of the 32-bit key.  Pass p builds a
//    2048-bin LDS histogram of digit p over the elements whose higher digits
//    equal the threshold prefix found so far, and picks the bin that holds
//    the K-th largest.  After the last pass the K-th largest key T and the
//    number of copies of T to take (lowest indices first) are exact.  The K
//    winners are collected as composites in LDS, bitonic-sorted descending,
//    and the softmax is applied in the same kernel.
// ===========================================================================
constexpr int kRadixThreads = 1024;
constexpr int kRadixBins = 2048;

__device__ inline uint32_t block_excl_scan_1024(uint32_t v, uint32_t* wsum, uint32_t* total) {
  // Exclusive prefix sum over a 1024-thread block; wsum needs 16 slots.
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  uint32_t incl = v;
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    const uint32_t t = __shfl_up(incl, d, kWave);
    if (lane >= d) incl += t;
  }
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

template <typename T, typename IdxT>
__global__ __launch_bounds__(kRadixThreads) void topk_radix_kernel(
    const T* __restrict__ logits, int64_t M, int64_t N, int64_t ld, int K, int Kpad,
    float* __restrict__ scores, IdxT* __restrict__ indices) {
  extern __shared__ uint64_t sbuf[];  // [Kpad] winner composites
  __shared__ uint32_t hist[kRadixBins];
  __shared__ uint32_t wsum[kRadixThreads / kWave];
  __shared__ uint32_t s_bin, s_above, s_slot;
  __shared__ float s_red[kRadixThreads / kWave];

  const int tid = threadIdx.x;
  const int64_t row = blockIdx.x;
  const T* x = logits + row * ld;

  uint32_t prefix = 0, fixed = 0;  // digits decided so far
  uint32_t need = (uint32_t)K;      // how many still to take at/below prefix
  uint32_t eq_count = 0;            // copies of the final threshold key
  bool all_taken = false;
  const int shifts[3] = {21, 10, 0};
  const uint32_t dmask[3] = {0x7FFu, 0x7FFu, 0x3FFu};

  for (int pass = 0; pass < 3 && !all_taken; ++pass) {
    const int sh = shifts[pass];
    const uint32_t dm = dmask[pass];
    for (int b = tid; b < kRadixBins; b += kRadixThreads) hist[b] = 0;
    __syncthreads();
    for (int64_t i = tid; i < N; i += kRadixThreads) {
      const uint32_t key = key_of_bits(Elem<T>::bits(x + i));
      if ((key & fixed) == prefix) atomicAdd(&hist[(key >> sh) & dm], 1u);
    }
    __syncthreads();
    // Bins in descending order: thread t owns bins 2047-2t and 2046-2t.
    const int b0 = kRadixBins - 1 - 2 * tid, b1 = b0 - 1;
    const uint32_t h0 = hist[b0], h1 = hist[b1];
    const uint32_t above0 = block_excl_scan_1024(h0 + h1, wsum, nullptr);
    const uint32_t above1 = above0 + h0;
    if (above0 < need && need <= above0 + h0) { s_bin = b0; s_above = above0; }
    if (above1 < need && need <= above1 + h1) { s_bin = b1; s_above = above1; }
    __syncthreads();
    const uint32_t bin = s_bin;
    need -= s_above;
    prefix |= bin << sh;
    fixed |= dm << sh;
    eq_count = hist[bin];
    if (eq_count == need) all_taken = true;  // whole bin selected
    __syncthreads();
  }

  // Selection rule: key > thr, or key == thr among the first `need` by index.
  // When a whole bin is taken, every key with the decided digits == prefix
  // qualifies: express that as "masked key >= prefix".
  if (tid == 0) s_slot = 0;
  __syncthreads();
  const bool ties_partial = !all_taken && eq_count > need;
  for (int64_t i = tid; i < N; i += kRadixThreads) {
    const uint32_t key = key_of_bits(Elem<T>::bits(x + i));
    const uint32_t mk = key & fixed;
    const bool take = ties_partial ? (mk > prefix) : (mk >= prefix);
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
    for (int64_t i = lo; i < hi; ++i) cnt += key_of_bits(Elem<T>::bits(x + i)) == prefix;
    uint32_t before = block_excl_scan_1024(cnt, wsum, nullptr);
    for (int64_t i = lo; i < hi && before < need; ++i) {
      const uint32_t key = key_of_bits(Elem<T>::bits(x + i));
      if (key == prefix) {
        const uint32_t s = atomicAdd(&s_slot, 1u);
        if (s < (uint32_t)Kpad) sbuf[s] = make_comp(key, (uint32_t)i);
        ++before;
      }
    }
  }
  __syncthreads();
  for (int i = K + tid; i < Kpad; i += kRadixThreads) sbuf[i] = 0;
  __syncthreads();

  // Descending bitonic sort of Kpad composites in LDS.
  for (int k = 2; k <= Kpad; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int p = tid; p < Kpad / 2; p += kRadixThreads) {
        const int i = 2 * p - (p & (j - 1));
        const int l = i + j;
        const uint64_t a = sbuf[i], b = sbuf[l];
        const bool desc = (i & k) == 0;
        if (desc ? (a < b) : (a > b)) { sbuf[i] = b; sbuf[l] = a; }
      }
      __syncthreads();
    }
  }

  // Softmax epilogue.
  const float vmax = value_of_key(comp_key(sbuf[0]));
  float part = 0.0f;
  for (int r = tid; r < K; r += kRadixThreads) part += expf(value_of_key(comp_key(sbuf[r])) - vmax);
#pragma unroll
  for (int m = 1; m < kWave; m <<= 1) part += __shfl_xor(part, m, kWave);
  if ((tid & (kWave - 1)) == 0) s_red[tid / kWave] = part;
  __syncthreads();
  float sum = 0.0f;
#pragma unroll
  for (int w = 0; w < kRadixThreads / kWave; ++w) sum += s_red[w];
  for (int r = tid; r < K; r += kRadixThreads) {
    const uint64_t w = sbuf[r];
    store_out(scores, indices, row * K + r, expf(value_of_key(comp_key(w)) - vmax) / sum,
              comp_idx(w));
  }
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

template <typename T, typename IdxT>
static int launch_radix(const T* x, int64_t M, int64_t N, int64_t ld, int K, float* s, IdxT* id,
                        hipStream_t st) {
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
