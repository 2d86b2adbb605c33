// Expert grouped GEMM for gfx950: device-side routing sort + bf16/fp16 MFMA.
//
// One call of moe_grouped_gemm is four stream-ordered kernels and no host
// synchronisation:
//   route_count_kernel    per-chunk expert histograms (LDS atomics)
//   route_scan_kernel     one workgroup: (expert, chunk) exclusive scan ->
//                         segment offsets, then the M-tile table
//   route_scatter_kernel  stable placement of each routed row into its
//                         expert segment (wave ballots + per-wave counts)
//   grouped_gemm_kernel   128x128x64 tiles, LDS double buffer, 2x2 waves of
//                         64x64 built from v_mfma_f32_32x32x16_{bf16,f16};
//                         the X row gather (r / topk) is fused into the A
//                         tile load and the un-permute into the epilogue store
// This replaces the reference's host-side argsort, bincount().tolist()
// synchronisation, Python offset/tile loops and per-call weight transpose
// (kernels/grouped_gemm_tilelang.py:700-732) and its E=256 per-expert
// torch.mm fallback (kernels/grouped_gemm_tilelang.py:542-601).
#include "common.h"

#include <algorithm>

namespace moe {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kRouteThreads = 256;
constexpr int kMaxExperts = 4096;
constexpr int kScanThreads = 1024;

template <typename IdxT>
__device__ inline int bucket_of(IdxT v, int E) {
  return (v >= 0 && v < (IdxT)E) ? (int)v : E;
}

// ---------------------------------------------------------------------------
// Routing sort.
// Rows are cut into chunks of `chunk` rows; blockcnt is laid out expert-major
// ([E+1][nb]) so that one exclusive scan over it yields, for every (expert,
// chunk), where that chunk's rows of that expert start in sorted_rows.
// Bucket E collects rows whose id is outside [0, E).
// ---------------------------------------------------------------------------
template <typename IdxT>
__global__ __launch_bounds__(kRouteThreads) void route_count_kernel(
    const IdxT* __restrict__ ids, int64_t R, int E, int chunk, int nb, int32_t* __restrict__ blockcnt) {
  extern __shared__ int32_t hist[];  // [E+1]
  for (int e = threadIdx.x; e <= E; e += kRouteThreads) hist[e] = 0;
  __syncthreads();
  const int64_t lo = (int64_t)blockIdx.x * chunk;
  const int64_t hi = std::min<int64_t>(R, lo + chunk);
  for (int64_t r = lo + threadIdx.x; r < hi; r += kRouteThreads) atomicAdd(&hist[bucket_of(ids[r], E)], 1);
  __syncthreads();
  for (int e = threadIdx.x; e <= E; e += kRouteThreads) blockcnt[(int64_t)e * nb + blockIdx.x] = hist[e];
}

__device__ inline int32_t block_excl_scan(int32_t v, int32_t* wsum) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int nw = blockDim.x / kWave;
  const int32_t incl = (int32_t)wave_incl_scan((uint32_t)v);
  if (lane == kWave - 1) wsum[wave] = incl;
  __syncthreads();
  int32_t base = 0;
  for (int w = 0; w < nw; ++w) base += (w < wave) ? wsum[w] : 0;
  __syncthreads();
  return base + incl - v;
}

// Single workgroup.  In: blockcnt ([E+1][nb] counts, nb <= 64).  Out:
// blockcnt[e][b] = rows of expert e in chunks before b (one wave scans one
// expert's nb counts with a single coalesced load), counts[E], offsets[E+1]
// and, when bm > 0, the GEMM M-tile table (tile_expert, tile_mstart,
// meta[0] = number of tiles).
__global__ __launch_bounds__(kScanThreads) void route_scan_kernel(
    int32_t* __restrict__ blockcnt, int64_t R, int E, int nb, int32_t* __restrict__ counts,
    int32_t* __restrict__ offsets, int bm, int32_t* __restrict__ tile_expert,
    int32_t* __restrict__ tile_mstart, int32_t* __restrict__ meta) {
  constexpr int NW = kScanThreads / kWave;
  constexpr int UNROLL = 4;
  __shared__ int32_t wsum[NW];
  __shared__ int32_t s_off[kMaxExperts + 2];
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  for (int e0 = wave * UNROLL; e0 <= E; e0 += NW * UNROLL) {
    int32_t v[UNROLL];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u)
      v[u] = (e0 + u <= E && lane < nb) ? blockcnt[(int64_t)(e0 + u) * nb + lane] : 0;
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      const int32_t incl = (int32_t)wave_incl_scan((uint32_t)v[u]);
      if (e0 + u <= E) {
        if (lane < nb) blockcnt[(int64_t)(e0 + u) * nb + lane] = incl - v[u];
        if (lane == kWave - 1) s_off[e0 + u] = incl;  // expert total
      }
    }
  }
  __syncthreads();
  // Exclusive scan of the E+1 expert totals (contiguous runs per thread).
  const int per = (E + 1 + kScanThreads - 1) / kScanThreads;
  const int lo = std::min(E + 1, tid * per), hi = std::min(E + 1, lo + per);
  int32_t tot[8], sum = 0;  // per <= 5 for E <= 4096
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    tot[q] = (lo + q < hi) ? s_off[lo + q] : 0;
    sum += tot[q];
  }
  int32_t run = block_excl_scan(sum, wsum);
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    if (lo + q < hi) s_off[lo + q] = run;
    run += tot[q];
  }
  if (tid == 0) s_off[E + 1] = (int32_t)R;
  __syncthreads();
  for (int e = tid; e <= E; e += kScanThreads) {
    offsets[e] = s_off[e];
    if (e < E) counts[e] = s_off[e + 1] - s_off[e];
  }
  if (bm <= 0) return;

  // Tile table: expert e owns ceil(count_e / bm) consecutive M tiles.
  const int perE = (E + kScanThreads - 1) / kScanThreads;
  const int elo = std::min(E, tid * perE), ehi = std::min(E, elo + perE);
  int32_t nt = 0;
  for (int e = elo; e < ehi; ++e) nt += (s_off[e + 1] - s_off[e] + bm - 1) / bm;
  int32_t t = block_excl_scan(nt, wsum);
  for (int e = elo; e < ehi; ++e) {
    const int32_t c = s_off[e + 1] - s_off[e];
    for (int32_t m = 0; m < c; m += bm, ++t) {
      tile_expert[t] = e;
      tile_mstart[t] = s_off[e] + m;
    }
  }
  if (ehi == E && elo < ehi) meta[0] = t;  // the thread owning the last expert
}

template <typename IdxT>
__global__ __launch_bounds__(kRouteThreads) void route_scatter_kernel(
    const IdxT* __restrict__ ids, int64_t R, int E, int chunk, int nb,
    const int32_t* __restrict__ blockoff, const int32_t* __restrict__ offsets,
    int32_t* __restrict__ sorted_rows) {
  extern __shared__ int32_t sm[];  // base[E+1], wcnt[4][E+1]
  constexpr int NW = kRouteThreads / kWave;
  int32_t* base = sm;
  int32_t* wcnt = sm + (E + 1);
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  const int nbits = 32 - __clz(E);  // bucket values lie in [0, E]
  for (int e = tid; e <= E; e += kRouteThreads) base[e] = offsets[e] + blockoff[(int64_t)e * nb + blockIdx.x];
  const int64_t lo = (int64_t)blockIdx.x * chunk;
  const int64_t hi = std::min<int64_t>(R, lo + chunk);
  const uint64_t lt_mask = (1ull << lane) - 1ull;
  for (int64_t sub = lo; sub < hi; sub += kRouteThreads) {
    for (int i = tid; i < NW * (E + 1); i += kRouteThreads) wcnt[i] = 0;
    __syncthreads();
    const int64_t r = sub + tid;
    const bool valid = r < hi;
    const int e = valid ? bucket_of(ids[r], E) : 0;
    // Lanes holding the same bucket: intersect the ballots of every bit.
    uint64_t match = __ballot(valid);
    for (int b = 0; b < nbits; ++b) {
      const uint64_t bal = __ballot((e >> b) & 1);
      match &= ((e >> b) & 1) ? bal : ~bal;
    }
    const int rank = __popcll(match & lt_mask);
    if (valid && rank == 0) wcnt[wave * (E + 1) + e] = __popcll(match);
    __syncthreads();
    if (valid) {
      int32_t prev = 0;
      for (int w = 0; w < wave; ++w) prev += wcnt[w * (E + 1) + e];
      sorted_rows[base[e] + prev + rank] = (int32_t)r;
    }
    __syncthreads();
    for (int b = tid; b <= E; b += kRouteThreads) {
      int32_t s = 0;
      for (int w = 0; w < NW; ++w) s += wcnt[w * (E + 1) + b];
      base[b] += s;
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// MFMA grouped GEMM.
// ---------------------------------------------------------------------------
constexpr int kBM = 128, kBN = 128, kBK = 64, kGemmThreads = 256;

template <typename T> struct MfmaOp;
template <> struct MfmaOp<uint16_t> {  // bfloat16
  static __device__ inline f32x16 run(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  static __device__ inline uint16_t cvt(float f) {  // round to nearest even
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0;
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
  }
};
template <> struct MfmaOp<Half16> {  // float16
  static __device__ inline f32x16 run(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  static __device__ inline uint16_t cvt(float f) {
    _Float16 h = (_Float16)f;
    uint16_t u;
    __builtin_memcpy(&u, &h, 2);
    return u;
  }
};

// LDS tile: rows of kBK = 64 elements = 8 chunks of 16 bytes; chunk c of row
// r is stored at chunk position c ^ (r & 7) so that the 32 rows read by one
// MFMA operand fetch spread over all banks.
__device__ inline int lds_slot(int r, int c) { return r * 8 + (c ^ (r & 7)); }

template <typename T>
__global__ __launch_bounds__(kGemmThreads, 2) void grouped_gemm_kernel(
    const uint16_t* __restrict__ X, const uint16_t* __restrict__ W, uint16_t* __restrict__ Y,
    int64_t H, int64_t I, int topk, int64_t R, int E, int ntn,
    const int32_t* __restrict__ sorted_rows, const int32_t* __restrict__ offsets,
    const int32_t* __restrict__ tile_expert, const int32_t* __restrict__ tile_mstart,
    const int32_t* __restrict__ meta) {
  __shared__ u32x4 As[2][kBM * kBK / 8];
  __shared__ u32x4 Bs[2][kBN * kBK / 8];
  __shared__ int32_t srow[kBM];

  const int tid = threadIdx.x;
  // XCD-aware order: the hardware deals consecutive workgroups round-robin
  // over the 8 XCDs, so give each XCD a contiguous range of the work list
  // (neighbouring N tiles of one M tile share the gathered X rows in L2).
  const int G = gridDim.x;  // multiple of 8
  const int w = (blockIdx.x & 7) * (G >> 3) + (blockIdx.x >> 3);
  const int mt = w / ntn, nt = w % ntn;
  const int n0 = nt * kBN;
  const int n_tiles = meta[0];

  if (mt >= n_tiles) {
    // Spare tiles zero the rows whose expert id lies outside [0, E).
    const int64_t z0 = (int64_t)offsets[E] + (int64_t)(mt - n_tiles) * kBM;
    for (int i = tid; i < kBM * kBN; i += kGemmThreads) {
      const int64_t p = z0 + i / kBN;
      const int64_t col = n0 + i % kBN;
      if (p < R && col < I) Y[(int64_t)sorted_rows[p] * I + col] = 0;
    }
    return;
  }

  const int e = tile_expert[mt];
  const int m0 = tile_mstart[mt];
  const int mend = offsets[e + 1];
  if (tid < kBM) srow[tid] = (m0 + tid < mend) ? sorted_rows[m0 + tid] : -1;
  __syncthreads();

  // Global -> LDS copy plan: thread owns chunk kc of rows tid/8 + 32q.
  const int kc = tid & 7;
  const uint16_t* a_ptr[4];
  const uint16_t* b_ptr[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int r = (tid >> 3) + 32 * q;
    const int sr = srow[r];
    a_ptr[q] = sr >= 0 ? X + (int64_t)(sr / topk) * H + kc * 8 : nullptr;
    const int64_t n = n0 + r;
    b_ptr[q] = n < I ? W + ((int64_t)e * I + n) * H + kc * 8 : nullptr;
  }

  const int nk = (int)((H + kBK - 1) / kBK);
  u32x4 ra[4], rb[4];
  const u32x4 zero = {0u, 0u, 0u, 0u};
  auto gload = [&](int kt) {
    const int64_t k = (int64_t)kt * kBK;
    const bool kin = k + kc * 8 < H;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      ra[q] = (a_ptr[q] && kin) ? *reinterpret_cast<const u32x4*>(a_ptr[q] + k) : zero;
      rb[q] = (b_ptr[q] && kin) ? *reinterpret_cast<const u32x4*>(b_ptr[q] + k) : zero;
    }
  };
  auto sstore = [&](int buf) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int r = (tid >> 3) + 32 * q;
      As[buf][lds_slot(r, kc)] = ra[q];
      Bs[buf][lds_slot(r, kc)] = rb[q];
    }
  };

  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;
  const int wm = wave >> 1, wn = wave & 1;
  f32x16 acc[2][2];
#pragma unroll
  for (int mi = 0; mi < 2; ++mi)
#pragma unroll
    for (int ni = 0; ni < 2; ++ni)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[mi][ni][v] = 0.0f;

  gload(0);
  sstore(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    if (kt + 1 < nk) gload(kt + 1);
    const int buf = kt & 1;
#pragma unroll
    for (int s = 0; s < kBK / 16; ++s) {
      const int c = 2 * s + (lane >> 5);
      u32x4 a[2], b[2];
#pragma unroll
      for (int mi = 0; mi < 2; ++mi) {
        const int r = wm * 64 + mi * 32 + (lane & 31);
        a[mi] = As[buf][lds_slot(r, c)];
      }
#pragma unroll
      for (int ni = 0; ni < 2; ++ni) {
        const int r = wn * 64 + ni * 32 + (lane & 31);
        b[ni] = Bs[buf][lds_slot(r, c)];
      }
#pragma unroll
      for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int ni = 0; ni < 2; ++ni) acc[mi][ni] = MfmaOp<T>::run(a[mi], b[ni], acc[mi][ni]);
    }
    if (kt + 1 < nk) sstore((kt + 1) & 1);
    __syncthreads();
  }

  // Epilogue: accumulator v of lane l holds row 8*(v/4) + 4*(l/32) + v%4,
  // column l%32 of its 32x32 block.  Rows are scattered back to their
  // original routed-row position.
#pragma unroll
  for (int mi = 0; mi < 2; ++mi) {
#pragma unroll
    for (int ni = 0; ni < 2; ++ni) {
      const int64_t col = n0 + wn * 64 + ni * 32 + (lane & 31);
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int i = (v >> 2) * 8 + (lane >> 5) * 4 + (v & 3);
        const int sr = srow[wm * 64 + mi * 32 + i];
        if (sr >= 0 && col < I) Y[(int64_t)sr * I + col] = MfmaOp<T>::cvt(acc[mi][ni][v]);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------
struct RoutePlan {
  int chunk, nb;
};

static RoutePlan route_plan(int64_t R) {
  // At most one wave's worth (64) of chunks, so the scan of an expert's
  // per-chunk counts is a single wave-wide load.
  const int64_t per_chunk = (R + kWave - 1) / kWave;
  const int64_t chunk = std::max<int64_t>(kRouteThreads, (per_chunk + kRouteThreads - 1) / kRouteThreads * kRouteThreads);
  RoutePlan p;
  p.chunk = (int)chunk;
  p.nb = (int)std::max<int64_t>(1, (R + chunk - 1) / chunk);
  return p;
}

static size_t align_up(size_t v) { return (v + 255) & ~(size_t)255; }

static size_t route_scratch_bytes(int64_t R, int64_t E) {
  return align_up((size_t)(E + 1) * route_plan(R).nb * sizeof(int32_t));
}

struct GemmLayout {
  size_t blockcnt, counts, offsets, sorted, tile_expert, tile_mstart, meta, total;
  int64_t mt_ub;
};

static GemmLayout gemm_layout(int64_t R, int64_t E) {
  GemmLayout g;
  g.mt_ub = (R + kBM - 1) / kBM + E + 1;
  size_t o = 0;
  g.blockcnt = o; o += route_scratch_bytes(R, E);
  g.counts = o; o += align_up(E * sizeof(int32_t));
  g.offsets = o; o += align_up((E + 1) * sizeof(int32_t));
  g.sorted = o; o += align_up(std::max<int64_t>(R, 1) * sizeof(int32_t));
  g.tile_expert = o; o += align_up(g.mt_ub * sizeof(int32_t));
  g.tile_mstart = o; o += align_up(g.mt_ub * sizeof(int32_t));
  g.meta = o; o += align_up(4 * sizeof(int32_t));
  g.total = o;
  return g;
}

template <typename IdxT>
static int launch_route(const IdxT* ids, int64_t R, int E, int32_t* blockcnt, int32_t* counts,
                        int32_t* offsets, int32_t* sorted_rows, int bm, int32_t* tile_expert,
                        int32_t* tile_mstart, int32_t* meta, hipStream_t st) {
  const RoutePlan p = route_plan(R);
  const size_t hist_lds = (size_t)(E + 1) * sizeof(int32_t);
  route_count_kernel<IdxT><<<p.nb, kRouteThreads, hist_lds, st>>>(ids, R, E, p.chunk, p.nb, blockcnt);
  if (int rc = check_launch("route_count_kernel")) return rc;
  route_scan_kernel<<<1, kScanThreads, 0, st>>>(blockcnt, R, E, p.nb, counts, offsets, bm, tile_expert,
                                                 tile_mstart, meta);
  if (int rc = check_launch("route_scan_kernel")) return rc;
  const size_t scat_lds = (size_t)(E + 1) * (1 + kRouteThreads / kWave) * sizeof(int32_t);
  static bool attr_set = false;  // E = 4096 needs more than the default 64 KB
  if (!attr_set) {
    MOE_HIP_CHECK(hipFuncSetAttribute((const void*)route_scatter_kernel<IdxT>,
                                      hipFuncAttributeMaxDynamicSharedMemorySize,
                                      (int)((kMaxExperts + 1) * (1 + kRouteThreads / kWave) * sizeof(int32_t))));
    attr_set = true;
  }
  route_scatter_kernel<IdxT><<<p.nb, kRouteThreads, scat_lds, st>>>(ids, R, E, p.chunk, p.nb, blockcnt,
                                                                     offsets, sorted_rows);
  return check_launch("route_scatter_kernel");
}

}  // namespace moe

using namespace moe;

extern "C" size_t moe_route_sort_workspace_size(int64_t R, int64_t E) {
  if (R < 0 || E < 1) return 0;
  return route_scratch_bytes(R, E);
}

extern "C" int moe_route_sort(const void* expert_ids, int idx_dtype, int64_t R, int64_t E,
                              int32_t* counts, int32_t* offsets, int32_t* sorted_rows,
                              void* workspace, size_t ws_bytes, void* stream) {
  if (R < 0 || R >= INT32_MAX) return fail(MOE_EINVAL, "route_sort: need 0 <= R < 2^31");
  if (E < 1 || E > kMaxExperts) return fail(MOE_EUNSUP, "route_sort: need 1 <= E <= 4096");
  if (idx_dtype != MOE_I32 && idx_dtype != MOE_I64)
    return fail(MOE_EINVAL, "route_sort: expert ids must be int32 or int64");
  if (!counts || !offsets || (R > 0 && (!expert_ids || !sorted_rows)))
    return fail(MOE_EINVAL, "route_sort: null pointer");
  const size_t need = route_scratch_bytes(R, E);
  if (ws_bytes < need || !workspace)
    return fail(MOE_EINVAL, "route_sort: workspace too small (" + std::to_string(ws_bytes) + " < " +
                                std::to_string(need) + ")");
  hipStream_t st = static_cast<hipStream_t>(stream);
  int32_t* blockcnt = static_cast<int32_t*>(workspace);
  if (idx_dtype == MOE_I64)
    return launch_route(static_cast<const int64_t*>(expert_ids), R, (int)E, blockcnt, counts, offsets,
                        sorted_rows, 0, nullptr, nullptr, nullptr, st);
  return launch_route(static_cast<const int32_t*>(expert_ids), R, (int)E, blockcnt, counts, offsets,
                      sorted_rows, 0, nullptr, nullptr, nullptr, st);
}

extern "C" size_t moe_grouped_gemm_workspace_size(int64_t T, int64_t topk, int64_t E, int64_t I) {
  (void)I;
  if (T < 0 || topk < 1 || E < 1) return 0;
  return gemm_layout(T * topk, E).total;
}

extern "C" int moe_grouped_gemm(const void* X, const void* W, const void* expert_ids, int dtype,
                                int idx_dtype, int64_t T, int64_t topk, int64_t H, int64_t I,
                                int64_t E, void* Y, void* workspace, size_t ws_bytes, void* stream) {
  if (T < 0 || topk < 1 || H < 1 || I < 1)
    return fail(MOE_EINVAL, "grouped_gemm: need T >= 0, topk >= 1, H >= 1, I >= 1");
  if (E < 1 || E > kMaxExperts) return fail(MOE_EUNSUP, "grouped_gemm: need 1 <= E <= 4096");
  if (H % 8 != 0) return fail(MOE_EUNSUP, "grouped_gemm: H must be a multiple of 8");
  const int64_t R = T * topk;
  if (R >= INT32_MAX || (R + kBM - 1) / kBM + E + 1 > (int64_t)INT32_MAX / ((I + kBN - 1) / kBN))
    return fail(MOE_EUNSUP, "grouped_gemm: problem too large");
  if (dtype != MOE_BF16 && dtype != MOE_F16)
    return fail(MOE_EINVAL, "grouped_gemm: X, W and Y must be bfloat16 or float16");
  if (idx_dtype != MOE_I32 && idx_dtype != MOE_I64)
    return fail(MOE_EINVAL, "grouped_gemm: expert ids must be int32 or int64");
  if (R == 0) return MOE_OK;
  if (!X || !W || !expert_ids || !Y) return fail(MOE_EINVAL, "grouped_gemm: null pointer");
  if (((uintptr_t)X | (uintptr_t)W) & 15)
    return fail(MOE_EINVAL, "grouped_gemm: X and W must be 16-byte aligned");
  const GemmLayout g = gemm_layout(R, E);
  if (!workspace || ws_bytes < g.total)
    return fail(MOE_EINVAL, "grouped_gemm: workspace too small (" + std::to_string(ws_bytes) + " < " +
                                std::to_string(g.total) + ")");
  hipStream_t st = static_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  int32_t* blockcnt = reinterpret_cast<int32_t*>(ws + g.blockcnt);
  int32_t* counts = reinterpret_cast<int32_t*>(ws + g.counts);
  int32_t* offsets = reinterpret_cast<int32_t*>(ws + g.offsets);
  int32_t* sorted = reinterpret_cast<int32_t*>(ws + g.sorted);
  int32_t* t_exp = reinterpret_cast<int32_t*>(ws + g.tile_expert);
  int32_t* t_ms = reinterpret_cast<int32_t*>(ws + g.tile_mstart);
  int32_t* meta = reinterpret_cast<int32_t*>(ws + g.meta);
  int rc;
  if (idx_dtype == MOE_I64)
    rc = launch_route(static_cast<const int64_t*>(expert_ids), R, (int)E, blockcnt, counts, offsets, sorted,
                      kBM, t_exp, t_ms, meta, st);
  else
    rc = launch_route(static_cast<const int32_t*>(expert_ids), R, (int)E, blockcnt, counts, offsets, sorted,
                      kBM, t_exp, t_ms, meta, st);
  if (rc) return rc;
  const int ntn = (int)((I + kBN - 1) / kBN);
  int64_t grid = g.mt_ub * ntn;
  grid = (grid + 7) / 8 * 8;
  const uint16_t* x = static_cast<const uint16_t*>(X);
  const uint16_t* w = static_cast<const uint16_t*>(W);
  uint16_t* y = static_cast<uint16_t*>(Y);
  if (dtype == MOE_BF16)
    grouped_gemm_kernel<uint16_t><<<dim3((unsigned)grid), kGemmThreads, 0, st>>>(
        x, w, y, H, I, (int)topk, R, (int)E, ntn, sorted, offsets, t_exp, t_ms, meta);
  else
    grouped_gemm_kernel<Half16><<<dim3((unsigned)grid), kGemmThreads, 0, st>>>(
        x, w, y, H, I, (int)topk, R, (int)E, ntn, sorted, offsets, t_exp, t_ms, meta);
  return check_launch("grouped_gemm_kernel");
}
