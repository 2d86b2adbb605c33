// Router GEMM and the fused router GEMM + TopK + softmax for gfx950.
//
// Replaces the reference's fused router kernels
// (kernels/router_gemm_topk_softmax.py:148-267 and the five variants after
// it) and its standalone router GEMM (:78-122).  logits = X[T,H] . W[H,E]
// in fp32; the fused form keeps the logits tile in LDS and writes only the
// K scores and indices per token.
//
// The weights are used transposed, Wt[E,H] (moe_router_weight_transpose):
// then both MFMA operands are K-contiguous rows and the tile k loop is the
// grouped GEMM's LDS-DMA pipeline (mfma_tile.h) unchanged.  A block owns
// BM = 64 tokens x BN (128 or 256) experts.  When the token count gives
// fewer tiles than CUs, H is split over G blocks per tile: block g stores its
// partial logits row-major in part[g][T][E] and is done.  The sum of the G
// partials, in split order (deterministic), is taken by whoever reads the
// logits next, spread over many workgroups: router_reduce_kernel for the
// logits entry point, the selection kernel itself (topk_select_partials)
// for the fused one.  (Split plans have too few tiles for a per-tile
// selection epilogue.)
//
// Fused epilogue (unsplit plans): the tile's logits go to LDS; a 16-lane
// segment selects one row (lane pos holds the keys of columns pos + 16 i):
// a filter from the lane maxima, then a sort of the few surviving
// composites (key << 32 | ~column), ties to the lower column; then the
// softmax over the K winners (Convention B, as topk_softmax).  The reference's fused
// kernels break ties toward the higher column instead
// (kernels/router_gemm_topk_softmax.py:224-229); this build keeps one tie
// rule for every router entry point.
#include "common.h"
#include "mfma_tile.h"
#include "moe_hip.h"

#include <algorithm>
#include <string>

namespace moe {

// ---------------------------------------------------------------------------
// Wt[E,H] = W[H,E]^T through a padded 64x64 LDS tile (16-byte accesses when
// rows are aligned and H, E are multiples of 8).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void router_transpose_kernel(const uint16_t* __restrict__ W,
                                                               uint16_t* __restrict__ Wt, int64_t H,
                                                               int64_t E, int64_t ldw, int vec) {
  __shared__ __attribute__((aligned(16))) uint16_t tile[64][72];  // rows padded to 144 bytes
  const int64_t h0 = (int64_t)blockIdx.y * 64, e0 = (int64_t)blockIdx.x * 64;
  if (vec) {
    // 16-byte aligned rows and H, E multiples of 8 (vec), so every 8-column
    // chunk lies wholly inside or outside the matrix: chunk c of the tile is
    // row c / 8, columns 8 (c % 8) ..  Each thread moves two chunks in and
    // two out; chunks past H or E are skipped (their LDS slots are unused).
#pragma unroll
    for (int c = threadIdx.x; c < 512; c += 256) {
      const int r = c >> 3, q = c & 7;
      if (h0 + r < H && e0 + 8 * q < E)
        *reinterpret_cast<uint4*>(&tile[r][8 * q]) = *reinterpret_cast<const uint4*>(W + (h0 + r) * ldw + e0 + 8 * q);
    }
    __syncthreads();
#pragma unroll
    for (int c = threadIdx.x; c < 512; c += 256) {
      const int r = c >> 3, q = c & 7;  // output row e0 + r, columns h0 + 8q ..
      if (e0 + r >= E || h0 + 8 * q >= H) continue;
      uint16_t v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = tile[8 * q + j][r];
      uint4 o;
      o.x = v[0] | ((uint32_t)v[1] << 16);
      o.y = v[2] | ((uint32_t)v[3] << 16);
      o.z = v[4] | ((uint32_t)v[5] << 16);
      o.w = v[6] | ((uint32_t)v[7] << 16);
      *reinterpret_cast<uint4*>(Wt + (e0 + r) * H + h0 + 8 * q) = o;
    }
    return;
  }
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  for (int r = ty; r < 64; r += 4) {
    const int64_t h = h0 + r, e = e0 + tx;
    tile[r][tx] = (h < H && e < E) ? W[h * ldw + e] : (uint16_t)0;
  }
  __syncthreads();
  for (int r = ty; r < 64; r += 4) {
    const int64_t e = e0 + r, h = h0 + tx;
    if (e < E && h < H) Wt[e * H + h] = tile[tx][r];
  }
}


using CfgRouter128 = GemmCfg<64, 128, 2, 2, 64, 3>;     // 4 waves of 32x64, 72 KB LDS
using CfgRouter192 = GemmCfg<64, 192, 2, 2, 64, 2>;     // 4 waves of 32x96, 64 KB LDS: two per CU
using CfgRouter256 = GemmCfg<64, 256, 1, 4, 64, 2>;     // 4 waves of 64x64, 80 KB LDS
constexpr int kRouterSeg = 16;                         // lanes per row in the fused epilogue
constexpr int kRouterMaxK = 2 * kRouterSeg;            // winners held two per lane
constexpr int64_t kRouterMinSplitK = 256;              // fewest k per split


// EPI 0: logits[T,E] fp32.  EPI 1: scores/indices [T,K] (requires one N tile).
template <typename T, typename Cfg, int EPI, typename IdxT>
__global__ __launch_bounds__(Cfg::THREADS) void router_gemm_kernel(
    const uint16_t* __restrict__ X, const uint16_t* __restrict__ Wt, int64_t Tn, int64_t H, int E, int K,
    int NT, int G, int64_t kchunk, float* __restrict__ logits, float* __restrict__ scores,
    IdxT* __restrict__ indices, float* __restrict__ part) {
  constexpr int BM = Cfg::BM, BN = Cfg::BN, CPR = Cfg::CPR;
  extern __shared__ __attribute__((aligned(16))) uint16_t smem[];

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;
  const int g = blockIdx.x % G;
  const int t = blockIdx.x / G;  // output tile
  const int nt = t % NT;
  const int64_t m0 = (int64_t)(t / NT) * BM;
  const int n0 = nt * BN;
  const int64_t kb = (int64_t)g * kchunk;
  const int64_t ke = min(H, kb + kchunk);

  // Copy plan (as the grouped GEMM): lane l fills slot l of each 1 KB copy
  // instruction.  Rows past T and columns past E read row 0; their results
  // are never stored.
  const int crow = lane / CPR;
  const uint16_t* a_src[Cfg::A_INS];
  const uint16_t* b_src[Cfg::B_INS];
#pragma unroll
  for (int i = 0; i < Cfg::A_INS; ++i) {
    const int64_t r = m0 + Cfg::RPI * (wave * Cfg::A_INS + i) + crow;
    a_src[i] = X + (r < Tn ? r : 0) * H + Cfg::copy_chunk(wave, i, Cfg::A_INS, lane) * 8;
  }
#pragma unroll
  for (int i = 0; i < Cfg::B_INS; ++i) {
    const int n = n0 + Cfg::RPI * (wave * Cfg::B_INS + i) + crow;
    b_src[i] = Wt + (int64_t)(n < E ? n : 0) * H + Cfg::copy_chunk(wave, i, Cfg::B_INS, lane) * 8;
  }
  const int wm = wave / Cfg::WN, wn = wave % Cfg::WN;
  const int mcount = (int)min((int64_t)BM, Tn - m0);
  const int fm_act = __builtin_amdgcn_readfirstlane(min(Cfg::FM, max(0, (mcount - wm * Cfg::FM * 32 + 31) / 32)));
  f32x16 acc[Cfg::FM][Cfg::FN];
#pragma unroll
  for (int i = 0; i < Cfg::FM; ++i)
#pragma unroll
    for (int j = 0; j < Cfg::FN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;
  tile_mainloop<T, Cfg, 0>(smem, a_src, b_src, kb, ke, fm_act, acc);

  // Accumulator v of lane l: row 8*(v/4) + 4*(l/32) + v%4, column l%32 of
  // its 32x32 block.
  auto row_of = [&](int i, int v) { return (wm * Cfg::FM + i) * 32 + (v >> 2) * 8 + (lane >> 5) * 4 + (v & 3); };
  auto col_of = [&](int j) { return (wn * Cfg::FN + j) * 32 + (lane & 31); };
  if constexpr (EPI == 0) {
    // Unsplit: the logits.  Split: this block's partial, part[g][T][E].
    float* dst = G > 1 ? part + (size_t)g * Tn * E : logits;
#pragma unroll
    for (int i = 0; i < Cfg::FM; ++i)
#pragma unroll
      for (int j = 0; j < Cfg::FN; ++j) {
        const int c = n0 + col_of(j);
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int64_t r = m0 + row_of(i, v);
          if (r < Tn && c < E) dst[r * E + c] = acc[i][j][v];
        }
      }
    return;
  } else {
    // Logits tile to LDS (reusing the stage ring), row stride BN + 1.
    float* lt = reinterpret_cast<float*>(smem);
    constexpr int LDR = BN + 1;
    static_assert((size_t)BM * (BN + 1) * 4 + Cfg::THREADS * 8 <= Cfg::LDS_BYTES,
                  "logits tile and selection scratch must fit the stage ring");
    __syncthreads();  // every wave is done reading the operand stages
#pragma unroll
    for (int i = 0; i < Cfg::FM; ++i)
#pragma unroll
      for (int j = 0; j < Cfg::FN; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) lt[row_of(i, v) * LDR + col_of(j)] = acc[i][j][v];
    __syncthreads();

    // One 16-lane segment (a DPP row) per row: 16 rows per pass.
    constexpr int EPL = BN / kRouterSeg;
    constexpr int ROWS_PER_PASS = Cfg::THREADS / kRouterSeg;
    uint64_t* seg_scratch = reinterpret_cast<uint64_t*>(lt + BM * LDR) + (tid / kRouterSeg) * kRouterSeg;
    const int pos = lane & (kRouterSeg - 1);
    for (int r0 = 0; r0 < BM; r0 += ROWS_PER_PASS) {
      const int rl = r0 + tid / kRouterSeg;
      const int64_t row = m0 + rl;
      const bool live = row < Tn;
      uint32_t key[EPL];
#pragma unroll
      for (int i = 0; i < EPL; ++i) {
        const int col = pos + kRouterSeg * i;
        key[i] = (live && col < E) ? key_of_bits(__float_as_uint(lt[rl * LDR + col])) : 0u;
      }
      // Lane pos ends with winners pos and pos + 16 (composites, 0 = none).
      uint64_t win[kRouterMaxK / kRouterSeg] = {0, 0};
      if (!seg16_topk_filtered<EPL>(key, K, seg_scratch, win[0], [](int p, int i) { return p + kRouterSeg * i; })) {
        // Rounds of a segment max: K > 16, or more than 16 keys at or
        // above the filter (heavy ties).
        uint64_t c[EPL];
#pragma unroll
        for (int i = 0; i < EPL; ++i) c[i] = key[i] ? make_comp(key[i], (uint32_t)(pos + kRouterSeg * i)) : 0;
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
          if ((r & (kRouterSeg - 1)) == pos) win[r / kRouterSeg] = best;
        }
      }
      // Softmax over the K winners; winner 0 (lane 0) holds the maximum.
      const float vmax = value_of_key(comp_key(seg16_shfl_u64(win[0], 0)));
      float e[kRouterMaxK / kRouterSeg];
      float sum = 0.0f;
#pragma unroll
      for (int q = 0; q < kRouterMaxK / kRouterSeg; ++q) {
        const int r = pos + kRouterSeg * q;
        e[q] = r < K ? expf(value_of_key(comp_key(win[q])) - vmax) : 0.0f;
        sum += e[q];
      }
      sum += xor_lanes_f32<1>(sum);
      sum += xor_lanes_f32<2>(sum);
      sum += xor_lanes_f32<4>(sum);
      sum += xor_lanes_f32<8>(sum);
      if (live) {
#pragma unroll
        for (int q = 0; q < kRouterMaxK / kRouterSeg; ++q) {
          const int r = pos + kRouterSeg * q;
          if (r < K) {
            scores[row * K + r] = e[q] / sum;
            indices[row * K + r] = (IdxT)comp_idx(win[q]);
          }
        }
      }
    }
  }
}

// logits[i] = part[0][i] + part[1][i] + ... + part[G-1][i], summed in split
// order, over the n = T * E logits (4 per thread when n allows).
__global__ __launch_bounds__(256) void router_reduce_kernel(const float* __restrict__ part, int G, int64_t n,
                                                            float* __restrict__ logits) {
  const int64_t i4 = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (i4 >= n) return;
  if (n % 4 == 0) {
    float4 a = *reinterpret_cast<const float4*>(part + i4);
    for (int g = 1; g < G; ++g) {
      const float4 b = *reinterpret_cast<const float4*>(part + (size_t)g * n + i4);
      a.x += b.x; a.y += b.y; a.z += b.z; a.w += b.w;
    }
    *reinterpret_cast<float4*>(logits + i4) = a;
  } else {
    for (int64_t i = i4; i < min(n, i4 + 4); ++i) {
      float a = part[i];
      for (int g = 1; g < G; ++g) a += part[(size_t)g * n + i];
      logits[i] = a;
    }
  }
}

// ---------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------
struct RouterPlan {
  int cfg;  // 0: 64x128 tiles, 1: 64x256 tiles, 2: 64x192 tiles
  int NT, G;
  int64_t tiles, kchunk;
  size_t part_floats;
};

template <typename Cfg>
static RouterPlan router_plan_cfg(int cfg, int64_t T, int64_t H, int64_t E) {
  RouterPlan p;
  p.cfg = cfg;
  p.NT = (int)((E + Cfg::BN - 1) / Cfg::BN);
  p.tiles = (T + Cfg::BM - 1) / Cfg::BM * p.NT;
  // Split H until there are about two workgroups per CU (a tile's k loop is
  // bound by the latency of its operand copies, so a second resident
  // workgroup per CU overlaps them: DeepSeek-V2 T = 16384, 256 tiles, runs
  // 6% faster split in two), keeping at least kRouterMinSplitK per split so
  // the partial logits stay small next to the operands.
  int64_t G = 1;
  const int64_t want = 512;
  if (p.tiles < want) G = std::max<int64_t>(1, std::min<int64_t>(want / p.tiles, H / kRouterMinSplitK));
  int64_t kchunk = (H + G - 1) / G;
  kchunk = (kchunk + Cfg::BK - 1) / Cfg::BK * Cfg::BK;
  p.G = (int)((H + kchunk - 1) / kchunk);
  p.kchunk = kchunk;
  p.part_floats = p.G > 1 ? (size_t)p.G * T * E : 0;
  return p;
}

static RouterPlan router_plan(int64_t T, int64_t H, int64_t E) {
  // The narrowest tile that holds all E experts: the padding columns still
  // cost their weight-row copies.
  return E <= CfgRouter128::BN   ? router_plan_cfg<CfgRouter128>(0, T, H, E)
         : E <= CfgRouter192::BN ? router_plan_cfg<CfgRouter192>(2, T, H, E)
                                 : router_plan_cfg<CfgRouter256>(1, T, H, E);
}

// Bytes of the split-H partial logits [G][T][E] (split plans only).
static size_t router_part_bytes(const RouterPlan& p) { return (p.part_floats * sizeof(float) + 255) & ~(size_t)255; }
static size_t router_ws_bytes(const RouterPlan& p, int64_t T, int64_t E) {
  (void)T;
  (void)E;
  return kWsCtlBytes + router_part_bytes(p);
}

template <typename T, typename Cfg, int EPI, typename IdxT>
static int launch_router(const RouterPlan& p, const uint16_t* x, const uint16_t* wt, int64_t Tn, int64_t H,
                         int E, int K, float* logits, float* scores, IdxT* idx, void* ws, hipStream_t st) {
  static std::atomic<uint64_t> lds_cap_set{0};
  MOE_HIP_CHECK(lds_cap_once(lds_cap_set, (const void*)router_gemm_kernel<T, Cfg, EPI, IdxT>, (int)Cfg::LDS_BYTES, st));
  float* part = p.G > 1 ? reinterpret_cast<float*>(static_cast<char*>(ws) + kWsCtlBytes) : nullptr;
  const int64_t grid = p.tiles * p.G;
  router_gemm_kernel<T, Cfg, EPI, IdxT><<<dim3((unsigned)grid), Cfg::THREADS, Cfg::LDS_BYTES, st>>>(
      x, wt, Tn, H, E, K, p.NT, p.G, p.kchunk, logits, scores, idx, part);
  return check_launch("router_gemm_kernel");
}

template <int EPI, typename IdxT>
static int dispatch_router(int dtype, const RouterPlan& p, const void* X, const void* Wt, int64_t T, int64_t H,
                           int64_t E, int64_t K, float* logits, float* scores, IdxT* idx, void* ws, hipStream_t st) {
  const uint16_t* x = static_cast<const uint16_t*>(X);
  const uint16_t* wt = static_cast<const uint16_t*>(Wt);
  auto run = [&](auto t_tag, auto cfg_tag) {
    using TT = decltype(t_tag);
    using C = decltype(cfg_tag);
    return launch_router<TT, C, EPI, IdxT>(p, x, wt, T, H, (int)E, (int)K, logits, scores, idx, ws, st);
  };
  if (dtype == MOE_BF16)
    return p.cfg == 0 ? run(uint16_t{}, CfgRouter128{}) : p.cfg == 2 ? run(uint16_t{}, CfgRouter192{})
                                                                      : run(uint16_t{}, CfgRouter256{});
  return p.cfg == 0 ? run(Half16{}, CfgRouter128{}) : p.cfg == 2 ? run(Half16{}, CfgRouter192{})
                                                                  : run(Half16{}, CfgRouter256{});
}

static int router_check(const char* fn, const void* X, const void* Wt, int dtype, int64_t T, int64_t H, int64_t E,
                        void* ws, size_t ws_bytes, const RouterPlan& p) {
  const std::string f(fn);
  if (T < 0 || H < 1 || E < 1) return fail(MOE_EINVAL, f + ": need T >= 0, H >= 1, E >= 1");
  if (H % 8 != 0) return fail(MOE_EUNSUP, f + ": H must be a multiple of 8");
  if (dtype != MOE_BF16 && dtype != MOE_F16) return fail(MOE_EINVAL, f + ": X and Wt must be bfloat16 or float16");
  if (T > INT32_MAX || E > 65536) return fail(MOE_EUNSUP, f + ": problem too large");
  if (T == 0) return MOE_OK;
  if (!X || !Wt) return fail(MOE_EINVAL, f + ": null pointer");
  if (((uintptr_t)X | (uintptr_t)Wt) & 15) return fail(MOE_EINVAL, f + ": X and Wt must be 16-byte aligned");
  const size_t need = router_ws_bytes(p, T, E);
  if (!ws || ws_bytes < need)
    return fail(MOE_EINVAL, f + ": workspace too small (" + std::to_string(ws_bytes) + " < " + std::to_string(need) + ")");
  return MOE_OK;
}

}  // namespace moe

using namespace moe;

extern "C" int moe_router_weight_transpose(const void* W, int dtype, int64_t H, int64_t E, int64_t ldw, void* Wt,
                                           void* stream) {
  if (H < 1 || E < 1 || ldw < E) return fail(MOE_EINVAL, "router_weight_transpose: need H >= 1, E >= 1, ldw >= E");
  if (dtype != MOE_BF16 && dtype != MOE_F16)
    return fail(MOE_EINVAL, "router_weight_transpose: W must be bfloat16 or float16");
  if (!W || !Wt) return fail(MOE_EINVAL, "router_weight_transpose: null pointer");
  if ((H + 63) / 64 > 65535) return fail(MOE_EUNSUP, "router_weight_transpose: H too large");
  const dim3 grid((unsigned)((E + 63) / 64), (unsigned)((H + 63) / 64));
  // 16-byte path: W and Wt rows 16-byte aligned, whole 8-column chunks.
  const int vec = ((uintptr_t)W % 16 == 0) && ((uintptr_t)Wt % 16 == 0) && ldw % 8 == 0 && H % 8 == 0 && E % 8 == 0;
  router_transpose_kernel<<<grid, 256, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const uint16_t*>(W), static_cast<uint16_t*>(Wt), H, E, ldw, vec);
  return check_launch("router_transpose_kernel");
}

extern "C" size_t moe_router_workspace_size(int64_t T, int64_t H, int64_t E) {
  if (T < 1 || H < 1 || E < 1) return kWsCtlBytes;
  return router_ws_bytes(router_plan(T, H, E), T, E);
}

namespace moe {
int router_gemm_logits_or_partials(const void* X, const void* Wt, int dtype, int64_t T, int64_t H, int64_t E,
                                   float* logits, const float** part, int* G, void* workspace, size_t ws_bytes,
                                   hipStream_t st) {
  const RouterPlan p = router_plan(std::max<int64_t>(T, 1), std::max<int64_t>(H, 1), std::max<int64_t>(E, 1));
  if (int rc = router_check("router_gemm", X, Wt, dtype, T, H, E, workspace, ws_bytes, p)) return rc;
  *G = p.G;
  *part = p.G > 1 ? reinterpret_cast<const float*>(static_cast<char*>(workspace) + kWsCtlBytes) : nullptr;
  if (T == 0) return MOE_OK;
  if (p.G == 1 && !logits) return fail(MOE_EINVAL, "router_gemm: null pointer");
  return dispatch_router<0, int32_t>(dtype, p, X, Wt, T, H, E, 0, logits, nullptr, nullptr, workspace, st);
}
}  // namespace moe

extern "C" int moe_router_gemm(const void* X, const void* Wt, int dtype, int64_t T, int64_t H, int64_t E,
                               float* logits, void* workspace, size_t ws_bytes, void* stream) {
  const RouterPlan p = router_plan(std::max<int64_t>(T, 1), std::max<int64_t>(H, 1), std::max<int64_t>(E, 1));
  if (int rc = router_check("router_gemm", X, Wt, dtype, T, H, E, workspace, ws_bytes, p)) return rc;
  if (T == 0) return MOE_OK;
  if (!logits) return fail(MOE_EINVAL, "router_gemm: null pointer");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (int rc = dispatch_router<0, int32_t>(dtype, p, X, Wt, T, H, E, 0, logits, nullptr, nullptr, workspace, st))
    return rc;
  if (p.G > 1) {
    const float* part = reinterpret_cast<const float*>(static_cast<char*>(workspace) + kWsCtlBytes);
    const int64_t n = T * E;
    router_reduce_kernel<<<(unsigned)((n + 1023) / 1024), 256, 0, st>>>(part, p.G, n, logits);
    return check_launch("router_reduce_kernel");
  }
  return MOE_OK;
}

extern "C" int moe_router_topk_softmax(const void* X, const void* Wt, int dtype, int64_t T, int64_t H, int64_t E,
                                       int64_t K, float* scores, void* indices, int idx_dtype, void* workspace,
                                       size_t ws_bytes, void* stream) {
  if (K < 1 || K > E)
    return fail(MOE_EINVAL, "router_topk_softmax: need 1 <= K <= E (got K=" + std::to_string(K) + ", E=" +
                                std::to_string(E) + ")");
  if (E > CfgRouter256::BN || K > kRouterMaxK)
    return fail(MOE_EUNSUP, "router_topk_softmax: the fused path needs E <= 256 and K <= 32 "
                            "(use moe_router_gemm + moe_topk_softmax)");
  if (idx_dtype != MOE_I32 && idx_dtype != MOE_I64)
    return fail(MOE_EINVAL, "router_topk_softmax: indices must be int32 or int64");
  const RouterPlan p = router_plan(std::max<int64_t>(T, 1), std::max<int64_t>(H, 1), E);
  if (int rc = router_check("router_topk_softmax", X, Wt, dtype, T, H, E, workspace, ws_bytes, p)) return rc;
  if (T == 0) return MOE_OK;
  if (!scores || !indices) return fail(MOE_EINVAL, "router_topk_softmax: null pointer");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (p.G > 1) {
    // H is split over G workgroups per tile: the selection kernel (one wave
    // per token) sums each token's G partial rows in split order as it loads
    // them, then selects.  Same results as the fused epilogue.
    if (int rc = dispatch_router<0, int32_t>(dtype, p, X, Wt, T, H, E, 0, nullptr, nullptr, nullptr, workspace, st))
      return rc;
    const float* part = reinterpret_cast<const float*>(static_cast<char*>(workspace) + kWsCtlBytes);
    return topk_select_partials(part, p.G, T, (int)E, (int)K, MOE_SCORES_TOPK, scores, indices, idx_dtype, st);
  }
  if (idx_dtype == MOE_I64)
    return dispatch_router<1, int64_t>(dtype, p, X, Wt, T, H, E, K, nullptr, scores, static_cast<int64_t*>(indices),
                                       workspace, st);
  return dispatch_router<1, int32_t>(dtype, p, X, Wt, T, H, E, K, nullptr, scores, static_cast<int32_t*>(indices),
                                     workspace, st);
}
