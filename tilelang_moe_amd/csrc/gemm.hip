// Expert grouped GEMM for gfx950: device-side routing sort + bf16/fp16 MFMA.
//
// One call of moe_grouped_gemm is four stream-ordered kernels and no host
// synchronisation:
//   route_count_kernel    per-chunk expert histograms (LDS atomics)
//   route_scan_kernel     one workgroup: (expert, chunk) exclusive scan ->
//                         segment offsets, then the M-tile table
//   route_scatter_kernel  stable placement of each routed row into its
//                         expert segment (wave ballots + per-wave counts)
//   grouped_gemm_kernel   128x256 (or 64x128) tiles, 2x2 waves built from
//                         v_mfma_f32_32x32x16_{bf16,f16}, a 3-stage LDS ring
//                         filled by global_load_lds_dwordx4;
//                         the X row gather (r / topk) is fused into the A
//                         tile load and the un-permute into the epilogue store
// This replaces the reference's host-side argsort, bincount().tolist()
// synchronisation, Python offset/tile loops and per-call weight transpose
// (kernels/grouped_gemm_tilelang.py:700-732) and its E=256 per-expert
// torch.mm fallback (kernels/grouped_gemm_tilelang.py:542-601).
#include "common.h"
#include "mfma_tile.h"

#include <algorithm>
#include <mutex>
#include <string>
#include <type_traits>

namespace moe {

constexpr int kRouteThreads = 256;
constexpr int kMaxExperts = 4096;
constexpr int kScanThreads = 1024;
// Tile tables may mix two tile heights: an entry of tile_expert with this
// bit set is a short tile (the second configuration of the GEMM kernel).
// The tile height argument `bm` of the routing kernels is then
// bm_mixed(tall, short, blk, reserve): experts with at most `short` rows get
// one short tile, the others tiles of `tall` rows; blk and reserve order the
// table (build_tile_table).
constexpr int32_t kShortTile = 1 << 30;
constexpr int bm_mixed(int tall, int shrt, int blk, int reserve) {
  return tall | shrt << 10 | blk << 20 | reserve << 26;
}
// Byte offset of the grouped GEMM's nine schedule counters in the
// workspace control block.
constexpr size_t kGemmSchedOffset = 3072;

// MOE_GEMM_TUNE_MODE (tuning builds only): 1 = copies only, 2 = MFMAs only.
#ifndef MOE_GEMM_TUNE_MODE
#define MOE_GEMM_TUNE_MODE 0
#endif

// Bucket of routed row r.  Rows r < R_ids carry an expert id, valid in
// [0, E_ids); rows r >= R_ids (an appended set, e.g. a shared expert taken
// by every token) belong to expert E_ids.  Bucket E (the number of experts,
// E_ids or E_ids + 1) collects the invalid ids.
template <typename IdxT>
__device__ inline int bucket_of(const IdxT* ids, int64_t r, int64_t R_ids, int E_ids, int E) {
  if (r >= R_ids) return E_ids;
  const IdxT v = ids[r];
  return (v >= 0 && v < (IdxT)E_ids) ? (int)v : E;
}

// ---------------------------------------------------------------------------
// Routing sort.
// Rows are cut into chunks of `chunk` rows; blockcnt is laid out expert-major
// ([E+1][nb]) so that one exclusive scan over it yields, for every (expert,
// chunk), where that chunk's rows of that expert start in sorted_rows.
// Bucket E collects rows whose id is invalid (bucket_of).
// ---------------------------------------------------------------------------
template <typename IdxT>
__global__ __launch_bounds__(kRouteThreads) void route_count_kernel(
    const IdxT* __restrict__ ids, int64_t R, int64_t R_ids, int E_ids, int E, int chunk, int nb,
    int32_t* __restrict__ blockcnt) {
  extern __shared__ int32_t hist[];  // [E+1]
  for (int e = threadIdx.x; e <= E; e += kRouteThreads) hist[e] = 0;
  __syncthreads();
  const int64_t lo = (int64_t)blockIdx.x * chunk;
  const int64_t hi = std::min<int64_t>(R, lo + chunk);
  for (int64_t r = lo + threadIdx.x; r < hi; r += kRouteThreads) atomicAdd(&hist[bucket_of(ids, r, R_ids, E_ids, E)], 1);
  __syncthreads();
  for (int e = threadIdx.x; e <= E; e += kRouteThreads) blockcnt[(int64_t)e * nb + blockIdx.x] = hist[e];
}

__device__ inline int32_t block_excl_scan(int32_t v, int32_t* wsum) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int nw = blockDim.x / kWave;
  const int32_t incl = (int32_t)wave_incl_scan((uint32_t)v);
  if (lane == kWave - 1) wsum[wave] = incl;
  lds_barrier();
  int32_t base = 0;
  for (int w = 0; w < nw; ++w) base += (w < wave) ? wsum[w] : 0;
  lds_barrier();
  return base + incl - v;
}

__device__ inline void build_tile_table(const int32_t* s_off, int E, int bm, int32_t* wsum,
                                        int32_t* __restrict__ tile_expert, int32_t* __restrict__ tile_mstart,
                                        int32_t* __restrict__ meta);

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
  build_tile_table(s_off, E, bm, wsum, tile_expert, tile_mstart, meta);
}

// The M-tile table for tile height bm from segment offsets already in LDS
// (s_off[0..E], published by a barrier): expert e owns ceil(count_e / bm)
// consecutive M tiles, or one short tile when bm = bm_mixed(tall, short,
// blk, reserve) and count_e <= short; meta[0] = number of table entries.
// One block (any size).
//
// With blk > 0 the tall and the short tiles alternate in blocks of blk
// entries (T S T S ..., the longer list's remainder next), so that a GEMM
// that walks the table in super-tiles of blk M tiles runs weight-streaming
// short tiles beside compute-heavy tall ones; the last `reserve` short
// blocks are kept for the end of the table, so the schedule ends on cheap
// tiles.  A partial block that another block follows leaves holes, marked
// tile_expert = -1.
__device__ inline void build_tile_table(const int32_t* s_off, int E, int bm, int32_t* wsum,
                                        int32_t* __restrict__ tile_expert, int32_t* __restrict__ tile_mstart,
                                        int32_t* __restrict__ meta) {
  const int tid = threadIdx.x;
  const int tall = bm & 0x3FF, shrt = (bm >> 10) & 0x3FF, blk = (bm >> 20) & 0x3F, reserve = (bm >> 26) & 0x1F;
  const int perE = (E + (int)blockDim.x - 1) / (int)blockDim.x;
  const int elo = std::min(E, tid * perE), ehi = std::min(E, elo + perE);
  // Without interleaving (blk == 0) the tall tiles come first, then the
  // short ones: the GEMM's dynamic schedule then ends on the cheap tiles.
  int32_t nt = 0, ns = 0;
  for (int e = elo; e < ehi; ++e) {
    const int32_t c = s_off[e + 1] - s_off[e];
    if (c > 0 && c <= shrt) ++ns;
    else nt += (c + tall - 1) / tall;
  }
  __shared__ int32_t s_tall_total, s_short_total;
  int32_t t = block_excl_scan(nt, wsum);
  if (tid == (int)blockDim.x - 1) s_tall_total = t + nt;
  int32_t ts = block_excl_scan(ns, wsum);  // its barriers also publish s_tall_total
  if (blk == 0) {
    ts += s_tall_total;
    for (int e = elo; e < ehi; ++e) {
      const int32_t c = s_off[e + 1] - s_off[e];
      if (c > 0 && c <= shrt) {
        tile_expert[ts] = e | kShortTile;
        tile_mstart[ts] = s_off[e];
        ++ts;
        continue;
      }
      for (int32_t m = 0; m < c; m += tall, ++t) {
        tile_expert[t] = e;
        tile_mstart[t] = s_off[e] + m;
      }
    }
    if (tid == (int)blockDim.x - 1) meta[0] = ts;  // the last thread's short tiles end the table
    return;
  }
  if (tid == (int)blockDim.x - 1) s_short_total = ts + ns;
  __syncthreads();
  const int32_t nTb = (s_tall_total + blk - 1) / blk, nSb = (s_short_total + blk - 1) / blk;
  const int32_t s1 = nSb > reserve ? nSb - reserve : 0;  // short blocks interleaved with the tall ones
  const int32_t entries = (nTb + nSb) * blk;
  // Final position of entry i of the tall (short) list: tall block b goes to
  // 2b while interleaved short blocks remain (b < s1), after them
  // otherwise; short block b < s1 goes to 2b+1 while tall blocks remain;
  // every other short block follows all tall blocks.
  auto pos_tall = [&](int32_t i) { const int32_t b = i / blk; return (b < s1 ? 2 * b : s1 + b) * blk + i % blk; };
  auto pos_short = [&](int32_t i) {
    const int32_t b = i / blk;
    return (b < s1 && b < nTb ? 2 * b + 1 : nTb + b) * blk + i % blk;
  };
  for (int32_t i = tid; i < entries; i += (int)blockDim.x) tile_expert[i] = -1;  // holes stay -1
  __syncthreads();
  for (int e = elo; e < ehi; ++e) {
    const int32_t c = s_off[e + 1] - s_off[e];
    if (c > 0 && c <= shrt) {
      const int32_t p = pos_short(ts++);
      tile_expert[p] = e | kShortTile;
      tile_mstart[p] = s_off[e];
      continue;
    }
    for (int32_t m = 0; m < c; m += tall, ++t) {
      const int32_t p = pos_tall(t);
      tile_expert[p] = e;
      tile_mstart[p] = s_off[e] + m;
    }
  }
  if (tid == 0) meta[0] = entries;
}

// The tile table alone, for routing tables built by an earlier call for a
// different tile height (offsets[0..E] are final).
__global__ __launch_bounds__(kScanThreads) void route_tiles_kernel(const int32_t* __restrict__ offsets, int E, int bm,
                                                                  int32_t* __restrict__ tile_expert,
                                                                  int32_t* __restrict__ tile_mstart,
                                                                  int32_t* __restrict__ meta) {
  __shared__ int32_t wsum[kScanThreads / kWave];
  __shared__ int32_t s_off[kMaxExperts + 2];
  for (int e = threadIdx.x; e <= E; e += kScanThreads) s_off[e] = offsets[e];
  __syncthreads();
  build_tile_table(s_off, E, bm, wsum, tile_expert, tile_mstart, meta);
}

// SCAN = false: blockoff holds route_scan_kernel's per-chunk prefixes and
// offsets the segment starts.  SCAN = true (E + 1 <= 2 kRouteThreads, so the
// scan needs no launch of its own): blockoff holds route_count_kernel's raw
// per-chunk counts, from which every workgroup derives the segment starts
// and its chunk's prefixes, and workgroup 0 writes counts, offsets and the
// tile table as route_scan_kernel does.
template <typename IdxT, bool SCAN>
__global__ __launch_bounds__(kRouteThreads) void route_scatter_kernel(
    const IdxT* __restrict__ ids, int64_t R, int64_t R_ids, int E_ids, int E, int chunk, int nb,
    const int32_t* __restrict__ blockoff, int32_t* __restrict__ offsets, int32_t* __restrict__ sorted_rows,
    int32_t* __restrict__ counts, int bm, int32_t* __restrict__ tile_expert, int32_t* __restrict__ tile_mstart,
    int32_t* __restrict__ meta) {
  extern __shared__ int32_t sm[];  // base[E+1], wcnt[4][E+1]; SCAN: s_off[E+2], wsum[4]
  constexpr int NW = kRouteThreads / kWave;
  int32_t* base = sm;
  int32_t* wcnt = sm + (E + 1);
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  const int nbits = 32 - __clz(E);  // bucket values lie in [0, E]
  if constexpr (SCAN) {
    int32_t* s_off = wcnt + NW * (E + 1);
    int32_t* wsum = s_off + (E + 2);
    // Thread t scans buckets 2t and 2t + 1 (E + 1 <= 2 kRouteThreads).
    int32_t tot[2] = {0, 0}, pre[2] = {0, 0};
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int bk = 2 * tid + h;
      if (bk <= E) {
        const int32_t* row = blockoff + (int64_t)bk * nb;
#pragma unroll 8
        for (int b = 0; b < nb; ++b) {
          const int32_t c = row[b];
          tot[h] += c;
          pre[h] += b < (int)blockIdx.x ? c : 0;
        }
      }
    }
    const int32_t start0 = block_excl_scan(tot[0] + tot[1], wsum);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int bk = 2 * tid + h;
      const int32_t start = start0 + (h ? tot[0] : 0);
      if (bk <= E) {
        base[bk] = start + pre[h];
        s_off[bk] = start;
        if (blockIdx.x == 0) {
          offsets[bk] = start;
          if (bk < E) counts[bk] = tot[h];
        }
      }
    }
    if (blockIdx.x == 0) {
      if (tid == 0) s_off[E + 1] = (int32_t)R;
      if (bm > 0) {
        __syncthreads();
        build_tile_table(s_off, E, bm, wsum, tile_expert, tile_mstart, meta);
      }
    }
  } else {
    for (int e = tid; e <= E; e += kRouteThreads) base[e] = offsets[e] + blockoff[(int64_t)e * nb + blockIdx.x];
  }
  const int64_t lo = (int64_t)blockIdx.x * chunk;
  const int64_t hi = std::min<int64_t>(R, lo + chunk);
  const uint64_t lt_mask = (1ull << lane) - 1ull;
  for (int64_t sub = lo; sub < hi; sub += kRouteThreads) {
    for (int i = tid; i < NW * (E + 1); i += kRouteThreads) wcnt[i] = 0;
    __syncthreads();
    const int64_t r = sub + tid;
    const bool valid = r < hi;
    const int e = valid ? bucket_of(ids, r, R_ids, E_ids, E) : 0;
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

// The whole routing sort in one workgroup of kRouteSmallThreads, for small
// problems (R <= kRouteSmallRows, E <= kRouteSmallE): bucket counts, segment
// offsets, the tile table (bm > 0) and the stable scatter of route_count /
// route_scan / route_scatter, without their two launches and the blockcnt
// round trip.  Thread tid owns rows tid + kRouteSmallThreads q (q < PER), so
// row order is (q, wave, lane) order.  Each wave counts, per round q, the
// rows of every bucket in one ballot pass; a wave scan turns each bucket's
// column of (q, wave) counts into exclusive prefixes (their total is the
// bucket count); every row then goes to
//   segment start + rows of its bucket in earlier (q, wave) + rank in wave,
// with no further barrier.
constexpr int kRouteSmallThreads = 1024;
constexpr int64_t kRouteSmallRows = 4096;
constexpr int kRouteSmallE = 256;

template <typename IdxT>
__global__ __launch_bounds__(kRouteSmallThreads) void route_small_kernel(
    const IdxT* __restrict__ ids, int64_t R, int64_t R_ids, int E_ids, int E, int32_t* __restrict__ counts,
    int32_t* __restrict__ offsets, int32_t* __restrict__ sorted_rows, int bm, int32_t* __restrict__ tile_expert,
    int32_t* __restrict__ tile_mstart, int32_t* __restrict__ meta) {
  constexpr int NW = kRouteSmallThreads / kWave;
  constexpr int PER = (int)(kRouteSmallRows / kRouteSmallThreads);
  constexpr int NS = PER * NW;  // (round, wave) segments
  static_assert(kRouteSmallRows % kRouteSmallThreads == 0, "whole rounds of rows");
  static_assert(kRouteSmallRows <= 65535, "prefixes are 16-bit");
  static_assert(kRouteSmallE + 1 <= kRouteSmallThreads, "one thread per bucket");
  static_assert(NS == kWave, "a bucket's segment column is one wave");
  __shared__ int32_t s_off[kRouteSmallE + 2];                 // segment starts
  __shared__ uint16_t segcnt[NS * (kRouteSmallE + 1)];        // [segment][bucket]
  __shared__ int32_t wsum[NW];
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  const int W1 = E + 1;  // buckets: experts, then ids outside [0, E)
  int bk[PER];
#pragma unroll
  for (int q = 0; q < PER; ++q) {
    const int64_t r = tid + (int64_t)kRouteSmallThreads * q;
    bk[q] = r < R ? bucket_of(ids, r, R_ids, E_ids, E) : -1;
  }
  for (int i = tid; i < NS * W1; i += kRouteSmallThreads) segcnt[i] = 0;
  lds_barrier();
  // Lanes holding the same bucket: intersect the ballots of every bit.
  const int nbits = 32 - __clz(E);
  const uint64_t lt_mask = (1ull << lane) - 1ull;
  int rank[PER];
#pragma unroll
  for (int q = 0; q < PER; ++q) {
    rank[q] = 0;
    if ((int64_t)kRouteSmallThreads * q >= R) continue;  // no rows in this round
    const bool valid = bk[q] >= 0;
    const int e = valid ? bk[q] : 0;
    uint64_t match = __ballot(valid);
    for (int b = 0; b < nbits; ++b) {
      const uint64_t bal = __ballot((e >> b) & 1);
      match &= ((e >> b) & 1) ? bal : ~bal;
    }
    rank[q] = __popcll(match & lt_mask);
    if (valid && rank[q] == 0) segcnt[(q * NW + wave) * W1 + e] = (uint16_t)__popcll(match);
  }
  lds_barrier();
  // Wave w scans the columns of buckets w, w + NW, ...: lane = segment.
  for (int e = wave; e < W1; e += NW) {
    const uint32_t c = segcnt[lane * W1 + e];
    const uint32_t incl = wave_incl_scan(c);
    segcnt[lane * W1 + e] = (uint16_t)(incl - c);
    if (lane == kWave - 1) s_off[e] = (int32_t)incl;  // the bucket's count
  }
  lds_barrier();
  const int32_t tot = tid < W1 ? s_off[tid] : 0;
  const int32_t start = block_excl_scan(tot, wsum);
  if (tid < W1) {
    s_off[tid] = start;
    offsets[tid] = start;
    if (tid < E) counts[tid] = tot;
  }
  if (tid == 0) s_off[W1] = (int32_t)R;
  lds_barrier();
  if (bm > 0) build_tile_table(s_off, E, bm, wsum, tile_expert, tile_mstart, meta);
#pragma unroll
  for (int q = 0; q < PER; ++q)
    if (bk[q] >= 0)
      sorted_rows[s_off[bk[q]] + segcnt[(q * NW + wave) * W1 + bk[q]] + rank[q]] =
          (int32_t)(tid + kRouteSmallThreads * q);
}

// ---------------------------------------------------------------------------
// MFMA grouped GEMM.
// ---------------------------------------------------------------------------
constexpr int kMinBM = 64;  // smallest M tile of any configuration (workspace sizing)

using CfgHuge = GemmCfg<256, 256, 2, 4, 64, 2, 1>;   // 8 waves of 128x64, 128 KB LDS, 1 per CU
using CfgLarge = GemmCfg<128, 256, 2, 2, 32, 2, 2>;  // 4 waves of 64x128,  48 KB LDS, 2 per CU
using CfgSmall = GemmCfg<64, 128, 2, 2, 64, 3, 2>;   // 4 waves of 32x64,   72 KB LDS, 2 per CU
using CfgShort = GemmCfg<128, 256, 2, 4, 64, 3, 1>;  // 8 waves of 64x64, 144 KB LDS: short tiles beside CfgHuge
template <typename C> struct TypeC { using type = C; };

// One output tile: rows m0 .. min(m0 + BM, mend) of expert e's segment,
// output columns n0 .. n0 + OBN.  PREFILLED: the caller has put the tile's
// routed rows in srow (-1 past the segment); m0 .. mend only bounds their
// count.
// EPI 0: Y = X W^T.  EPI 1 (SwiGLU): Y = silu(X Wg^T) * (X Wu^T) with W = Wg and
// W2 = Wu, both [E, I, H]; a tile then covers BN/2 output columns, its even
// 32-column blocks holding gate rows and its odd blocks the up rows of the
// same output columns, so a lane holds both factors of each output element.
// A K split of one output tile (gemm_tile with SPLIT): this workgroup
// computes k in [kb, ke) only, publishes its fp32 partial tile, and the last
// of the S workgroups of the tile to count in sums the S partials in split
// order (so the result does not depend on which finished last) and stores
// the tile.  cnt[tile] is zero before and after.
// pt: the threads that publish partials, the first pt of the workgroup
// (all, or with at most 32 rows per tile the waves of the first 32-row
// block: the others hold zeros).  nv: accumulators published per 32x32
// block, the template's SPLITNV (accumulator v of a lane holds row
// 8 (v / 4) + 4 (lane / 32) + v % 4, so with at most 8 m rows per tile only
// v < 4 m can be non-zero).
struct SplitK {
  float* part;
  uint32_t* cnt;
  int tile, sk, S, pt;
  int64_t kb, ke;
};

template <typename T, typename Cfg, int MODE, int EPI, bool PREFILLED = false, int SPLITNV = 0>
__device__ __attribute__((always_inline)) inline void gemm_tile(uint16_t* smem, int32_t* srow, const uint16_t* __restrict__ X,
                                 const uint16_t* __restrict__ W, const uint16_t* __restrict__ W2,
                                 const uint16_t* __restrict__ Wx, const uint16_t* __restrict__ W2x,
                                 uint16_t* __restrict__ Y, int64_t H, int64_t I, int topk, int64_t R_ids, int E_ids,
                                 int64_t x_shift, const int32_t* __restrict__ sorted_rows, int e, int m0, int mend,
                                 int n0, const SplitK* sp = nullptr) {
  constexpr int BM = Cfg::BM;
  static_assert(EPI == 0 || Cfg::FN % 2 == 0, "SwiGLU pairs 32-column blocks within a wave");
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;
  if constexpr (!PREFILLED)
    for (int r = tid; r < BM; r += Cfg::THREADS) srow[r] = (m0 + r < mend) ? sorted_rows[m0 + r] : -1;
  // Expert e < E_ids reads W[e] (and W2[e]); the appended expert E_ids reads
  // Wx (and W2x).  X row of routed row r: r / topk for r < R_ids, else
  // r - R_ids + x_shift.
  const uint16_t* We = e < E_ids ? W + (int64_t)e * I * H : Wx;
  const uint16_t* W2e = e < E_ids ? W2 + (int64_t)e * I * H : W2x;
  __syncthreads();

  // Copy plan: instruction i of wave v covers tile rows RPI*(v*INS + i) ..;
  // lane l fills slot l: row l / CPR, position l % CPR.
  constexpr int CPR = Cfg::CPR;
  const int crow = lane / CPR;
  // Row offsets in 16-byte chunks (H is a multiple of 8; the host checks
  // that X and one expert's weights span fewer than 2^32 chunks).
  RowOffs<Cfg::A_INS> a_src;
  a_src.base = X;
  using BSrc = std::conditional_t<EPI == 0, RowOffs<Cfg::B_INS>, const uint16_t* [Cfg::B_INS]>;
  BSrc b_src;
  const int64_t hc = H / 8;
#pragma unroll
  for (int i = 0; i < Cfg::A_INS; ++i) {
    const int r = Cfg::RPI * (wave * Cfg::A_INS + i) + crow;
    const int sr = srow[r];
    // Rows past the expert's segment read X row 0; their results are never stored.
    const int64_t xr = sr < 0 ? 0 : (sr < R_ids ? sr / topk : sr - R_ids + x_shift);
    a_src.o[i] = (uint32_t)(xr * hc + Cfg::copy_chunk(wave, i, Cfg::A_INS, lane));
  }
  if constexpr (EPI == 0) b_src.base = We;
#pragma unroll
  for (int i = 0; i < Cfg::B_INS; ++i) {
    const int nl = Cfg::RPI * (wave * Cfg::B_INS + i) + crow;  // tile row
    if constexpr (EPI == 0) {
      const int64_t n = n0 + nl;
      b_src.o[i] = (uint32_t)((n < I ? n : 0) * hc + Cfg::copy_chunk(wave, i, Cfg::B_INS, lane));
    } else {
      const int blk = nl / 32;
      const int64_t n = n0 + (blk >> 1) * 32 + (nl & 31);
      b_src[i] = ((blk & 1) ? W2e : We) + (n < I ? n : 0) * H + Cfg::copy_chunk(wave, i, Cfg::B_INS, lane) * 8;
    }
  }
  const int wm = wave / Cfg::WN, wn = wave % Cfg::WN;
  // 32-row blocks of this wave that hold routed rows (wave-uniform): the
  // MFMAs of the others are skipped, so a tile costs MFMA time in
  // proportion to its rows, rounded up to 32.
  const int mcount = min(BM, mend - m0);
  const int fm_act = __builtin_amdgcn_readfirstlane(min(Cfg::FM, max(0, (mcount - wm * Cfg::FM * 32 + 31) / 32)));
  f32x16 acc[Cfg::FM][Cfg::FN];
#pragma unroll
  for (int i = 0; i < Cfg::FM; ++i)
#pragma unroll
    for (int j = 0; j < Cfg::FN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  if constexpr (SPLITNV > 0) {
    tile_mainloop<T, Cfg, MODE>(smem, a_src, b_src, sp->kb, sp->ke, fm_act, acc);
    // Publish the partial with agent-scope stores (they reach memory past
    // this XCD's L2), wait for them, then count in.  No fence: only the
    // counting workgroup reads them, after its count.
    constexpr int NV = Cfg::FM * Cfg::FN * 16;
    // Element u of thread t at [(tile * S + split) * NV + u][t]: a wave's
    // stores and loads of one element are contiguous.
    const int pt = sp->pt;
    constexpr int nv = SPLITNV;
    constexpr int NP = Cfg::FM * Cfg::FN * nv;  // published values per thread
    if (tid < pt) {
      float* mine = sp->part + (size_t)(sp->tile * sp->S + sp->sk) * NP * pt + tid;
#pragma unroll
      for (int i = 0; i < Cfg::FM; ++i)
#pragma unroll
        for (int j = 0; j < Cfg::FN; ++j)
#pragma unroll
          for (int v = 0; v < 16; ++v)
            if (v < nv)
              __hip_atomic_store(mine + ((i * Cfg::FN + j) * nv + v) * pt, acc[i][j][v], __ATOMIC_RELAXED,
                                 __HIP_MEMORY_SCOPE_AGENT);
    }
    __builtin_amdgcn_s_waitcnt(0);  // every counter, vmcnt included
    __syncthreads();
    __shared__ int s_last;
    if (tid == 0)
      s_last = __hip_atomic_fetch_add(sp->cnt + sp->tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
               (uint32_t)(sp->S - 1);
    __syncthreads();
    if (!s_last) return;
    // Sum the S partials in split order (this workgroup's own from
    // registers): each split's values are loaded together, then added.
    f32x16 sum[Cfg::FM][Cfg::FN];
#pragma unroll
    for (int i = 0; i < Cfg::FM; ++i)
#pragma unroll
      for (int j = 0; j < Cfg::FN; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) sum[i][j][v] = 0.0f;
    for (int q = 0; q < sp->S && tid < pt; ++q) {
      if (q == sp->sk) {
#pragma unroll
        for (int i = 0; i < Cfg::FM; ++i)
#pragma unroll
          for (int j = 0; j < Cfg::FN; ++j) sum[i][j] += acc[i][j];
        continue;
      }
      const float* pq = sp->part + (size_t)(sp->tile * sp->S + q) * NP * pt + tid;
      float buf[NV];
#pragma unroll
      for (int i = 0; i < Cfg::FM; ++i)
#pragma unroll
        for (int j = 0; j < Cfg::FN; ++j)
#pragma unroll
          for (int v = 0; v < 16; ++v)
            buf[(i * Cfg::FN + j) * 16 + v] =
                v < nv ? __hip_atomic_load(pq + ((i * Cfg::FN + j) * nv + v) * pt, __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT)
                       : 0.0f;
#pragma unroll
      for (int i = 0; i < Cfg::FM; ++i)
#pragma unroll
        for (int j = 0; j < Cfg::FN; ++j)
#pragma unroll
          for (int v = 0; v < 16; ++v) sum[i][j][v] += buf[(i * Cfg::FN + j) * 16 + v];
    }
#pragma unroll
    for (int i = 0; i < Cfg::FM; ++i)
#pragma unroll
      for (int j = 0; j < Cfg::FN; ++j) acc[i][j] = sum[i][j];
    if (tid == 0) __hip_atomic_store(sp->cnt + sp->tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  } else {
    tile_mainloop<T, Cfg, MODE>(smem, a_src, b_src, 0, H, fm_act, acc);
  }

  // Epilogue: accumulator v of lane l holds row 8*(v/4) + 4*(l/32) + v%4,
  // column l%32 of its 32x32 block.  Rows go back to their routed position.
#pragma unroll
  for (int i = 0; i < Cfg::FM; ++i) {
    if (i >= fm_act) continue;
    int sr[16];  // routed rows of this lane's 16 accumulator rows, 4 per LDS read
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int4 q = *reinterpret_cast<const int4*>(srow + (wm * Cfg::FM + i) * 32 + g * 8 + (lane >> 5) * 4);
      sr[4 * g] = q.x; sr[4 * g + 1] = q.y; sr[4 * g + 2] = q.z; sr[4 * g + 3] = q.w;
    }
    if constexpr (EPI == 0) {
#pragma unroll
      for (int j = 0; j < Cfg::FN; ++j) {
        const int64_t col = n0 + (wn * Cfg::FN + j) * 32 + (lane & 31);
#pragma unroll
        for (int v = 0; v < 16; ++v)
          if (sr[v] >= 0 && col < I) Y[(int64_t)sr[v] * I + col] = MfmaOp<T>::cvt(acc[i][j][v]);
      }
    } else {
      // Blocks 2m (gate) and 2m+1 (up) of the tile hold output block m.
#pragma unroll
      for (int j = 0; j < Cfg::FN; j += 2) {
        const int64_t col = n0 + ((wn * Cfg::FN + j) >> 1) * 32 + (lane & 31);
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const float g = acc[i][j][v], u = acc[i][j + 1][v];
          if (sr[v] >= 0 && col < I) Y[(int64_t)sr[v] * I + col] = MfmaOp<T>::cvt(g / (1.0f + expf(-g)) * u);
        }
      }
    }
  }
}

// Grouped GEMM with each tile split along K over S workgroups, for problems
// whose tiles would leave most CUs idle (a few routed rows: decode).  Items
// 0 .. n_tiles * S - 1 are (tile, split) pairs, tile-major; the items after
// them zero the rows whose expert id is invalid, as in the persistent kernel.
template <typename T, typename Cfg, int EPI, int NVP>
__global__ __launch_bounds__(Cfg::THREADS, Cfg::MINB) void grouped_gemm_splitk_kernel(
    const uint16_t* __restrict__ X, const uint16_t* __restrict__ W, const uint16_t* __restrict__ W2,
    uint16_t* __restrict__ Y, int64_t H, int64_t I, int topk, int64_t R, int E, int ntn, int S, int tiles_ub,
    int64_t kchunk, int pt, const int32_t* __restrict__ sorted_rows, const int32_t* __restrict__ offsets,
    const int32_t* __restrict__ tile_expert, const int32_t* __restrict__ tile_mstart,
    const int32_t* __restrict__ meta, float* __restrict__ part, uint32_t* __restrict__ cnt) {
  constexpr int BM = Cfg::BM;
  constexpr int OBN = EPI == 1 ? Cfg::BN / 2 : Cfg::BN;
  extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
  __shared__ __attribute__((aligned(16))) int32_t srow[BM];
  const int tid = threadIdx.x;
  const int w = (int)blockIdx.x;
  const int n_tiles = meta[0] * ntn;
  if (w >= tiles_ub * S) {
    // Zero the rows past offsets[E] (invalid ids), BM rows x OBN columns per item.
    const int z = w - tiles_ub * S;
    const int64_t z0 = (int64_t)offsets[E] + (int64_t)(z / ntn) * BM;
    const int n0z = (z % ntn) * OBN;
    for (int i = tid; i < BM * OBN; i += Cfg::THREADS) {
      const int64_t p = z0 + i / OBN;
      const int64_t col = n0z + i % OBN;
      if (p < R && col < I) Y[(int64_t)sorted_rows[p] * I + col] = 0;
    }
    return;
  }
  const int tile = w / S, sk = w % S;
  if (tile >= n_tiles) return;  // the grid covers an upper bound on the tiles
  const int mt = tile / ntn, nt = tile % ntn;
  const int e = tile_expert[mt];
  const int m0 = tile_mstart[mt];
  SplitK sp{part, cnt, tile, sk, S, pt, (int64_t)sk * kchunk, min(H, (int64_t)(sk + 1) * kchunk)};
  gemm_tile<T, Cfg, 0, EPI, false, NVP>(smem, srow, X, W, W2, nullptr, nullptr, Y, H, I, topk, R, E, 0, sorted_rows,
                                          e, m0, offsets[e + 1], nt * OBN, &sp);
}

// The K-split GEMM for at most 64 routed rows without a routing sort:
// every workgroup's first wave reads the ids (one row per lane) and groups
// the rows by bucket in ascending bucket order (wave min, ballot); group g
// with bucket e < E is expert e's one M tile, its rows in ascending order,
// and the tiles are the groups in order times the N tiles.  Items are as in
// grouped_gemm_splitk_kernel; one more workgroup (the last) writes the
// routing sort's tables for calls that reuse this routing.
template <typename T, typename Cfg, typename IdxT, int EPI, int NVP>
__global__ __launch_bounds__(Cfg::THREADS, Cfg::MINB) void grouped_gemm_splitk_self_kernel(
    const uint16_t* __restrict__ X, const uint16_t* __restrict__ W, const uint16_t* __restrict__ W2,
    uint16_t* __restrict__ Y, int64_t H, int64_t I, int topk, int R, int E, int ntn, int S, int tiles_ub,
    int64_t kchunk, int pt, const IdxT* __restrict__ ids, int32_t* __restrict__ counts,
    int32_t* __restrict__ offsets, int32_t* __restrict__ sorted_rows, int bm, int32_t* __restrict__ tile_expert,
    int32_t* __restrict__ tile_mstart, int32_t* __restrict__ meta, float* __restrict__ part,
    uint32_t* __restrict__ cnt) {
  constexpr int BM = Cfg::BM;
  static_assert(BM >= kWave, "a group's rows fit one M tile");
  constexpr int OBN = EPI == 1 ? Cfg::BN / 2 : Cfg::BN;
  extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
  __shared__ __attribute__((aligned(16))) int32_t srow[BM];
  __shared__ int32_t g_bucket[kWave];
  __shared__ uint64_t g_mask[kWave];
  __shared__ int32_t s_ng;
  const int tid = threadIdx.x;
  const int w = (int)blockIdx.x;
  if (tid < kWave) {
    int b = -1;
    if (tid < R) {
      const IdxT v = ids[tid];
      b = (v >= 0 && v < (IdxT)E) ? (int)v : E;
    }
    uint64_t active = __ballot(b >= 0);
    int ng = 0;
    while (active) {
      const uint32_t key = ((active >> tid) & 1ull) ? ~(uint32_t)b : 0u;
      const int bv = (int)~wave_max_u32(key);  // the smallest bucket left
      const uint64_t m = __ballot(b == bv) & active;
      if (tid == 0) {
        g_bucket[ng] = bv;
        g_mask[ng] = m;
      }
      active &= ~m;
      ++ng;
    }
    if (tid == 0) s_ng = ng;
  }
  __syncthreads();
  const int ng = s_ng;
  const bool has_bad = ng > 0 && g_bucket[ng - 1] == E;
  const int n_exp = ng - (has_bad ? 1 : 0);

  if (w == (int)gridDim.x - 1) {
    // The routing sort's tables: segment starts, counts, sorted rows (each
    // group's rows in order at its segment) and the M-tile table.
    // s_off in the pipeline's LDS (this workgroup runs no tile), which keeps
    // the kernel's static LDS small enough for two workgroups per CU.
    static_assert((kMaxExperts + 2) * 4 <= (int)Cfg::LDS_BYTES, "segment starts fit the stages");
    int32_t* s_off = reinterpret_cast<int32_t*>(smem);
    __shared__ int32_t wsum[Cfg::THREADS / kWave];
    for (int e = tid; e <= E; e += Cfg::THREADS) {
      int32_t st = 0;
      for (int g = 0; g < ng; ++g) st += g_bucket[g] < e ? __popcll(g_mask[g]) : 0;
      s_off[e] = st;
      offsets[e] = st;
    }
    if (tid == 0) s_off[E + 1] = R;
    __syncthreads();
    for (int e = tid; e < E; e += Cfg::THREADS) counts[e] = s_off[e + 1] - s_off[e];
    if (tid < kWave)
      for (int g = 0; g < ng; ++g) {
        const uint64_t m = g_mask[g];
        if ((m >> tid) & 1ull) sorted_rows[s_off[g_bucket[g]] + __popcll(m & ((1ull << tid) - 1ull))] = tid;
      }
    build_tile_table(s_off, E, bm, wsum, tile_expert, tile_mstart, meta);
    return;
  }
  if (w >= tiles_ub * S) {
    // Rows whose id is invalid (the last group): zeros, OBN columns per item.
    if (!has_bad) return;
    const uint64_t m = g_mask[ng - 1];
    const int n0z = (w - tiles_ub * S) * OBN;
    for (int i = tid; i < kWave * OBN; i += Cfg::THREADS) {
      const int r = i / OBN;
      const int64_t col = n0z + i % OBN;
      if (((m >> r) & 1ull) && col < I) Y[(int64_t)r * I + col] = 0;
    }
    return;
  }
  const int tile = w / S, sk = w % S;
  const int gi = tile / ntn, nt = tile % ntn;
  if (gi >= n_exp) return;  // the grid covers an upper bound on the tiles
  const uint64_t m = g_mask[gi];
  for (int r = tid; r < BM; r += Cfg::THREADS) srow[r] = -1;
  __syncthreads();
  if (tid < kWave && ((m >> tid) & 1ull)) srow[__popcll(m & ((1ull << tid) - 1ull))] = tid;
  SplitK sp{part, cnt, tile, sk, S, pt, (int64_t)sk * kchunk, min(H, (int64_t)(sk + 1) * kchunk)};
  gemm_tile<T, Cfg, 0, EPI, true, NVP>(smem, srow, X, W, W2, nullptr, nullptr, Y, H, I, topk, R, E, 0, nullptr,
                                        g_bucket[gi], 0, __popcll(m), nt * OBN, &sp);
}

// The persistent grouped GEMM over the tile table.  Tiles of Cfg's height,
// and, when CfgS is not void, short tiles (kShortTile) of CfgS's height:
// the tile table gives experts with at most CfgS::BM rows one short tile,
// whose three-stage pipeline keeps twice the weight bytes in flight of the
// tall tiles' two stages.  Both share the N tiling, the workgroup size and
// one LDS buffer.
template <typename T, typename Cfg, typename CfgS, int MODE = 0, int EPI = 0>  // MODE: tuning builds only (1 = copies only, 2 = MFMA only)
__global__ __launch_bounds__(Cfg::THREADS, Cfg::MINB) void grouped_gemm_kernel(
    const uint16_t* __restrict__ X, const uint16_t* __restrict__ W, const uint16_t* __restrict__ W2,
    const uint16_t* __restrict__ Wx, const uint16_t* __restrict__ W2x, uint16_t* __restrict__ Y,
    int64_t H, int64_t I, int topk, int64_t R, int E, int ntn, int64_t R_ids, int E_ids, int64_t x_shift,
    const int32_t* __restrict__ sorted_rows, const int32_t* __restrict__ offsets,
    const int32_t* __restrict__ tile_expert, const int32_t* __restrict__ tile_mstart,
    const int32_t* __restrict__ meta, uint32_t* __restrict__ sched) {
  constexpr bool MIXED = !std::is_void<CfgS>::value;
  using CS = typename std::conditional<MIXED, CfgS, Cfg>::type;
  static_assert(CS::THREADS == Cfg::THREADS && CS::BN == Cfg::BN && CS::MINB == Cfg::MINB,
                "tile configurations of one kernel share threads, N tiling and occupancy");
  constexpr int BM = Cfg::BM, BN = Cfg::BN;
  constexpr int OBN = EPI == 1 ? BN / 2 : BN;  // output columns per tile
  extern __shared__ __attribute__((aligned(16))) uint16_t smem[];  // [S][(BM+BN)*BK] of either configuration
  __shared__ __attribute__((aligned(16))) int32_t srow[BM > CS::BM ? BM : CS::BM];

  const int tid = threadIdx.x;

  // Work list and its order.  The grid is persistent: gridDim.x = 8 * SUPER
  // workgroups, SUPER per XCD (the hardware deals consecutive workgroups
  // round-robin over the 8 XCDs, so workgroup b runs on XCD b % 8).  Work is
  // cut into super-tiles of SUPER items, SM M tiles x SN N tiles; in round i
  // XCD x processes super-tile 8i + x, one item per workgroup.  The SN N
  // tiles of an M tile share its gathered X rows and the SM M tiles of one
  // expert share its weight slices in that XCD's L2, at the same K position,
  // so a hot expert's weights are read from HBM about ceil(M_e / (SM*BM))
  // times instead of once per M tile.  The tiles that zero rows whose
  // expert id lies outside [0, E) follow the super-tiles.
  constexpr int SUPER = Cfg::SUPER;
  const int SN = min(ntn, Cfg::SN_MAX);
  const int SM = SUPER / SN;
  const int NG = (ntn + SN - 1) / SN;
  const int n_tiles = meta[0];
  const int n_super_raw = (n_tiles + SM - 1) / SM * NG * SUPER;
  // Super-tile order needs the persistent grid and enough super-tiles to
  // keep every XCD busy for a few rounds.
  const bool by_super_raw = gridDim.x == 8 * SUPER && n_super_raw / SUPER >= 16;
  // Length of the tile part of the list: padded to whole super-tiles when
  // ordered by super-tile, exact otherwise.
  const int n_super_items = by_super_raw ? n_super_raw : n_tiles * ntn;
  const int64_t n_bad = R - offsets[E];
  const int n_zero = (int)((n_bad + BM - 1) / BM) * ntn;
  const int total = n_super_items + n_zero;
  // Otherwise (small problems) each XCD takes one contiguous eighth of the
  // list, its gridDim.x / 8 workgroups walking it in strides.
  //
  // In super-tile order with two tile heights the items are handed out
  // dynamically: XCD x's queue holds super-tiles x, x + 8, ... in order,
  // its workgroups take the next item from it with an atomic counter
  // (sched[x]), and a workgroup whose queue is empty takes items from the
  // other XCDs' queues.  Items differ in cost (tall tiles take about twice
  // as long as short ones, which come last), so a static assignment left
  // the last workgroups finishing hundreds of microseconds after the
  // first.  The counters live in the workspace's control block: the last
  // workgroup to finish (sched[8]) sets them back to zero.
  const bool by_super = by_super_raw;
  const bool dynamic = MIXED && by_super;  // items of one height cost alike: static order
  const int xcd = blockIdx.x & 7, slot = blockIdx.x >> 3;
  const int share = (total + 7) >> 3;
  int w = dynamic ? -1 : by_super ? xcd * SUPER + slot : xcd * share + slot;
  const int w_end = by_super ? total : min(total, (xcd + 1) * share);
  const int step = dynamic ? 0 : by_super ? (int)gridDim.x : (int)(gridDim.x >> 3);
  __shared__ int s_item;
  int q = xcd;  // thread 0: the queue it drains
  // Position p of XCD queue qq: item p % SUPER of super-tile 8 (p / SUPER) + qq.
  auto item_of = [&](uint32_t p, int qq) -> int {
    const int64_t cand = ((int64_t)(p / SUPER) * 8 + qq) * SUPER + p % SUPER;
    return cand < total ? (int)cand : -1;
  };
  for (;; w += step) {
    __syncthreads();  // the previous tile's LDS reads (and s_item reads) are done
    if (dynamic) {
      if (tid == 0) {
        int item = item_of(atomicAdd(&sched[q], 1u), q);
        for (int tried = 1; tried < 8 && item < 0; ++tried) {
          q = (q + 1) & 7;  // queue q is empty: take from the next XCD's queue
          item = item_of(atomicAdd(&sched[q], 1u), q);
        }
        s_item = item;
      }
      __syncthreads();
      w = s_item;
      if (w < 0) break;
    } else if (w >= w_end) {
      break;
    }
    if (w >= n_super_items) {
      const int z = w - n_super_items;
      const int64_t z0 = (int64_t)offsets[E] + (int64_t)(z / ntn) * BM;
      const int n0z = (z % ntn) * OBN;
      for (int i = tid; i < BM * OBN; i += Cfg::THREADS) {
        const int64_t p = z0 + i / OBN;
        const int64_t col = n0z + i % OBN;
        if (p < R && col < I) Y[(int64_t)sorted_rows[p] * I + col] = 0;
      }
      continue;
    }
    int mt, nt;
    if (by_super) {
      const int sup = w / SUPER, within = w % SUPER;
      mt = (sup / NG) * SM + within / SN;
      nt = (sup % NG) * SN + within % SN;
    } else {
      mt = w / ntn;  // list order M-major
      nt = w % ntn;
    }
    if (mt >= n_tiles || nt >= ntn) continue;
    const int te = tile_expert[mt];
    if (te < 0) continue;  // a hole of an interleaved table
    const int e = te & ~kShortTile;
    const int m0 = tile_mstart[mt];
    const int mend = offsets[e + 1];
    if (MIXED && (te & kShortTile))
      gemm_tile<T, CS, MODE, EPI>(smem, srow, X, W, W2, Wx, W2x, Y, H, I, topk, R_ids, E_ids, x_shift,
                                     sorted_rows, e, m0, mend, nt * OBN);
    else
      gemm_tile<T, Cfg, MODE, EPI>(smem, srow, X, W, W2, Wx, W2x, Y, H, I, topk, R_ids, E_ids, x_shift,
                                        sorted_rows, e, m0, mend, nt * OBN);
  }  // tile loop
  if (dynamic && tid == 0 && atomicAdd(&sched[8], 1u) == gridDim.x - 1) {
    // Every workgroup has found every queue empty: no counter is read again.
#pragma unroll
    for (int i = 0; i <= 8; ++i) sched[i] = 0;
  }
}

// ---------------------------------------------------------------------------
// Self-routing grouped GEMM for small routings: R <= kSelfRows routed rows
// and E <= kSelfMaxE experts, in one launch instead of the routing sort's
// launches followed by the GEMM's.
//
// Every workgroup reads all R expert ids (coalesced: thread t holds the ids
// of rows (q * 256 + t) * VEC .. + VEC - 1 of load round q, 4 bits each) and
// derives what the sort would hand it: the per-expert row counts (hence the
// M-tile list, experts in order, then the tiles of rows whose id is
// invalid) and its own tile's rows.  Those are expert e's rows ranked in
// (thread, slot) order: the block-exclusive prefix of the per-thread counts
// of e plus the count of e in the thread's earlier slots.  Every workgroup
// ranks alike, so the M tiles of e partition its rows; a row's result does
// not depend on which tile holds it, so the output is bitwise that of the
// sorted path.  Per-thread counts (at most kSelfPer = 32) are formed by SWAR
// over the packed buckets; the wave and block sums are 16-bit fields, two
// buckets per 32-bit word (R <= 8192), so one 32-bit wave scan serves two
// buckets and never carries from one into the other.
//
// One extra workgroup (the last) writes the routing tables that the sort
// would have written (counts, offsets, sorted_rows in stable row order, the
// M-tile table), so a later call that reuses this workspace's routing finds
// them; it holds rows t * kSelfPer .. t * kSelfPer + kSelfPer - 1 per thread,
// which makes that order the (thread, slot) order.
// ---------------------------------------------------------------------------
constexpr int kSelfPer = 32;
constexpr int64_t kSelfRows = 8192;  // CfgSmall's 256 threads x kSelfPer
constexpr int kSelfMaxE = 14;  // buckets 0 .. E (E = invalid ids); 15 marks "no row"

// Adds one to 8-bit field b of the pair (lo: buckets 0-7, hi: 8-14; 15 is
// not counted).
__device__ inline void self_count(uint64_t& lo, uint64_t& hi, uint32_t b) {
  const uint64_t inc = (uint64_t)1 << ((b & 7) * 8);
  lo += b < 8 ? inc : 0;
  hi += (b >= 8 && b < 15) ? inc : 0;
}

__device__ inline uint32_t self_bucket(int64_t v, int E) { return (uint64_t)v < (uint64_t)E ? (uint32_t)v : (uint32_t)E; }
__device__ inline uint32_t self_bucket(int32_t v, int E) { return (uint32_t)v < (uint32_t)E ? (uint32_t)v : (uint32_t)E; }

// Count of bucket b among the 32 nibbles of pk.  After the XOR a nibble
// equal to b is zero; adding 7 to the low three bits of a nibble sets its
// bit 3 unless they are all zero, so bit 3 of the complement flags exactly
// the zero nibbles.
template <int P>
__device__ inline uint32_t self_count_of(const uint32_t (&pk)[P / 8], uint32_t b) {
  const uint32_t pat = 0x11111111u * b;
  uint32_t c = 0;
#pragma unroll
  for (int j = 0; j < P / 8; ++j) {
    const uint32_t x = pk[j] ^ pat;
    const uint32_t z = ~(((x & 0x77777777u) + 0x77777777u) | x | 0x77777777u);
    c += (uint32_t)__builtin_popcount(z);
  }
  return c;
}

// Buckets of kSelfPer rows of this thread, 4 bits each (15: past R).  Slot
// s = q * VEC + v (VEC ids per 16-byte load) holds row
//   (q * NT + tid) * VEC + v    when STRIDED (a wave's loads are contiguous),
//   tid * kSelfPer + s          otherwise (a thread's rows are contiguous).
template <bool STRIDED, int NT, int P, typename IdxT>
__device__ inline void self_load(const IdxT* __restrict__ ids, int R, int E, int tid, uint32_t (&pk)[P / 8]) {
  constexpr int VEC = 16 / (int)sizeof(IdxT);
  constexpr int NQ = P / VEC;
  static_assert(P % VEC == 0 && P % 8 == 0, "whole loads and bucket words");
#pragma unroll
  for (int j = 0; j < P / 8; ++j) pk[j] = 0;
  u32x4 v[NQ];
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    const int base = STRIDED ? (q * NT + tid) * VEC : tid * P + q * VEC;
    if (base + VEC <= R) {
      v[q] = *reinterpret_cast<const u32x4*>(ids + base);
    } else {
      // The last partial load: ids past R read as -1 (never counted below).
#pragma unroll
      for (int i = 0; i < 4; ++i) v[q][i] = 0xFFFFFFFFu;
#pragma unroll
      for (int i = 0; i < VEC; ++i)
        if (base + i < R) {
          const IdxT id = ids[base + i];
          if constexpr (sizeof(IdxT) == 8) {
            v[q][2 * i] = (uint32_t)(uint64_t)id;
            v[q][2 * i + 1] = (uint32_t)((uint64_t)id >> 32);
          } else {
            v[q][i] = (uint32_t)id;
          }
        }
    }
  }
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    const int base = STRIDED ? (q * NT + tid) * VEC : tid * P + q * VEC;
#pragma unroll
    for (int i = 0; i < VEC; ++i) {
      const int sl = q * VEC + i;
      IdxT id;
      if constexpr (sizeof(IdxT) == 8)
        id = (IdxT)(((uint64_t)v[q][2 * i + 1] << 32) | v[q][2 * i]);
      else
        id = (IdxT)v[q][i];
      const uint32_t b = base + i < R ? self_bucket(id, E) : 15u;
      pk[sl / 8] |= b << ((sl % 8) * 4);
    }
  }
}

template <typename T, typename Cfg, typename IdxT, int EPI, int PER>
__global__ __launch_bounds__(Cfg::THREADS, Cfg::MINB) void grouped_gemm_selfroute_kernel(
    const uint16_t* __restrict__ X, const uint16_t* __restrict__ W, const uint16_t* __restrict__ W2,
    uint16_t* __restrict__ Y, int64_t H, int64_t I, int topk, int R, int E, int ntn, int share,
    const IdxT* __restrict__ ids, int32_t* __restrict__ counts, int32_t* __restrict__ offsets,
    int32_t* __restrict__ sorted_rows, int bm, int32_t* __restrict__ tile_expert,
    int32_t* __restrict__ tile_mstart, int32_t* __restrict__ meta) {
  constexpr int BM = Cfg::BM, NT = Cfg::THREADS, NW = NT / kWave;
  // Tile workgroups load 32 ids per thread with coalesced (strided) loads;
  // with 8 per thread each thread's rows are contiguous, so that a tile's
  // rows are consecutive rows of its expert, as in the sorted path.
  constexpr bool STRIDED = PER > 8;
  constexpr int OBN = EPI == 1 ? Cfg::BN / 2 : Cfg::BN;
  constexpr int VEC = 16 / (int)sizeof(IdxT);
  constexpr int NQ = PER / VEC;
  extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
  __shared__ __attribute__((aligned(16))) int32_t srow[BM];
  __shared__ uint32_t wtot[NW][8];
  __shared__ uint32_t s_tot[8];
  __shared__ int32_t s_off[kSelfMaxE + 3];
  __shared__ int32_t wsum[NW];
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  const bool writer = (int)blockIdx.x == 8 * share;
  // Work item of this workgroup: XCD x takes items x * share .. x * share +
  // share - 1 (the hardware deals workgroups round-robin over the 8 XCDs),
  // so the M tiles of one expert share its weights in one L2.
  const int w = (int)(blockIdx.x & 7) * share + (int)(blockIdx.x >> 3);

  uint32_t pk[PER / 8];
  if (writer)
    self_load<false, NT, PER>(ids, R, E, tid, pk);
  else
    self_load<STRIDED, NT, PER>(ids, R, E, tid, pk);
  // Per-bucket counts of this thread's rows in 16-bit fields: word k holds
  // buckets 2k and 2k + 1.
  uint32_t own[8], pre[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    own[k] = 0;
    if (2 * k <= E) own[k] = self_count_of<PER>(pk, 2 * k);
    if (2 * k + 1 <= E) own[k] |= self_count_of<PER>(pk, 2 * k + 1) << 16;
  }
  // Words past bucket E are never read: their scans are skipped.
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    if (2 * k > E) break;
    const uint32_t incl = wave_incl_scan(own[k]);
    pre[k] = incl - own[k];
    if (lane == kWave - 1) wtot[wave][k] = incl;
  }
  lds_barrier();
  // Block totals (and, in the writer, the per-thread prefixes) go to LDS,
  // where a bucket's field is read with a computed address: a register
  // array indexed by bucket would be placed in scratch memory.  The
  // prefixes use the pipeline's stages, free until the tile starts.
  uint32_t* s_pre = reinterpret_cast<uint32_t*>(smem);  // [8][NT]
  static_assert(8 * NT * 4 <= BM * Cfg::BK * 2, "prefixes fit stage 0's A rows");
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    if (2 * k > E) break;
    uint32_t t = 0;
#pragma unroll
    for (int v = 0; v < NW; ++v) {
      const uint32_t s = wtot[v][k];
      pre[k] += v < wave ? s : 0u;
      t += s;
    }
    s_pre[k * NT + tid] = pre[k];
    if (tid == 0) s_tot[k] = t;
  }
  lds_barrier();
  auto field = [](uint32_t word, int b) { return (int)((word >> ((b & 1) * 16)) & 0xFFFFu); };
  auto total = [&](int b) { return field(s_tot[b >> 1], b); };
  auto prefix = [&](int b) { return field(s_pre[(b >> 1) * NT + tid], b); };
  auto nib = [&](int sl) { return (int)((pk[sl / 8] >> ((sl % 8) * 4)) & 15u); };

  if (writer) {
    // The tables of the routing sort, for calls that reuse this routing.
    // Thread t holds rows t * PER .. t * PER + PER - 1 here, so a row's
    // place is its bucket's start + the thread's prefix + the count of the
    // bucket earlier in the thread's rows.
    if (tid <= E + 1) {
      int32_t start = 0;
      for (int b = 0; b < tid && b <= E; ++b) start += total(b);
      s_off[tid] = tid == E + 1 ? R : start;
      if (tid <= E) offsets[tid] = start;
      if (tid < E) counts[tid] = total(tid);
    }
    lds_barrier();
    build_tile_table(s_off, E, bm, wsum, tile_expert, tile_mstart, meta);
    uint64_t rlo = 0, rhi = 0;  // running per-bucket counts of this thread's rows
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      const uint32_t b = (uint32_t)nib(q);
      if (b != 15u) {
        const uint32_t run = (uint32_t)(((b < 8 ? rlo : rhi) >> ((b & 7) * 8)) & 0xFFu);
        sorted_rows[s_off[b] + prefix((int)b) + (int32_t)run] = tid * PER + q;
      }
      self_count(rlo, rhi, b);
    }
    return;
  }

  // This workgroup's tile: M tile mt of the list, N tile nt.  The totals
  // are read once into registers; the bucket loop is unrolled so that every
  // field index is a constant.
  const int mt = w / ntn, nt = w % ntn;
  uint32_t tw[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) tw[k] = s_tot[k];
  int e = -1, mloc = 0, acc = 0;
#pragma unroll
  for (int b = 0; b <= kSelfMaxE; ++b) {
    const int n = b <= E ? (field(tw[b >> 1], b) + BM - 1) / BM : 0;
    if (e < 0 && mt < acc + n) {
      e = b;
      mloc = (mt - acc) * BM;
    }
    acc += n;
  }
  if (e < 0) return;  // past the tile list (the grid covers an upper bound)
  const int rows = min(BM, total(e) - mloc);
  const int n0 = nt * OBN;
  // The tile's rows: expert e's rows ranked in (thread, slot) order, which
  // every workgroup of the launch shares, so the M tiles of e partition its
  // rows.  (A row's result does not depend on which tile holds it.)
  for (int r = tid; r < BM; r += NT) srow[r] = -1;
  lds_barrier();
  {
    // Only the slots holding e are visited: the SWAR zero-nibble mask of
    // each bucket word (as in self_count_of) marks them, lowest slot first.
    int rk = prefix(e) - mloc;
    const uint32_t pat = 0x11111111u * (uint32_t)e;
#pragma unroll
    for (int j = 0; j < PER / 8; ++j) {
      const uint32_t xw = pk[j] ^ pat;
      uint32_t z = ~(((xw & 0x77777777u) + 0x77777777u) | xw | 0x77777777u);
      while (z) {
        const int sl = j * 8 + (__builtin_ctz(z) >> 2);
        z &= z - 1u;
        if ((unsigned)rk < (unsigned)BM)
          srow[rk] = STRIDED ? ((sl / VEC) * NT + tid) * VEC + sl % VEC : tid * PER + sl;
        ++rk;
      }
    }
  }
  if (e == E) {  // rows whose id is invalid: zeros
    __syncthreads();
    for (int i = tid; i < BM * OBN; i += NT) {
      const int r = srow[i / OBN];
      const int64_t col = n0 + i % OBN;
      if (r >= 0 && col < I) Y[(int64_t)r * I + col] = 0;
    }
    return;
  }
  gemm_tile<T, Cfg, 0, EPI, true>(smem, srow, X, W, W2, nullptr, nullptr, Y, H, I, topk, R, E, 0, nullptr, e, 0, rows,
                                  n0);
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

// K split of small problems (grouped_gemm_splitk_kernel): at most
// kSplitRows routed rows (then every expert has one M tile of CfgSmall), at
// most kSplitMaxTiles tiles, partial tiles in a workspace region of
// kSplitPartBytes and per-tile counters in the control block.
constexpr int64_t kSplitRows = 64;
constexpr size_t kSplitPartBytes = (size_t)3 << 20;
constexpr size_t kSplitCntOffset = 3200;
constexpr int kSplitMaxTiles = 128;
static_assert(kSplitCntOffset + kSplitMaxTiles * 4 <= kWsCtlBytes, "split counters fit the control block");
static_assert(kSplitCntOffset >= kGemmSchedOffset + 9 * 4, "split counters clear of the schedule counters");

struct GemmLayout {
  size_t blockcnt, counts, offsets, sorted, tile_expert, tile_mstart, meta, split, total;
  int64_t mt_ub;
};

static GemmLayout gemm_layout(int64_t R, int64_t E) {
  GemmLayout g;
  g.mt_ub = (R + kMinBM - 1) / kMinBM + E + 1;
  size_t o = 0;
  g.blockcnt = o; o += route_scratch_bytes(R, E);
  g.counts = o; o += align_up(E * sizeof(int32_t));
  g.offsets = o; o += align_up((E + 1) * sizeof(int32_t));
  g.sorted = o; o += align_up(std::max<int64_t>(R, 1) * sizeof(int32_t));
  g.tile_expert = o; o += align_up(g.mt_ub * sizeof(int32_t));
  g.tile_mstart = o; o += align_up(g.mt_ub * sizeof(int32_t));
  g.meta = o; o += align_up(4 * sizeof(int32_t));
  g.split = o; if (R <= kSplitRows) o += kSplitPartBytes;
  g.total = o;
  return g;
}

// Rows r < R_ids carry ids valid in [0, E_ids); rows R_ids .. R-1 belong to
// expert E_ids (E = E_ids + 1 then, else E = E_ids).
template <typename IdxT>
static int launch_route(const IdxT* ids, int64_t R, int64_t R_ids, int E_ids, int E, int32_t* blockcnt,
                        int32_t* counts, int32_t* offsets, int32_t* sorted_rows, int bm, int32_t* tile_expert,
                        int32_t* tile_mstart, int32_t* meta, hipStream_t st) {
  // One workgroup up to 2048 rows; beyond that the count + scatter pair is
  // faster (measured), unless E + 1 buckets need route_scan_kernel as well.
  if (E <= kRouteSmallE && (R <= 2048 || (R <= kRouteSmallRows && E + 1 > kRouteThreads))) {
    route_small_kernel<IdxT><<<1, kRouteSmallThreads, 0, st>>>(ids, R, R_ids, E_ids, E, counts, offsets, sorted_rows, bm,
                                                          tile_expert, tile_mstart, meta);
    return check_launch("route_small_kernel");
  }
  const RoutePlan p = route_plan(R);
  const size_t hist_lds = (size_t)(E + 1) * sizeof(int32_t);
  route_count_kernel<IdxT><<<p.nb, kRouteThreads, hist_lds, st>>>(ids, R, R_ids, E_ids, E, p.chunk, p.nb, blockcnt);
  if (int rc = check_launch("route_count_kernel")) return rc;
  const size_t scat_lds = (size_t)(E + 1) * (1 + kRouteThreads / kWave) * sizeof(int32_t);
  if (E + 1 <= 2 * kRouteThreads) {
    // Few buckets: each scatter workgroup scans the count table itself.
    const size_t lds = scat_lds + (size_t)(E + 2 + kRouteThreads / kWave) * sizeof(int32_t);
    route_scatter_kernel<IdxT, true><<<p.nb, kRouteThreads, lds, st>>>(
        ids, R, R_ids, E_ids, E, p.chunk, p.nb, blockcnt, offsets, sorted_rows, counts, bm, tile_expert, tile_mstart,
        meta);
    return check_launch("route_scatter_kernel");
  }
  route_scan_kernel<<<1, kScanThreads, 0, st>>>(blockcnt, R, E, p.nb, counts, offsets, bm, tile_expert,
                                                 tile_mstart, meta);
  if (int rc = check_launch("route_scan_kernel")) return rc;
  static std::atomic<uint64_t> lds_cap_set{0};  // E = 4096 needs more than the default 64 KB
  MOE_HIP_CHECK(lds_cap_once(lds_cap_set, (const void*)route_scatter_kernel<IdxT, false>,
                              (int)((kMaxExperts + 1) * (1 + kRouteThreads / kWave) * sizeof(int32_t)), st));
  route_scatter_kernel<IdxT, false><<<p.nb, kRouteThreads, scat_lds, st>>>(
      ids, R, R_ids, E_ids, E, p.chunk, p.nb, blockcnt, offsets, sorted_rows, nullptr, 0, nullptr, nullptr, nullptr);
  return check_launch("route_scatter_kernel");
}

template <typename T, typename Cfg, typename CfgS, int MODE = 0, int EPI = 0>
static int launch_gemm(hipStream_t st, const uint16_t* x, const uint16_t* w, const uint16_t* w2, const uint16_t* wx,
                       const uint16_t* w2x, uint16_t* y, int64_t H, int64_t I, int topk, int64_t R, int E, int ntn,
                       int64_t R_ids, int E_ids, int64_t x_shift, const int32_t* sorted, const int32_t* offsets,
                       const int32_t* t_exp, const int32_t* t_ms, const int32_t* meta, uint32_t* sched) {
  using CS = typename std::conditional<std::is_void<CfgS>::value, Cfg, CfgS>::type;
  constexpr size_t lds = Cfg::LDS_BYTES > CS::LDS_BYTES ? Cfg::LDS_BYTES : CS::LDS_BYTES;
  static std::atomic<uint64_t> lds_cap_set{0};
  MOE_HIP_CHECK(lds_cap_once(lds_cap_set, (const void*)grouped_gemm_kernel<T, Cfg, CfgS, MODE, EPI>, (int)lds, st));
  // Persistent grid of SUPER workgroups per XCD (8 XCDs x 32 CUs x MINB) when
  // the tile list can be long; otherwise one workgroup per possible tile.
  const int64_t ub = ((R + Cfg::BM - 1) / Cfg::BM + E + 1) * ntn;  // tiles, upper bound
  const int64_t grid = ub >= 16 * Cfg::SUPER ? 8 * Cfg::SUPER : (ub + 7) / 8 * 8;
  grouped_gemm_kernel<T, Cfg, CfgS, MODE, EPI><<<dim3((unsigned)grid), Cfg::THREADS, lds, st>>>(
      x, w, w2, wx, w2x, y, H, I, topk, R, E, ntn, R_ids, E_ids, x_shift, sorted, offsets, t_exp, t_ms, meta, sched);
  return MOE_OK;
}

template <typename T, typename IdxT, int EPI, int PER>
static int launch_selfroute(hipStream_t st, const uint16_t* x, const uint16_t* w, const uint16_t* w2, uint16_t* y,
                            int64_t H, int64_t I, int topk, int64_t R, int E, int ntn, const IdxT* ids,
                            int32_t* counts, int32_t* offsets, int32_t* sorted, int bm, int32_t* t_exp,
                            int32_t* t_ms, int32_t* meta) {
  using C = CfgSmall;
  static_assert(C::THREADS * kSelfPer == kSelfRows, "one thread per kSelfPer rows");
  static std::atomic<uint64_t> lds_cap_set{0};
  MOE_HIP_CHECK(lds_cap_once(lds_cap_set, (const void*)grouped_gemm_selfroute_kernel<T, C, IdxT, EPI, PER>,
                              (int)C::LDS_BYTES, st));
  // Items: an upper bound on the M tiles (every bucket may end in a partial
  // tile) times the N tiles; one more workgroup writes the routing tables.
  const int64_t items = ((R + C::BM - 1) / C::BM + E + 1) * ntn;
  const int share = (int)((items + 7) / 8);
  grouped_gemm_selfroute_kernel<T, C, IdxT, EPI, PER><<<dim3((unsigned)(8 * share + 1)), C::THREADS, C::LDS_BYTES, st>>>(
      x, w, w2, y, H, I, topk, (int)R, E, ntn, share, ids, counts, offsets, sorted, bm, t_exp, t_ms, meta);
  return check_launch("grouped_gemm_selfroute_kernel");
}

}  // namespace moe

using namespace moe;

extern "C" size_t moe_route_sort_workspace_size(int64_t R, int64_t E) {
  if (R < 0 || E < 1) return 0;
  return kWsCtlBytes + route_scratch_bytes(R, E);
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
  const size_t need = kWsCtlBytes + route_scratch_bytes(R, E);
  if (ws_bytes < need || !workspace)
    return fail(MOE_EINVAL, "route_sort: workspace too small (" + std::to_string(ws_bytes) + " < " +
                                std::to_string(need) + ")");
  hipStream_t st = static_cast<hipStream_t>(stream);
  int32_t* blockcnt = reinterpret_cast<int32_t*>(static_cast<char*>(workspace) + kWsCtlBytes);
  if (idx_dtype == MOE_I64)
    return launch_route(static_cast<const int64_t*>(expert_ids), R, R, (int)E, (int)E, blockcnt, counts, offsets,
                        sorted_rows, 0, nullptr, nullptr, nullptr, st);
  return launch_route(static_cast<const int32_t*>(expert_ids), R, R, (int)E, (int)E, blockcnt, counts, offsets,
                      sorted_rows, 0, nullptr, nullptr, nullptr, st);
}

extern "C" size_t moe_grouped_gemm_workspace_size(int64_t T, int64_t topk, int64_t E, int64_t I) {
  (void)I;
  if (T < 0 || topk < 1 || E < 1) return 0;
  return kWsCtlBytes + gemm_layout(T * topk, E).total;
}

namespace moe {

size_t grouped_gemm_ws_bytes(int64_t R, int64_t E) { return kWsCtlBytes + gemm_layout(R, E).total; }

// Shared by moe_grouped_gemm (EPI 0), moe_grouped_gemm_swiglu (EPI 1,
// W2 = the up weights; I is the output width, the tile rows cover 2 I) and,
// through grouped_gemm_run, the FusedMoE path (an appended expert, routing
// tables reused across calls).
template <int EPI>
static int grouped_gemm_impl(const char* fn, const void* X, const void* W, const void* W2, const void* expert_ids,
                             int dtype, int idx_dtype, int64_t T, int64_t topk, int64_t H, int64_t I, int64_t E,
                             const GemmExtra& ex, void* Y, void* workspace, size_t ws_bytes, void* stream,
                             int* bm_used) {
  const std::string f(fn);
  if (T < 0 || topk < 1 || H < 1 || I < 1 || ex.Tx < 0) return fail(MOE_EINVAL, f + ": need T >= 0, topk >= 1, H >= 1, I >= 1");
  if (E < 1 || E + (ex.Tx > 0) > kMaxExperts) return fail(MOE_EUNSUP, f + ": need 1 <= E <= 4096");
  if (H % 8 != 0) return fail(MOE_EUNSUP, f + ": H must be a multiple of 8");
  const int64_t R_ids = T * topk;
  const int64_t R = R_ids + ex.Tx;
  const int64_t Et = E + (ex.Tx > 0 ? 1 : 0);  // the appended rows form expert E
  const int64_t Iv = EPI == 1 ? 2 * I : I;  // weight rows per expert the tiles walk
  if (R >= INT32_MAX || (R + kMinBM - 1) / kMinBM + Et + 1 > (int64_t)INT32_MAX / ((Iv + 63) / 64))
    return fail(MOE_EUNSUP, f + ": problem too large");
  // The tiles address X and one expert's weights in 16-byte chunks with 32-bit offsets.
  if (std::max(T, ex.x_shift + ex.Tx) * (H / 8) > (int64_t)UINT32_MAX || I * (H / 8) > (int64_t)UINT32_MAX)
    return fail(MOE_EUNSUP, f + ": X or one expert's weights exceed 64 GiB");
  if (dtype != MOE_BF16 && dtype != MOE_F16)
    return fail(MOE_EINVAL, f + ": X, W and Y must be bfloat16 or float16");
  if (idx_dtype != MOE_I32 && idx_dtype != MOE_I64) return fail(MOE_EINVAL, f + ": expert ids must be int32 or int64");
  if (R == 0) return MOE_OK;
  if (!X || !W || (R_ids > 0 && !expert_ids && ex.reuse_bm == 0) || !Y || (EPI == 1 && !W2) ||
      (ex.Tx > 0 && (!ex.Wx || (EPI == 1 && !ex.W2x))))
    return fail(MOE_EINVAL, f + ": null pointer");
  if (((uintptr_t)X | (uintptr_t)W | (uintptr_t)W2 | (uintptr_t)ex.Wx | (uintptr_t)ex.W2x) & 15)
    return fail(MOE_EINVAL, f + ": X and the weights must be 16-byte aligned");
  const GemmLayout g = gemm_layout(R, Et);
  if (!workspace || ws_bytes < kWsCtlBytes + g.total)
    return fail(MOE_EINVAL, f + ": workspace too small (" + std::to_string(ws_bytes) + " < " +
                                std::to_string(kWsCtlBytes + g.total) + ")");
  hipStream_t st = static_cast<hipStream_t>(stream);
  // Dynamic-schedule counters of the GEMM kernel in the control block (zero
  // before and after every call).
  uint32_t* sched = reinterpret_cast<uint32_t*>(static_cast<char*>(workspace) + kGemmSchedOffset);
  char* ws = static_cast<char*>(workspace) + kWsCtlBytes;
  int32_t* blockcnt = reinterpret_cast<int32_t*>(ws + g.blockcnt);
  int32_t* counts = reinterpret_cast<int32_t*>(ws + g.counts);
  int32_t* offsets = reinterpret_cast<int32_t*>(ws + g.offsets);
  int32_t* sorted = reinterpret_cast<int32_t*>(ws + g.sorted);
  int32_t* t_exp = reinterpret_cast<int32_t*>(ws + g.tile_expert);
  int32_t* t_ms = reinterpret_cast<int32_t*>(ws + g.tile_mstart);
  int32_t* meta = reinterpret_cast<int32_t*>(ws + g.meta);
  // The largest tiles that still give every CU about two of them: 256x256
  // (BK 64, full 128-byte lines per row copy) moves the least data per
  // MFMA; smaller problems take smaller tiles to fill the chip.
  auto tiles_of = [&](int64_t bm, int64_t bn) { return ((R + bm - 1) / bm) * ((Iv + bn - 1) / bn); };
  // Also the mixed 256/128-row configuration when experts average at most
  // 128 rows and there are enough 128x256 tiles for every CU: each expert
  // is then one short tile per N tile, streaming its weights once.
  const bool short_experts = R <= 128 * Et && tiles_of(CfgShort::BM, CfgShort::BN) >= 256;
  const int cfg = tiles_of(CfgHuge::BM, CfgHuge::BN) >= 512 || short_experts ? 2
                  : tiles_of(CfgLarge::BM, CfgLarge::BN) >= 512              ? 1
                                                                             : 0;
  const int bn = cfg == 2 ? CfgHuge::BN : cfg == 1 ? CfgLarge::BN : CfgSmall::BN;
  const int obn = EPI == 1 ? bn / 2 : bn;
  const int ntn = (int)((I + obn - 1) / obn);
  // Mixed tables alternate tall and short tiles in blocks of one
  // super-tile's M tiles (the kernel's SM).  The interleaved table holds at
  // most R/256 + E entries plus two partial blocks of holes, which the
  // workspace's R/64 + E + 1 entries cover when 3R/256 >= 2 blk.  The last
  // round of the persistent grid (8 x SUPER items) is kept for short tiles.
  const int il_cand = CfgHuge::SUPER / std::min(ntn, CfgHuge::SN_MAX);
  const int il_blk = cfg == 2 && 3 * R >= 512 * (int64_t)il_cand ? il_cand : 0;
  const int il_reserve =
      il_blk ? (int)std::min<int64_t>(31, (8 * CfgHuge::SUPER + (int64_t)il_blk * ntn - 1) / ((int64_t)il_blk * ntn)) : 0;
  const int bm = cfg == 2 ? bm_mixed(CfgHuge::BM, CfgShort::BM, il_blk, il_reserve) : cfg == 1 ? CfgLarge::BM : CfgSmall::BM;
  if (bm_used) *bm_used = bm;
  const uint16_t* x = static_cast<const uint16_t*>(X);
  const uint16_t* w = static_cast<const uint16_t*>(W);
  const uint16_t* w2 = static_cast<const uint16_t*>(W2);
  uint16_t* y = static_cast<uint16_t*>(Y);
  // Few rows (decode): split each tile along K so that the weights stream
  // through many more CUs; the per-tile sums stay in a fixed order.
  struct {
    int S = 0, tiles_ub = 0, pt = 0, nv = 0;
    int64_t kchunk = 0;
    unsigned grid = 0;
  } split;
  if (cfg == 0 && ex.Tx == 0 && R <= kSplitRows && MOE_GEMM_TUNE_MODE == 0) {
    using C = CfgSmall;
    const int64_t nk = (H + C::BK - 1) / C::BK;
    const int64_t tiles_ub = std::min<int64_t>(Et, R) * ntn;
    // With at most 32 rows only the waves of the first 32-row block publish.
    static_assert(C::FM == 1 && C::WM == 2, "the second row block is the second half of the workgroup");
    const int pt = R <= 32 ? C::THREADS / 2 : C::THREADS;
    const int nv = R <= 8 ? 4 : R <= 16 ? 8 : 16;  // accumulators that can hold a row
    const int64_t per_item = (int64_t)pt * C::FM * C::FN * nv * sizeof(float);
    const int64_t S = std::min<int64_t>({6, nk / 4, (int64_t)(kSplitPartBytes / per_item) / tiles_ub, 384 / tiles_ub});
    if (S >= 2 && tiles_ub <= kSplitMaxTiles) {
      split.S = (int)S;
      split.tiles_ub = (int)tiles_ub;
      split.pt = pt;
      split.nv = nv;
      split.kchunk = (nk + S - 1) / S * C::BK;
      split.grid = (unsigned)(tiles_ub * S + ntn);  // + the invalid-id rows (at most one M tile)
    }
  }
  // Split calls that route themselves: no sort launch.
  if (split.S >= 2 && ex.reuse_bm == 0) {
    float* part = reinterpret_cast<float*>(ws + g.split);
    uint32_t* cnt = reinterpret_cast<uint32_t*>(static_cast<char*>(workspace) + kSplitCntOffset);
    const uint16_t* x0 = static_cast<const uint16_t*>(X);
    const uint16_t* w0 = static_cast<const uint16_t*>(W);
    const uint16_t* w20 = static_cast<const uint16_t*>(W2);
    uint16_t* y0 = static_cast<uint16_t*>(Y);
    auto launch = [&](auto t_tag, auto nv_tag, const auto* ids) {
      using TT = decltype(t_tag);
      using IT = std::remove_cv_t<std::remove_pointer_t<decltype(ids)>>;
      using C = CfgSmall;
      constexpr int NVP = decltype(nv_tag)::value;
      static std::atomic<uint64_t> lds_cap_set{0};
      MOE_HIP_CHECK(lds_cap_once(lds_cap_set, (const void*)grouped_gemm_splitk_self_kernel<TT, C, IT, EPI, NVP>,
                                  (int)C::LDS_BYTES, st));
      grouped_gemm_splitk_self_kernel<TT, C, IT, EPI, NVP><<<split.grid + 1, C::THREADS, C::LDS_BYTES, st>>>(
          x0, w0, w20, y0, H, I, (int)topk, (int)R, (int)Et, ntn, split.S, split.tiles_ub, split.kchunk, split.pt, ids,
          counts, offsets, sorted, bm, t_exp, t_ms, meta, part, cnt);
      return check_launch("grouped_gemm_splitk_self_kernel");
    };
    auto by_nv = [&](auto t_tag, const auto* ids) {
      return split.nv == 4 ? launch(t_tag, IntC<4>{}, ids) : split.nv == 8 ? launch(t_tag, IntC<8>{}, ids)
                                                                           : launch(t_tag, IntC<16>{}, ids);
    };
    auto by_idx = [&](auto t_tag) {
      return idx_dtype == MOE_I64 ? by_nv(t_tag, static_cast<const int64_t*>(expert_ids))
                                  : by_nv(t_tag, static_cast<const int32_t*>(expert_ids));
    };
    return dtype == MOE_BF16 ? by_idx(uint16_t{}) : by_idx(Half16{});
  }
  // Small routings without an appended expert (and not split): one
  // self-routing launch instead of the routing sort's launches and the GEMM.
  // Each thread groups kSelfPer rows above 2048 rows, 8 up to 2048.
#ifndef MOE_SELF_MIN
#define MOE_SELF_MIN 0
#endif
  if (cfg == 0 && ex.reuse_bm == 0 && ex.Tx == 0 && E <= kSelfMaxE && R > MOE_SELF_MIN && R <= kSelfRows &&
      ((uintptr_t)expert_ids & 15) == 0) {
    auto self = [&](auto t_tag, const auto* ids) {
      using TT = decltype(t_tag);
      using IT = std::remove_cv_t<std::remove_pointer_t<decltype(ids)>>;
      return R <= 2048 ? launch_selfroute<TT, IT, EPI, 8>(st, x, w, w2, y, H, I, (int)topk, R, (int)E, ntn, ids,
                                                           counts, offsets, sorted, bm, t_exp, t_ms, meta)
                       : launch_selfroute<TT, IT, EPI, kSelfPer>(st, x, w, w2, y, H, I, (int)topk, R, (int)E, ntn,
                                                                   ids, counts, offsets, sorted, bm, t_exp, t_ms, meta);
    };
    if (dtype == MOE_BF16)
      return idx_dtype == MOE_I64 ? self(uint16_t{}, static_cast<const int64_t*>(expert_ids))
                                  : self(uint16_t{}, static_cast<const int32_t*>(expert_ids));
    return idx_dtype == MOE_I64 ? self(Half16{}, static_cast<const int64_t*>(expert_ids))
                                : self(Half16{}, static_cast<const int32_t*>(expert_ids));
  }
  int rc = MOE_OK;
  if (ex.reuse_bm == 0) {
    if (idx_dtype == MOE_I64)
      rc = launch_route(static_cast<const int64_t*>(expert_ids), R, R_ids, (int)E, (int)Et, blockcnt, counts, offsets,
                        sorted, bm, t_exp, t_ms, meta, st);
    else
      rc = launch_route(static_cast<const int32_t*>(expert_ids), R, R_ids, (int)E, (int)Et, blockcnt, counts, offsets,
                        sorted, bm, t_exp, t_ms, meta, st);
  } else if (ex.reuse_bm > 0 && ex.reuse_bm != bm) {  // reuse_bm < 0: the tables were built for this shape
    route_tiles_kernel<<<1, kScanThreads, 0, st>>>(offsets, (int)Et, bm, t_exp, t_ms, meta);
    rc = check_launch("route_tiles_kernel");
  }
  if (rc) return rc;
  const uint16_t* wx = static_cast<const uint16_t*>(ex.Wx);
  const uint16_t* w2x = static_cast<const uint16_t*>(ex.W2x);
  auto run = [&](auto cfg_tag, auto cfgs_tag) {
    using C = decltype(cfg_tag);
    using CS = typename decltype(cfgs_tag)::type;
    return dtype == MOE_BF16
               ? launch_gemm<uint16_t, C, CS, MOE_GEMM_TUNE_MODE, EPI>(st, x, w, w2, wx, w2x, y, H, I, (int)topk, R, (int)Et, ntn,
                                                     R_ids, (int)E, ex.x_shift, sorted, offsets, t_exp, t_ms, meta,
                                                     sched)
               : launch_gemm<Half16, C, CS, MOE_GEMM_TUNE_MODE, EPI>(st, x, w, w2, wx, w2x, y, H, I, (int)topk, R, (int)Et, ntn,
                                                   R_ids, (int)E, ex.x_shift, sorted, offsets, t_exp, t_ms, meta,
                                                   sched);
  };
  if (split.S >= 2) {
    float* part = reinterpret_cast<float*>(ws + g.split);
    uint32_t* cnt = reinterpret_cast<uint32_t*>(static_cast<char*>(workspace) + kSplitCntOffset);
    auto launch = [&](auto t_tag, auto nv_tag) {
      using TT = decltype(t_tag);
      using C = CfgSmall;
      constexpr int NVP = decltype(nv_tag)::value;
      static std::atomic<uint64_t> lds_cap_set{0};
      MOE_HIP_CHECK(lds_cap_once(lds_cap_set, (const void*)grouped_gemm_splitk_kernel<TT, C, EPI, NVP>,
                                  (int)C::LDS_BYTES, st));
      grouped_gemm_splitk_kernel<TT, C, EPI, NVP><<<split.grid, C::THREADS, C::LDS_BYTES, st>>>(
          x, w, w2, y, H, I, (int)topk, R, (int)Et, ntn, split.S, split.tiles_ub, split.kchunk, split.pt, sorted,
          offsets, t_exp, t_ms, meta, part, cnt);
      return check_launch("grouped_gemm_splitk_kernel");
    };
    auto by_nv = [&](auto t_tag) {
      return split.nv == 4 ? launch(t_tag, IntC<4>{}) : split.nv == 8 ? launch(t_tag, IntC<8>{})
                                                                      : launch(t_tag, IntC<16>{});
    };
    return dtype == MOE_BF16 ? by_nv(uint16_t{}) : by_nv(Half16{});
  }
  rc = cfg == 2 ? run(CfgHuge{}, TypeC<CfgShort>{}) : cfg == 1 ? run(CfgLarge{}, TypeC<void>{})
                                                              : run(CfgSmall{}, TypeC<void>{});
  if (rc) return rc;
  return check_launch("grouped_gemm_kernel");
}

int grouped_gemm_run(int epi, const void* X, const void* W, const void* W2, const void* expert_ids, int dtype,
                     int idx_dtype, int64_t T, int64_t topk, int64_t H, int64_t I, int64_t E, const GemmExtra& ex,
                     void* Y, void* workspace, size_t ws_bytes, hipStream_t stream, int* bm_used) {
  return epi == 1 ? grouped_gemm_impl<1>("grouped_gemm_swiglu", X, W, W2, expert_ids, dtype, idx_dtype, T, topk, H,
                                         I, E, ex, Y, workspace, ws_bytes, stream, bm_used)
                  : grouped_gemm_impl<0>("grouped_gemm", X, W, nullptr, expert_ids, dtype, idx_dtype, T, topk, H, I,
                                         E, ex, Y, workspace, ws_bytes, stream, bm_used);
}

}  // namespace moe

extern "C" int moe_grouped_gemm(const void* X, const void* W, const void* expert_ids, int dtype,
                                int idx_dtype, int64_t T, int64_t topk, int64_t H, int64_t I,
                                int64_t E, void* Y, void* workspace, size_t ws_bytes, void* stream) {
  return grouped_gemm_impl<0>("grouped_gemm", X, W, nullptr, expert_ids, dtype, idx_dtype, T, topk, H, I, E,
                              GemmExtra{}, Y, workspace, ws_bytes, stream, nullptr);
}

extern "C" int moe_grouped_gemm_swiglu(const void* X, const void* Wg, const void* Wu, const void* expert_ids,
                                       int dtype, int idx_dtype, int64_t T, int64_t topk, int64_t H,
                                       int64_t I, int64_t E, void* Y, void* workspace, size_t ws_bytes,
                                       void* stream) {
  return grouped_gemm_impl<1>("grouped_gemm_swiglu", X, Wg, Wu, expert_ids, dtype, idx_dtype, T, topk, H, I, E,
                              GemmExtra{}, Y, workspace, ws_bytes, stream, nullptr);
}

extern "C" int moe_grouped_gemm_routed(const void* X, const void* W, int dtype, int64_t T, int64_t topk, int64_t H,
                                       int64_t I, int64_t E, void* Y, void* workspace, size_t ws_bytes,
                                       void* stream) {
  GemmExtra ex;
  ex.reuse_bm = -1;  // the routing tables of the previous call of this shape on this workspace
  return grouped_gemm_impl<0>("grouped_gemm_routed", X, W, nullptr, nullptr, dtype, MOE_I32, T, topk, H, I, E, ex, Y,
                              workspace, ws_bytes, stream, nullptr);
}

// ---------------------------------------------------------------------------
// moe_grouped_gemm_noalloc: moe_grouped_gemm with its workspace in a
// file-scope device array, for callers that cannot allocate.
// ---------------------------------------------------------------------------
namespace moe {

// The workspace of moe_grouped_gemm_noalloc (control block + routing
// tables).  Every device holds its own copy for the life of the process and
// every call on a device uses that device's copy.  In host code the name
// `scratch` is only a handle: kernels get the address that
// hipGetSymbolAddress returns (noalloc_scratch), never the symbol itself.
static __device__ __align__(256) unsigned char scratch[MOE_NOALLOC_SCRATCH_BYTES];

__global__ void zero_words_kernel(uint32_t* __restrict__ p, int n) {
  for (int i = threadIdx.x; i < n; i += blockDim.x) p[i] = 0u;
}

constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kMaxDevices];  // device address of `scratch`, per device

// Device address of the current device's `scratch`, looked up on the first
// call on that device (with that device current) and kept.
static int noalloc_scratch(void** out) {
  int dev = 0;
  MOE_HIP_CHECK(hipGetDevice(&dev));
  if (dev < 0 || dev >= kMaxDevices) return fail(MOE_EUNSUP, "grouped_gemm_noalloc: device index beyond 63");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    MOE_HIP_CHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    if (!p) return fail(MOE_EHIP, "grouped_gemm_noalloc: hipGetSymbolAddress returned a null address");
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return MOE_OK;
}

}  // namespace moe

extern "C" int moe_grouped_gemm_noalloc(const void* X, const void* W, const void* expert_ids, int dtype,
                                        int idx_dtype, int64_t T, int64_t topk, int64_t H, int64_t I, int64_t E,
                                        void* Y, void* stream) {
  if (T < 0 || topk < 1 || H < 1 || I < 1) return fail(MOE_EINVAL, "grouped_gemm_noalloc: need T >= 0, topk >= 1, H >= 1, I >= 1");
  if (E < 1 || E > kMaxExperts) return fail(MOE_EUNSUP, "grouped_gemm_noalloc: need 1 <= E <= 4096");
  if (T == 0) return MOE_OK;
  if (T > (int64_t)INT32_MAX / topk) return fail(MOE_EUNSUP, "grouped_gemm_noalloc: problem too large");
  const size_t need = kWsCtlBytes + gemm_layout(T * topk, E).total;
  if (need > (size_t)MOE_NOALLOC_SCRATCH_BYTES)
    return fail(MOE_EUNSUP, "grouped_gemm_noalloc: " + std::to_string(T * topk) + " routed rows over " +
                                std::to_string(E) + " experts need " + std::to_string(need) +
                                " bytes of scratch, more than its fixed " +
                                std::to_string((size_t)MOE_NOALLOC_SCRATCH_BYTES) +
                                "; use moe_grouped_gemm with a workspace");
  void* ws = nullptr;
  if (int rc = noalloc_scratch(&ws)) return rc;
  // The control block must be zero; every completed call leaves it so, and
  // this clears it after a call that stopped part-way.  A kernel, not
  // hipMemsetAsync, so that the call can be captured into a HIP graph.
  hipStream_t st = static_cast<hipStream_t>(stream);
  zero_words_kernel<<<1, 256, 0, st>>>(static_cast<uint32_t*>(ws), (int)(kWsCtlBytes / 4));
  if (int rc = check_launch("zero_words_kernel")) return rc;
  return grouped_gemm_impl<0>("grouped_gemm_noalloc", X, W, nullptr, expert_ids, dtype, idx_dtype, T, topk, H, I, E,
                              GemmExtra{}, Y, ws, (size_t)MOE_NOALLOC_SCRATCH_BYTES, stream, nullptr);
}
