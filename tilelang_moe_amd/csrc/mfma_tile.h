// MFMA tile machinery shared by the grouped GEMM and the router GEMM:
// operand types, the gfx950 v_mfma_f32_32x32x16 wrappers, tile
// configurations and the LDS-DMA pipelined k loop of one output tile.
#pragma once
#include "common.h"

namespace moe {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

typedef __attribute__((address_space(3))) void lds_void_t;

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

// s_waitcnt vmcnt(N) with every other counter left alone (N <= 63).
template <int N>
__device__ inline void vm_wait() {
  static_assert(N >= 0 && N <= 63, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | (((N >> 4) & 3) << 14) | 0x0F70);
}

template <int V> struct IntC { static constexpr int value = V; };

// Calls fn(IntC<min(n, F)>) for a wave-uniform n >= 0: one specialised body
// per value, chosen by scalar branches.
template <int F, typename Fn>
__device__ inline void with_count(int n, Fn&& fn) {
  if constexpr (F == 0) {
    fn(IntC<0>{});
  } else {
    if (n >= F) fn(IntC<F>{});
    else with_count<F - 1>(n, fn);
  }
}

// Tile configurations.  A workgroup computes a BM x BN tile of one expert
// with WM x WN waves, each owning FM x FN blocks of 32x32 (v_mfma 32x32x16);
// K advances BK elements per k-tile and STAGES k-tiles are in LDS (STAGES-1
// in flight while one is consumed).
//
// LDS layout of a stage: A rows then B rows, each row BK elements = CPR
// chunks of 16 bytes.  Chunk c of row r sits at position
//   c ^ ((r / SWZ) % CPR),   SWZ = 16 / CPR,
// so the 16 lanes an LDS cycle serves in a 16-byte MFMA operand fetch (16
// consecutive rows, one chunk each: 256 bytes over 64 four-byte banks) hit 16
// different 16-byte bank groups.
//
// Global -> LDS copies are gfx950 global_load_lds_dwordx4: every lane
// fetches one 16-byte chunk straight into LDS and a wave instruction fills
// 1 KB (64 / CPR rows), so copies use no VGPRs.  A lane picks the global
// chunk that belongs in its LDS slot.
template <int BM_, int BN_, int WM_, int WN_, int BK_, int STAGES_, int MINB_ = 1>
struct GemmCfg {
  static constexpr int BM = BM_, BN = BN_, WM = WM_, WN = WN_, BK = BK_, STAGES = STAGES_;
  static constexpr int MINB = MINB_;              // workgroups resident per CU
  static constexpr int SUPER = 32 * MINB;         // workgroups per XCD (32 CUs each)
  static constexpr int SN_MAX = 4;                // N tiles per super-tile
  static constexpr int CPR = BK / 8;             // 16-byte chunks per row
  static constexpr int RPI = kWave / CPR;        // rows per copy instruction
  static constexpr int WAVES = WM * WN, THREADS = WAVES * kWave;
  static constexpr int FM = BM / WM / 32, FN = BN / WN / 32;
  static constexpr int A_INS = BM / RPI / WAVES, B_INS = BN / RPI / WAVES;  // per thread per stage
  static constexpr int STAGE_ELEMS = (BM + BN) * BK;
  static constexpr size_t LDS_BYTES = (size_t)STAGES * STAGE_ELEMS * 2;
  static_assert(CPR == 4 || CPR == 8, "BK must be 32 or 64");
  static_assert(STAGES >= 2, "at least two stages");
  static_assert(FM >= 1 && FN >= 1 && A_INS >= 1 && B_INS >= 1, "bad tile configuration");
  static_assert(A_INS * WAVES * RPI == BM && B_INS * WAVES * RPI == BN, "rows must split evenly over waves");
  static_assert(LDS_BYTES + BM * 4 <= 160 * 1024, "LDS budget");
  static constexpr int SWZ = 16 / CPR;  // consecutive rows sharing one XOR key
  // Position of chunk c in row r, and (XOR is an involution) the chunk that
  // position c of row r holds.
  static __device__ inline int pos(int r, int c) { return c ^ ((r / SWZ) % CPR); }
  static __device__ inline int slot(int r, int c) { return r * CPR + pos(r, c); }
  // The 16-byte chunk that lane `lane` copies in copy instruction `ins` of
  // wave `wave` (INS instructions per wave): it fills position lane % CPR of
  // operand row RPI * (wave * INS + ins) + lane / CPR.
  static __device__ inline int copy_chunk(int wave, int ins, int INS, int lane) {
    return pos(RPI * (wave * INS + ins) + lane / CPR, lane % CPR);
  }
};

// Copy-slot rows as 32-bit offsets, in 16-byte chunks, from one base: half
// the registers of per-row pointers (a chunk index reaches 64 GiB past the
// base), at one address add per copy.
template <int N>
struct RowOffs {
  const uint16_t* base;
  uint32_t o[N];
};
template <int N>
__device__ inline const uint16_t* src_row(const uint16_t* const (&p)[N], int i) { return p[i]; }
template <int N>
__device__ inline const uint16_t* src_row(const RowOffs<N>& r, int i) { return r.base + (uint64_t)r.o[i] * 8; }

// The k loop of one output tile: acc[i][j] += A-rows x B-rows over k in
// [kb, ke) (kb a multiple of BK; elements at k >= ke count as zero).
// a_src / b_src give this thread's copy-slot rows (pointer arrays or
// RowOffs), already offset by the 16-byte chunk of its slot (Cfg::copy_chunk); fm_act is the
// wave-uniform count of 32-row blocks of this wave that hold rows (the
// MFMAs of the others are skipped).  MODE (tuning builds only): 1 = copies
// only, 2 = MFMAs only.
template <typename T, typename Cfg, int MODE, typename ASrc, typename BSrc>
__device__ inline void tile_mainloop(uint16_t* smem, const ASrc& a_src, const BSrc& b_src, int64_t kb,
                                     int64_t ke, int fm_act, f32x16 (&acc)[Cfg::FM][Cfg::FN]) {
  constexpr int BM = Cfg::BM, BN = Cfg::BN, BK = Cfg::BK, S = Cfg::STAGES, CPR = Cfg::CPR;
  constexpr int INS = Cfg::A_INS + Cfg::B_INS;
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;
  const int wm = wave / Cfg::WN, wn = wave % Cfg::WN;
  const int nk = (int)((ke - kb + BK - 1) / BK);
  const bool ktail = ((ke - kb) % BK) != 0;
  auto stage = [&](int t) { return smem + (t % S) * Cfg::STAGE_ELEMS; };

  // Copies of k-tile t into its stage.  Chunks at or past ke (last k-tile
  // only) read the row start; they are zeroed in LDS before use.
  auto issue = [&](int t) {
    if (t >= nk || MODE == 2) return;
    uint16_t* st = stage(t);
    const int64_t k = kb + (int64_t)t * BK;
    const bool tail = ktail && t == nk - 1;
    auto koff = [&](int c) -> int64_t { return (!tail || k + c * 8 < ke) ? k : -(int64_t)c * 8; };
#pragma unroll
    for (int i = 0; i < Cfg::A_INS; ++i)
      __builtin_amdgcn_global_load_lds((const void*)(src_row(a_src, i) + koff(Cfg::copy_chunk(wave, i, Cfg::A_INS, lane))),
                                       (lds_void_t*)(st + (wave * Cfg::A_INS + i) * 512), 16, 0, 0);
#pragma unroll
    for (int i = 0; i < Cfg::B_INS; ++i)
      __builtin_amdgcn_global_load_lds(
          (const void*)(src_row(b_src, i) + koff(Cfg::copy_chunk(wave, i, Cfg::B_INS, lane))),
          (lds_void_t*)(st + BM * BK + (wave * Cfg::B_INS + i) * 512), 16, 0, 0);
  };

  // The k loop, specialised on the number FA of active 32-row blocks so
  // that the skip is a scalar branch taken once per tile.
  //
  // Operand fragments are double buffered in registers: the LDS reads of
  // step s+1 are issued between the MFMAs of step s.  The k-tile boundary
  // sits inside the last step of a k-tile: once that step's fragments are
  // in registers, the thread waits for its copies of the next k-tile (the
  // S-2 younger k-tiles stay in flight), the workgroup meets at a barrier
  // (every wave is then done reading the k-tile's stage and every copy of
  // the next k-tile has landed), the freed stage is refilled, and the last
  // step's MFMAs run while the next k-tile's first fragments are read.  So
  // the MFMAs do not wait for a fresh LDS round trip after the barrier.
  auto k_loop = [&](auto fa_tag) {
    constexpr int FA = decltype(fa_tag)::value;
    constexpr int FAR = FA > 0 ? FA : 1;
    constexpr int STEPS = BK / 16;
    constexpr bool LOADS = FA > 0 || MODE == 1;
    u32x4 a[2][FAR], b[2][Cfg::FN];
    auto load = [&](int t, int s, int q) {
      const u32x4* As = reinterpret_cast<const u32x4*>(stage(t));
      const u32x4* Bs = reinterpret_cast<const u32x4*>(stage(t) + BM * BK);
      const int c = 2 * s + (lane >> 5);
#pragma unroll
      for (int i = 0; i < FA; ++i) a[q][i] = As[Cfg::slot(wm * Cfg::FM * 32 + i * 32 + (lane & 31), c)];
#pragma unroll
      for (int j = 0; j < Cfg::FN; ++j) b[q][j] = Bs[Cfg::slot(wn * Cfg::FN * 32 + j * 32 + (lane & 31), c)];
    };
    auto mfmas = [&](int q) {
      if constexpr (MODE == 1) {
        acc[0][0][0] += __uint_as_float(a[q][0][0] ^ b[q][0][0]);
      } else {
#pragma unroll
        for (int i = 0; i < FA; ++i)
#pragma unroll
          for (int j = 0; j < Cfg::FN; ++j) acc[i][j] = MfmaOp<T>::run(a[q][i], b[q][j], acc[i][j]);
      }
    };
    // Pins one step's order: each MFMA followed by one of the next reads.
    auto pin_step = [&]() {
      if constexpr (MODE != 1 && FA > 0) {
#pragma unroll
        for (int m = 0; m < FA * Cfg::FN; ++m) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          if (m < FA + Cfg::FN) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
      }
    };
    // Make k-tile t visible to the workgroup and refill the stage of t-1.
    auto arrive = [&](int t) {
      if (t + S - 2 < nk) vm_wait<(S - 2) * INS>();
      else vm_wait<0>();
      // Plain s_barrier: __syncthreads() would also wait for the younger
      // k-tiles still in flight (its release fence drains vmcnt).
      __builtin_amdgcn_s_barrier();
      issue(t + S - 1);
      if (ktail && t == nk - 1) {
        // Zero the chunks at or past ke of the last k-tile in both operands.
        uint16_t* sw = stage(t);
        const int64_t k = kb + (int64_t)t * BK;
        for (int q = tid; q < (BM + BN) * CPR; q += Cfg::THREADS) {
          const int r = q / CPR, c = Cfg::pos(r, q % CPR);
          if (k + c * 8 >= ke) *reinterpret_cast<u32x4*>(sw + q * 8) = u32x4{0u, 0u, 0u, 0u};
        }
        __syncthreads();
      }
    };

    if (nk <= 0) return;
#pragma unroll
    for (int t = 0; t < S - 1; ++t) issue(t);
    arrive(0);
    if constexpr (LOADS) load(0, 0, 0);
    // Steps 0 .. STEPS-2 of k-tile t (the last step differs per k-tile).
    auto front = [&](int t) {
#pragma unroll
      for (int s = 0; s + 1 < STEPS; ++s) {
        if constexpr (LOADS) load(t, s + 1, (s + 1) & 1);
        mfmas(s & 1);
      }
#pragma unroll
      for (int s = 0; s + 1 < STEPS; ++s) pin_step();
    };
    for (int kt = 0; kt + 1 < nk; ++kt) {
      front(kt);
      // The last step's fragments are in registers before the barrier, so
      // after it the stage of k-tile kt may be overwritten.
      __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
      arrive(kt + 1);
      if constexpr (LOADS) load(kt + 1, 0, 0);
      mfmas((STEPS - 1) & 1);
      pin_step();
    }
    front(nk - 1);
    mfmas((STEPS - 1) & 1);
  };
  with_count<Cfg::FM>(fm_act, k_loop);
}

}  // namespace moe
