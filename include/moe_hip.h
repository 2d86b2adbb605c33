/*
 * moe_hip.h — C ABI of the MI355X (gfx950) MoE routed-expert hot path.
 *
 * The reference (Wendy-Hamlet/tilelang_moe) has no FFI: its boundary is the
 * Python API in kernels/__init__.py, whose two hot-path names are
 *   topk_softmax  = topk_softmax_best   (kernels/__init__.py:21,
 *                                        kernels/topk_softmax_tilelang.py:1103-1135)
 *   grouped_gemm  = grouped_gemm_best   (kernels/__init__.py:34,
 *                                        kernels/grouped_gemm_tilelang.py:859-890)
 * This library is what those Python functions call in this build (through
 * ctypes, see tilelang_moe_amd/_lib.py).  Every entry point below cites the
 * reference function it replaces.
 *
 * Conventions shared by every entry point:
 *   - All data pointers are DEVICE pointers.  `stream` is a hipStream_t
 *     (pass torch.cuda.current_stream().cuda_stream, or NULL for the
 *     default stream).  Nothing here synchronises the stream, allocates or
 *     frees device memory.
 *   - Return value: 0 on success, a negative MOE_E* code on failure; the
 *     message of the last failure on the calling thread is moe_last_error().
 *   - Workspaces are caller-owned device buffers of at least the size the
 *     matching *_workspace_size() function returns.  Its first 4096 bytes
 *     are a control block (per-row counters of the split-row top-k) that
 *     must be all-zero before the first call; every entry point leaves that
 *     block all-zero when it returns successfully.  The bytes after it are
 *     scratch that any call overwrites.  So one workspace, zeroed once, can
 *     serve consecutive calls of any entry point on ONE stream.  Calls that
 *     overlap in time must use different workspaces.
 */
#ifndef MOE_HIP_H
#define MOE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types understood by the entry points. */
enum moe_dtype {
  MOE_F32 = 0,
  MOE_BF16 = 1,
  MOE_F16 = 2,
  MOE_I32 = 3,
  MOE_I64 = 4
};

/* Router algorithms (argument `algo` of moe_topk_softmax). */
enum moe_topk_algo {
  MOE_TOPK_AUTO = -1,      /* N<=64 bitonic, 65..512 selection, >512 radix */
  MOE_TOPK_BITONIC = 0,    /* wave64 register bitonic network, N <= 64     */
  MOE_TOPK_SELECTION = 1,  /* K rounds of wave64 argmax, N <= 1024         */
  MOE_TOPK_RADIX = 2       /* multi-pass radix select, any N, K <= 16384   */
};

/* Score conventions (argument `score_mode` of moe_topk_softmax_ex).  The
 * selected indices and their order are the same in every mode. */
enum moe_score_mode {
  MOE_SCORES_TOPK = 0,        /* Convention B: softmax over the K selected logits */
  MOE_SCORES_ALL = 1,         /* Convention A: softmax over all N logits, read at the K */
  MOE_SCORES_TOPK_RENORM = 2  /* Convention A + renormalisation: equal to B */
};

/* Error codes. */
#define MOE_OK 0
#define MOE_EINVAL (-1)   /* bad shape, dtype, pointer or alignment        */
#define MOE_EUNSUP (-2)   /* valid request outside the supported limits    */
#define MOE_EHIP (-3)     /* a HIP runtime call failed                     */

/* Message describing the last failure on the calling thread ("" if none). */
const char* moe_last_error(void);

/* Library ABI version (major*10000 + minor*100 + patch). */
int moe_version(void);

/* Algorithm MOE_TOPK_AUTO resolves to for a row length N and top-K.
 * Replaces _select_strategy (kernels/topk_softmax_tilelang.py:1056-1100),
 * with the thresholds of the reference README (README.md:120-122):
 * N<=64 -> bitonic, 65<=N<=512 -> selection, N>512 -> radix. */
int moe_topk_select_algo(int64_t N, int64_t K);

/* Workspace bytes moe_topk_softmax needs for this shape and algorithm
 * (0 for bitonic and selection). */
size_t moe_topk_softmax_workspace_size(int64_t M, int64_t N, int64_t K, int algo);

/* Fused TopK + softmax over the last dimension of a row-major [M, N] matrix.
 *
 * Replaces topk_softmax_best (kernels/topk_softmax_tilelang.py:1103-1135)
 * and, per branch, topk_softmax_bitonic (:895-921), topk_softmax_selection
 * (:983-1001) and topk_radix_tilelang + torch gather/softmax (:205-235,
 * :1128-1131).  Semantics are those of the reference's PyTorch baseline
 * topk_softmax_fused (kernels/topk_softmax_baseline.py:39-66):
 *     v, i = topk(logits, K, dim=-1)            (sorted, descending)
 *     scores = softmax(v, dim=-1, dtype=fp32)
 * with one deterministic tie rule: equal values are ordered by ascending
 * index; -0.0 equals +0.0; NaN ranks above +inf.
 *
 *   logits        [M, N] rows, row stride `ld` elements (ld >= N),
 *                 dtype MOE_F32, MOE_BF16 or MOE_F16
 *   scores        [M, K] fp32, contiguous; may be NULL (indices only, the
 *                 reference's topk_radix_tilelang)
 *   indices       [M, K] contiguous, idx_dtype MOE_I32 or MOE_I64
 *   algo          enum moe_topk_algo
 *   workspace     >= moe_topk_softmax_workspace_size(M, N, K, algo) bytes
 *                 (may be NULL when that size is 0)
 */
int moe_topk_softmax(const void* logits, int logits_dtype, int64_t M, int64_t N,
                     int64_t ld, int64_t K, float* scores, void* indices,
                     int idx_dtype, int algo, void* workspace, size_t ws_bytes,
                     void* stream);

/* moe_topk_softmax with a score convention.
 * MOE_SCORES_ALL replaces topk_softmax_separate
 * (kernels/topk_softmax_baseline.py:15-36: softmax over all experts, then
 * top-K; here the order is by logit, which only refines the order of the
 * rounded probabilities) with one extra pass over the rows;
 * MOE_SCORES_TOPK_RENORM replaces topk_softmax_conv_a_renorm (:223-237),
 * algebraically equal to Convention B, and computes exactly that. */
int moe_topk_softmax_ex(const void* logits, int logits_dtype, int64_t M, int64_t N,
                        int64_t ld, int64_t K, float* scores, void* indices,
                        int idx_dtype, int algo, int score_mode, void* workspace,
                        size_t ws_bytes, void* stream);

/* Workspace bytes moe_route_sort needs for R routed rows over E experts. */
size_t moe_route_sort_workspace_size(int64_t R, int64_t E);

/* Workspace bytes moe_grouped_gemm needs for R = T*topk routed rows over E
 * experts with output width I. */
size_t moe_grouped_gemm_workspace_size(int64_t T, int64_t topk, int64_t E, int64_t I);

/* Device-side counting sort of routed rows by expert: the segment-offset
 * pass that replaces the host-side argsort / bincount().tolist() / Python
 * offset loops of grouped_gemm_tilelang_v2 and grouped_gemm_pytorch
 * (kernels/grouped_gemm_tilelang.py:562-569, :700-729).
 *
 *   expert_ids  [R] expert id per row, idx_dtype MOE_I32 or MOE_I64
 *   counts      [E]   rows per expert                       (int32, out)
 *   offsets     [E+1] exclusive prefix sum of counts; offsets[E] = number
 *               of rows whose id lies in [0, E)              (int32, out)
 *   sorted_rows [R]   row numbers grouped by expert: rows of expert e are
 *               sorted_rows[offsets[e] .. offsets[e+1]), in ascending row
 *               order; rows with an id outside [0, E) follow in ascending
 *               order at sorted_rows[offsets[E] .. R)         (int32, out)
 *   workspace   >= moe_route_sort_workspace_size(R, E) bytes
 *   Limits: R < 2^31, 1 <= E <= 4096.
 */
int moe_route_sort(const void* expert_ids, int idx_dtype, int64_t R, int64_t E,
                   int32_t* counts, int32_t* offsets, int32_t* sorted_rows,
                   void* workspace, size_t ws_bytes, void* stream);

/* Expert grouped GEMM: Y[r, :] = X[r / topk, :] @ W[expert_ids[r], :, :]^T
 *
 * Replaces grouped_gemm_best (kernels/grouped_gemm_tilelang.py:859-890) and
 * both of its branches, grouped_gemm_tilelang_v2 (:682-766) and the E>64
 * per-expert torch.mm loop grouped_gemm_pytorch (:542-601).  Semantics are
 * those of grouped_gemm_loop (kernels/grouped_gemm_baseline.py:14-57):
 * fp32 accumulation, output in the input dtype, rows whose expert id lies
 * outside [0, E) are zero.  topk == 1 is exactly the reference's 1-D
 * signature (X [R, H], expert_ids [R]); topk > 1 gathers token r / topk of
 * X [T, H] for routed row r of expert_ids [T, topk] (the identity
 * grouped_gemm(X.repeat_interleave(topk, 0), W, ids.flatten())).
 *
 *   X           [T, H] row-major, dtype MOE_BF16 or MOE_F16, 16-byte aligned
 *   W           [E, I, H] row-major, same dtype, 16-byte aligned
 *   expert_ids  [T*topk], idx_dtype MOE_I32 or MOE_I64
 *   Y           [T*topk, I] row-major, same dtype as X
 *   H must be a multiple of 8; T*H and I*H at most 2^35 elements each
 *   (64 GiB of X, or of one expert's weights); MOE_EUNSUP beyond.
 */
int moe_grouped_gemm(const void* X, const void* W, const void* expert_ids,
                     int dtype, int idx_dtype, int64_t T, int64_t topk, int64_t H,
                     int64_t I, int64_t E, void* Y, void* workspace,
                     size_t ws_bytes, void* stream);

/* The grouped GEMM of moe_grouped_gemm without its routing sort: it runs on
 * the routing tables that the previous moe_grouped_gemm call on the same
 * workspace built, which must have had the same expert_ids, T, topk, I and E
 * (with nothing else using the workspace since).  The reference's
 * benchmark does its routing once outside the timed region
 * (benchmarks/benchmark_grouped_gemm.py:116-130, argsort + bincount); this
 * is that split on the device, for callers that apply several weight sets
 * to one routing and for GEMM-only timing.  Arguments as moe_grouped_gemm.
 */
int moe_grouped_gemm_routed(const void* X, const void* W, int dtype, int64_t T,
                            int64_t topk, int64_t H, int64_t I, int64_t E, void* Y,
                            void* workspace, size_t ws_bytes, void* stream);

/* moe_grouped_gemm without the workspace arguments; it calls no allocating
 * routine.  It has no counterpart in the reference: it is for callers that
 * cannot allocate device memory (code under HIP graph capture, serving
 * loops, harnesses that forbid hipMalloc).  The workspace lives in a
 * file-scope device array of MOE_NOALLOC_SCRATCH_BYTES per device, held
 * from the first call on a device until the process ends.  Problems whose
 * workspace (moe_grouped_gemm_workspace_size) exceeds it are rejected with
 * MOE_EUNSUP (beyond about 990K routed rows at E = 256, 740K at E = 4096).  All
 * calls on one device share the array: calls that overlap in time on one
 * device (concurrent streams, or host threads) race and must not be
 * issued.  The current device must be the stream's device.  Arguments as
 * moe_grouped_gemm. */
#define MOE_NOALLOC_SCRATCH_BYTES (4u << 20)
int moe_grouped_gemm_noalloc(const void* X, const void* W, const void* expert_ids,
                             int dtype, int idx_dtype, int64_t T, int64_t topk,
                             int64_t H, int64_t I, int64_t E, void* Y, void* stream);

/* ---------------------------------------------------------------------
 * Router GEMM (logits = X . W) and the fused router GEMM + TopK + softmax.
 * The weights are used transposed, Wt [E, H], so that both MFMA operands
 * are K-contiguous; moe_router_weight_transpose builds Wt from the
 * reference's W [H, E] (a caller keeps Wt while W is unchanged).
 * ------------------------------------------------------------------- */

/* Wt [E, H] = W [H, E]^T (dtype MOE_BF16 or MOE_F16; W rows ldw >= E
 * elements apart, so a column-padded W [H, E_padded] is read in place).
 * Replaces the per-call weight padding of the reference's router wrappers
 * (_pad_W, kernels/router_gemm_topk_softmax.py:1160-1166): any E works, no
 * power-of-two padding is needed. */
int moe_router_weight_transpose(const void* W, int dtype, int64_t H, int64_t E,
                                int64_t ldw, void* Wt, void* stream);

/* Workspace bytes moe_router_gemm / moe_router_topk_softmax need for T
 * tokens (split-H partial tiles when T is small; always >= 4096). */
size_t moe_router_workspace_size(int64_t T, int64_t H, int64_t E);

/* logits [T, E] fp32 = X [T, H] . Wt [E, H]^T, fp32 accumulation.
 * Replaces router_gemm_kernel / get_router_gemm_kernel
 * (kernels/router_gemm_topk_softmax.py:78-145), which writes fp32 logits
 * of the padded width E_padded; here the output is exactly [T, E].
 *   X, Wt   dtype MOE_BF16 or MOE_F16, 16-byte aligned; H a multiple of 8.
 */
int moe_router_gemm(const void* X, const void* Wt, int dtype, int64_t T,
                    int64_t H, int64_t E, float* logits, void* workspace,
                    size_t ws_bytes, void* stream);

/* Fused router: per token, the K largest logits of X . Wt^T, their softmax
 * (Convention B, as moe_topk_softmax) and their expert indices; the logits
 * never leave LDS.
 * Replaces the fused kernels returned by get_fused_router_kernel
 * (kernels/router_gemm_topk_softmax.py:1169-1203: cpasync/tma/tma_auto x
 * selection/bitonic, :148-1150).  Results equal
 * moe_topk_softmax(moe_router_gemm(X, Wt)): indices bit-exact (ties to the
 * lower expert index; the reference's fused kernels pick the higher one,
 * :224-229), scores to fp32 rounding.
 *   scores  [T, K] fp32; indices [T, K] idx_dtype MOE_I32 or MOE_I64.
 *   Limits: E <= 256, K <= 32 (MOE_EUNSUP beyond: use moe_router_gemm and
 *   moe_topk_softmax).
 */
int moe_router_topk_softmax(const void* X, const void* Wt, int dtype, int64_t T,
                            int64_t H, int64_t E, int64_t K, float* scores,
                            void* indices, int idx_dtype, void* workspace,
                            size_t ws_bytes, void* stream);

/* Grouped GEMM with the SwiGLU epilogue:
 *   Y[r, :] = silu(X[r/topk] Wg[e]^T) * (X[r/topk] Wu[e]^T),  e = expert_ids[r]
 * one kernel, fp32 accumulation, output in the input dtype.  Replaces step 1
 * of the reference's routed-expert kernel (kernels/fusedmoe_tilelang.py:147-203:
 * gate and up GEMMs, SiLU(gate) * up, stored as up_logits) and its shared-
 * expert counterpart (:39-121).  Same arguments and workspace as
 * moe_grouped_gemm with Wg, Wu [E, I, H]; rows with an id outside [0, E)
 * are zero. */
int moe_grouped_gemm_swiglu(const void* X, const void* Wg, const void* Wu,
                            const void* expert_ids, int dtype, int idx_dtype,
                            int64_t T, int64_t topk, int64_t H, int64_t I,
                            int64_t E, void* Y, void* workspace, size_t ws_bytes,
                            void* stream);

/* out[t, :] = S[t, :] + sum_j w[t, j] * Yr[t*k + j, :]   (S may be NULL)
 * fp32 sums in a fixed order (deterministic), output in dtype.  Replaces the
 * weighting and scatter_reduce combine of the reference's routed experts
 * (kernels/fusedmoe_tilelang.py:227-229, :413-423).
 *   Yr [T*k, D], S [T, D], out [T, D] dtype MOE_BF16/F16; w [T, k] fp32. */
int moe_combine(const void* Yr, const void* S, const float* w, int dtype, int64_t T,
                int64_t k, int64_t D, void* out, void* stream);

/* Workspace bytes of moe_fused_moe (control block, scratch, intermediates). */
size_t moe_fused_moe_workspace_size(int64_t T, int64_t Dh, int64_t De, int64_t Ds,
                                    int64_t E, int64_t k);

/* Routed-expert FFN with a shared expert: out [T, Dh] for x [T, Dh].
 * Replaces FusedMoETileLang.forward / fusedmoe_best
 * (kernels/fusedmoe_tilelang.py:309-425, :654-690) with the semantics of
 * fusedmoe_pytorch (kernels/fusedmoe_baseline.py:41-168): router logits
 * x . router_w^T, Convention-A softmax top-k (softmax over all E, then the k
 * largest), routed experts silu(x Wg^T) * (x Wu^T) . Wd^T weighted by their
 * scores, plus the shared expert on every token.  The router works in fp32
 * (the reference rounds its logits and softmax to the input dtype).
 *   router_w [E, Dh]; shared_gate, shared_up [Ds, Dh]; shared_down [Dh, Ds]
 *   (Ds = 0: no shared expert); routed_gate, routed_up [E, De, Dh];
 *   routed_down [E, Dh, De]; all dtype, 16-byte aligned; Dh, De, Ds
 *   multiples of 8.  topk_weights [T, k] fp32 and topk_ids [T, k] int32
 *   receive the routing when not NULL. */
int moe_fused_moe(const void* x, const void* router_w, const void* shared_gate,
                  const void* shared_up, const void* shared_down, const void* routed_gate,
                  const void* routed_up, const void* routed_down, int dtype, int64_t T,
                  int64_t Dh, int64_t De, int64_t Ds, int64_t E, int64_t k, void* out,
                  float* topk_weights, void* topk_ids, void* workspace, size_t ws_bytes,
                  void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MOE_HIP_H */
