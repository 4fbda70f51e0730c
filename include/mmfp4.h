/*
 * mmfp4.h -- C ABI of libmmfp4.so, the gfx950 (MI355X) FP4-E2M1 / INT4
 * dequant-GEMM library and its MoE grouped-expert variant.
 *
 * Every entry point is asynchronous on the caller's HIP stream (`stream` is a
 * hipStream_t passed as void*; NULL = the default stream) and returns 0 on
 * success, 1 for an invalid argument, 2 for a launch failure; the message is
 * then available from mm_last_error() (thread-local).  Pointers are device
 * pointers; fp16 data is passed as uint16_t bit patterns.
 *
 * Data layout is the reference's "Marlin" layout:
 *   B       uint32 [K/8, N]   word (kp, n) holds rows k = 8kp+i in bits 4i..4i+3
 *   scales  fp16   [K/g, N]   (g = group_size along K)
 *   zeros   fp16   [K/g, N]   (INT4 only)
 *   A       fp16   [M, K] row-major, C fp16 [M, N] row-major
 */
#ifndef MMFP4_H
#define MMFP4_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Message of the last failing call on this thread ("" if none). */
const char* mm_last_error(void);

/* ---------------------------------------------------------------- dequant */

/* W[K,N] fp16 = fp16_RNE(E2M1[code] * scale), non-finite -> +0.
 * Replaces metal_marlin/kernels_core.py:2079-2133 (dequant_fp4, inline kernel
 * :747-791) and metal_marlin/metal_marlin.py:580-612 (dequant_fp4_bulk). */
int mm_fp4_dequant(const uint32_t* B, const uint16_t* scales, uint16_t* W, int K, int N,
                   int group_size, void* stream);

/* W[K,N] fp16 = fp16_RNE(fp16(q - clamp(z, +-127)) * s), non-finite -> +0.
 * Replaces metal_marlin/metal_marlin.py:615-678 (dequant_int4_bulk) and
 * :283-348 (unpack_u4_weights), kernel src/marlin_gemm.metal:1984-2012. */
int mm_u4_dequant(const uint32_t* B, const uint16_t* scales, const uint16_t* zeros, uint16_t* W,
                  int K, int N, int group_size, void* stream);

/* ---------------------------------------------------------------- quantize */

/* FP4 E2M1 quantizer from W[N,K] (fp16, or fp32 when w_is_f32 != 0) into
 * B[K/8,N] + scales[K/g,N].  Replaces metal_marlin/quantize_fp4.py:131-284
 * (quantize_fp4, weight-only path). */
int mm_fp4_quantize(const void* W, int w_is_f32, int N, int K, int group_size, uint32_t* B,
                    uint16_t* scales, void* stream);

/* Calibration-aware FP4 quantizer (the activation_ranges branch of
 * metal_marlin/quantize_fp4.py:205-256), same layouts as mm_fp4_quantize.
 * The host passes the constants numpy would derive from the calibration dict:
 *   use_pct, kprev, knext, gamma  percentile group max: numpy's 'linear'
 *                  interpolation between the kprev-th and knext-th smallest
 *                  |w| of a group with float32 weight gamma (use_pct 0: absmax)
 *   mode           0: no input range; 1: act > 1, float32 blend
 *                  c1 * gmax + c2 * gmax (c1 = f32(1 - sf), c2 = f32(sf));
 *                  2: act <= 1, float64 blend f32(c1 * gmax) + sf * gmax * att,
 *                  att = sqrt(act), and a float64 scale division
 * Scales are fp16(group max / 6), codes the nearest E2M1 of
 * w / f32(group max) * 6. */
int mm_fp4_quantize_calibrated(const void* W, int w_is_f32, int N, int K, int group_size,
                               int use_pct, int kprev, int knext, float gamma, int mode,
                               float c1, float c2, double sf, double att, uint32_t* B,
                               uint16_t* scales, void* stream);

/* Asymmetric INT4 quantizer from W[N,K] fp16 into B, scales, zeros.
 * Replaces metal_marlin/metal_marlin.py:184-280 (pack_u4_weights). */
int mm_u4_quantize(const uint16_t* W, int N, int K, int group_size, uint32_t* B,
                   uint16_t* scales, uint16_t* zeros, void* stream);

/* ------------------------------------------------------------------- GEMM */

/* Bytes of workspace mm_fp4_gemm / mm_u4_gemm need for this shape.  The
 * workspace starts with split-K arrival counters that must be zero before the
 * first use; every call leaves them at zero again, so one workspace can be
 * reused by consecutive calls on the same stream (not by concurrent calls). */
size_t mm_gemm_workspace_bytes(int M, int N, int K);

/* C[M,N] = A[M,K] . dequant_fp4(B, scales), fp32 accumulation, fp16 out.
 * Replaces metal_marlin/kernels_core.py:1830-1937 (marlin_gemm_fp4),
 * metal_marlin/metal_dispatch.py:4045-4181 (dispatch_gemm_fp4), :3914-4042
 * (_dispatch_decode_gemv_fp4), :1791-1861 (MetalKernelLibrary.fp4_gemm) and
 * the native FFI metal_marlin/cpp_extension.cpp:502-527 (_cpp_ext.mmfp4_gemm).
 * Requires K % 8 == 0, N % 4 == 0, group_size % 8 == 0, K % group_size == 0;
 * A, B 16-byte aligned; scales, C 8-byte aligned. */
int mm_fp4_gemm(const uint16_t* A, const uint32_t* B, const uint16_t* scales, uint16_t* C, int M,
                int N, int K, int group_size, void* ws, size_t ws_bytes, void* stream);

/* C[M,N] = A[M,K] . dequant_fp4(B, scales)^T for row-packed (MMFP4) weights:
 * B [N, K/8] uint32 (word (n, kp) holds k = 8kp .. 8kp+7 of row n), scales
 * fp16 [K/g, N] (scales_layout = 0, the layer's canonical [n_groups, N]) or
 * [N, K/g] (scales_layout = 1, the transposed layout the layer also accepts,
 * metal_marlin/layers/mmfp4_linear.py:53-86).  N % 4 == 0; M <= 32 runs the
 * decode kernels (g % 32 == 0), larger M the pipelined prefill kernel, which
 * needs g % 64 == 0, N % 8 == 0 and scales_layout 0.  Weights and scales are
 * read in place at every M (no transpose).  Workspace as
 * mm_gemm_workspace_bytes(M, N, K).  Replaces
 * metal_marlin/layers/mmfp4_linear.py:549-598 (mmfp4_gemm), which transposes
 * the row-packed words to the [K/8, N] layout on every call (:414-478). */
int mm_fp4_gemm_rowpacked(const uint16_t* A, const uint32_t* B, const uint16_t* scales,
                          uint16_t* C, int M, int N, int K, int group_size, int scales_layout,
                          void* ws, size_t ws_bytes, void* stream);

/* mm_fp4_gemm without a workspace argument, for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  No counterpart in the reference.  The split-K counters and
 * partial sums live in a 32 MiB device array built into the library (one copy
 * per device, held until the process ends); a shape whose
 * mm_gemm_workspace_bytes(M, N, K) exceeds 32 MiB is refused (status 1).  The
 * call makes no allocation.  All calls on one device share that device's
 * array, so calls that overlap on a device (several streams or threads) race.
 * Otherwise as mm_fp4_gemm, with the same results. */
int mm_fp4_gemm_noalloc(const uint16_t* A, const uint32_t* B, const uint16_t* scales, uint16_t* C,
                        int M, int N, int K, int group_size, void* stream);

/* INT4 asymmetric counterpart.  Replaces metal_marlin/kernels_core.py:1959-2066
 * (marlin_gemm_int4) and metal_marlin/metal_dispatch.py:1863-1937
 * (MetalKernelLibrary.int4_gemm). */
int mm_u4_gemm(const uint16_t* A, const uint32_t* B, const uint16_t* scales,
               const uint16_t* zeros, uint16_t* C, int M, int N, int K, int group_size, void* ws,
               size_t ws_bytes, void* stream);

/* mm_u4_gemm with the scales and zero points also given interleaved,
 * SZ[K/g, N/4, 8] fp16 (16-byte aligned): for each 4-column group its 4
 * scales then its 4 zero points.  The decode kernels (M <= 32) then load one
 * 16-byte piece per group instead of two 8-byte ones; the prefill kernels read
 * S and Z.  Results are bit-identical to mm_u4_gemm.  Replaces the same
 * reference interface as mm_u4_gemm (kernels_core.py:1959-2066); the
 * interleaved copy is a layout cache the Python layer keeps per (scales,
 * zeros) pair. */
int mm_u4_gemm_sz(const uint16_t* A, const uint32_t* B, const uint16_t* scales,
                  const uint16_t* zeros, const uint16_t* SZ, uint16_t* C, int M, int N, int K,
                  int group_size, void* ws, size_t ws_bytes, void* stream);

/* Gate and up projections over two packed FP4 matrices (Marlin [K/8, N],
 * scales [K/g, N]) in one launch, reading A once:
 *   act = 1:  C[M, N]  = silu(A . dequant(Bg, Sg)) * (A . dequant(Bu, Su))
 *             (SiLU on the fp32 sums);
 *   act = 0:  C[M, 2N] = [A . dequant(Bg, Sg) | A . dequant(Bu, Su)].
 * Replaces metal_marlin/kernels_core.py:4749-4774 (fused_gate_up_gemm,
 * mmfp4_fused_gate_up) -> MetalKernels.fused_gate_up_gemm :4220-4267 and
 * .mmfp4_fused_gate_up :4269-4408.  Workspace: mm_gemm_workspace_bytes(M, 2N, K).
 * Requires K % 8 == 0, N % 8 == 0, group_size % 8 == 0, K % group_size == 0,
 * K % 64 == 0 when M > 32; A, weights and scales 16-byte aligned, C 8-byte. */
int mm_fp4_gate_up(const uint16_t* A, const uint32_t* Bg, const uint16_t* Sg, const uint32_t* Bu,
                   const uint16_t* Su, uint16_t* C, int M, int N, int K, int group_size, int act,
                   void* ws, size_t ws_bytes, void* stream);

/* C[M,N] = A[M,K] . dequant_fp4(B, scales) with Marlin-layout words B
 * [K/8, N] and scales in the transposed [N, K/g] layout, read in place.
 * Decode sizes only (M <= 16); otherwise as mm_fp4_gemm (K % 8 == 0,
 * N % 4 == 0, group_size % 8 == 0 dividing K).  Workspace as
 * mm_gemm_workspace_bytes(M, N, K).  The reference's MMFP4 GEMM
 * (metal_marlin/kernels_core.py:4804-4812 -> MetalKernels.mmfp4_gemm
 * :4550-4633, shaders/mmfp4_gemm.metal:570-588) reads [K/g, N] scales, which
 * mm_fp4_gemm takes; its layer normalises [N, K/g] scales to that layout by a
 * transpose (layers/mmfp4_linear.py:53-86).  This entry point serves callers
 * holding [N, K/g] scales without that transpose. */
int mm_fp4_gemm_mmfp4(const uint16_t* A, const uint32_t* B, const uint16_t* scales, uint16_t* C,
                      int M, int N, int K, int group_size, void* ws, size_t ws_bytes,
                      void* stream);

/* mm_fp4_gate_up for row-packed (MMFP4) gate and up matrices read in place:
 * Bg, Bu [N, K/8] uint32, scales Sg, Su fp16 [K/g, N]; act as mm_fp4_gate_up.
 * N % 8 == 0; M <= 32 runs the decode kernel (g % 32 == 0), larger M the
 * pipelined prefill kernel (g % 64 == 0), both reading the words in place.
 * Workspace: mm_gemm_workspace_bytes(M, 2N, K).  Replaces
 * metal_marlin/kernels_core.py:4762-4774 (mmfp4_fused_gate_up) ->
 * MetalKernels.mmfp4_fused_gate_up :4269-4408 on its row-packed inputs,
 * without a transpose of the weights. */
int mm_fp4_gate_up_rowpacked(const uint16_t* A, const uint32_t* Bg, const uint16_t* Sg,
                             const uint32_t* Bu, const uint16_t* Su, uint16_t* C, int M, int N,
                             int K, int group_size, int act, void* ws, size_t ws_bytes,
                             void* stream);

/* Up to three FP4 products sharing A and K, one output each:
 * C[p] [M, N[p]] = A . dequant(B[p], S[p]), p < nmat <= 3 (B[p] Marlin
 * [K/8, N[p]], S[p] [K/g, N[p]]).  The tables are host arrays of device
 * pointers.  M <= 16 runs one launch over all the matrices' column tiles; larger
 * M runs one launch per matrix.  Replaces metal_marlin/kernels_core.py:4875-4948
 * (mmfp4_fused_qkv) and the Metal shaders/mmfp4_fused_qkv.metal dispatch.
 * Workspace: the larger of mm_gemm_workspace_bytes(M, sum N[p], K) and each
 * mm_gemm_workspace_bytes(M, N[p], K).  Other requirements as mm_fp4_gemm. */
int mm_fp4_gemm_multi(const uint16_t* A, int nmat, const uint32_t* const* B,
                      const uint16_t* const* S, uint16_t* const* C, const int* N, int M, int K,
                      int group_size, void* ws, size_t ws_bytes, void* stream);

/* -------------------------------------------------------------------- MoE */

/* Stable counting sort of the T*k (token, slot) assignments by expert.
 * expert_ids int32 [T, k]; outputs offsets int32 [E+1], sorted_idx int32 [T*k]
 * (flat index t*k+slot, ascending within an expert) and inverse int32 [T*k].
 * Replaces metal_marlin/moe_dispatch.py:493-555 (group_tokens_by_expert),
 * :726-786 (group_tokens_by_expert_full) and the Metal moe_gpu_sort
 * (src/moe_dispatch.metal:1600-1626).  Requires E <= 1024.  Ids outside
 * [0, E) (the reference requires them in range) are dropped: they are placed
 * after all experts' rows, in index order, so sorted_idx and inverse remain
 * permutations of the T*k assignments, and offsets[E] counts the valid ones. */
int mm_moe_sort(const int32_t* expert_ids, int T, int k, int E, int32_t* offsets,
                int32_t* sorted_idx, int32_t* inverse, void* stream);

/* mm_moe_sort for int64 expert ids (what torch.topk returns), so callers
 * need no conversion launch.  Same outputs and errors; replaces the same
 * reference functions. */
int mm_moe_sort_i64(const int64_t* expert_ids, int T, int k, int E, int32_t* offsets,
                    int32_t* sorted_idx, int32_t* inverse, void* stream);

/* Bytes of workspace mm_moe_router needs for T tokens (zeroed once before
 * first use; the kernel leaves its arrival counters at zero).  It may be the
 * same buffer as the GEMMs' workspace on the same stream. */
size_t mm_moe_router_workspace_bytes(int T, int H, int E);

/* Router: logits = X[T, H] . W[E, H]^T (+ bias[E] fp32, may be NULL), fp32
 * accumulate, rounded to fp16 (the gate nn.Linear's output dtype); fp32
 * softmax over the E experts; top-k descending (lower expert id first on
 * ties); renorm != 0 divides the k probabilities by their sum.  ids int64
 * [T, k], probs fp32 [T, k].  One launch.  Requires H % 32 == 0, E <= 1024,
 * 1 <= k <= min(E, 64); X, W 16-byte aligned.  Replaces
 * metal_marlin/moe_dispatch.py:178-219 (_fused_router_topk) and :328-449
 * (_fused_router_topk_metal, kernel moe_fused_router_sorted), and
 * metal_marlin/kernels/moe.py:729-740 (moe_router_topk). */
int mm_moe_router(const uint16_t* X, const uint16_t* W, const float* bias, int T, int H, int E,
                  int k, int renorm, int64_t* ids, float* probs, void* ws, size_t ws_bytes,
                  void* stream);

/* Softmax + top-k of given logits [T, E] (fp16, or fp32 when logits_f32),
 * same selection and outputs as mm_moe_router.  Replaces
 * metal_marlin/moe_dispatch.py:99-151 (_router_softmax_fusion) and
 * metal_marlin/kernels_core.py:241-247 / :966 (mmfp4_softmax_topk). */
int mm_softmax_topk(const void* logits, int logits_f32, int T, int E, int k, int renorm,
                    int64_t* ids, float* probs, void* stream);

/* Grouped expert GEMM over expert-sorted rows.  For expert e, rows
 * r in [offsets[e], offsets[e+1]) compute Y[r] = X[row(r)] . dequant(B[e], S[e]),
 * where row(r) = sorted_idx[r] / k when gather != 0 (rows of X are tokens)
 * and row(r) = r otherwise (X already in sorted order).  B: uint32 [E, K/8, N],
 * S: fp16 [E, K/g, N].  act = 0: Y is [T*k, N];  act = 1 (SwiGLU): the first
 * N/2 columns are gate and the last N/2 up, Y[r, j] = silu(gate_j) * up_j is
 * [T*k, N/2].  Replaces metal_marlin/kernels/moe.py:583-727
 * (moe_expert_gemm_fp4, kernel src/moe_expert_gemm.metal:557-782) and the
 * expert MLP of metal_marlin/moe_dispatch.py:1241-1431 (_fused_expert_mlp).
 * Status 1 when one expert's packed weights reach 4 GiB, or when gather != 0,
 * the groups are decode-sized (at most 24 rows per expert on average) and X
 * (T rows of K halves) reaches 2 GiB. */
int mm_moe_grouped_gemm(const uint16_t* X, const int32_t* sorted_idx, const int32_t* offsets,
                        int gather, int k, int T, const uint32_t* B, const uint16_t* S, int E,
                        int K, int N, int group_size, int act, uint16_t* Y, void* stream);

/* out[t, :] = sum_{j<k} probs[t, j] * Y[inverse[t*k + j], :] in fp32 (fixed
 * slot order, deterministic), written as fp16 [T, H].  Replaces
 * metal_marlin/moe_dispatch.py:812-925 (scatter_expert_outputs /
 * _aggregate_expert_outputs).  Every slot is read, including those of
 * dropped ids (their Y rows are whatever the caller wrote there). */
int mm_moe_combine(const uint16_t* Y, const float* probs, const int32_t* inverse, int T, int k,
                   int H, uint16_t* out, void* stream);

/* Routed-expert SwiGLU MLP over all experts in one call:
 *   h = X[t] . W_gu[e] ([E, H/8, 2I] packed, scales [E, H/g, 2I]);
 *   a = silu(h[:I]) * h[I:];  y = a . W_dn[e] ([E, I/8, H], scales [E, I/g, H]);
 *   out[t] = sum_j probs[t, j] * y(t, j)   (fp32, slot order; fp16 [T, H]).
 * expert_ids [T, k] int32 (ids_i64 = 0) or int64 (ids_i64 = 1); probs fp32
 * [T, k].  Scratch the caller provides: act_buf fp16 [T*k, I], y_buf fp16
 * [T*k, H], sort_buf int32 [E + 1 + 2*T*k].  Four launches (sort, gate_up,
 * down, combine), the same as mm_moe_sort + 2 x mm_moe_grouped_gemm +
 * mm_moe_combine.  Replaces metal_marlin/moe_dispatch.py:1241-1431
 * (_fused_expert_mlp) with the combine of :812-925. */
int mm_moe_mlp_fp4(const uint16_t* X, const void* expert_ids, int ids_i64, const float* probs,
                   int T, int k, int E, int H, int I, const uint32_t* Bgu, const uint16_t* Sgu,
                   const uint32_t* Bdn, const uint16_t* Sdn, int group_size, uint16_t* act_buf,
                   uint16_t* y_buf, int32_t* sort_buf, uint16_t* out, void* stream);

/* mm_moe_mlp_fp4 plus a shared expert that every token visits:
 *   out[t] = base[t] + sum_j probs[t, j] * y_routed(t, j) + shared_weight * y_shared(t)
 * with y_shared(t) = (silu(h[:I]) * h[I:]) . W_sdn, h = X[t] . W_sgu, W_sgu
 * [H/8, 2I] packed (scales [H/g, 2I]), W_sdn [I/8, H] (scales [I/g, H]).  The
 * shared expert runs as one more expert group in the same two grouped
 * launches as the routed experts.  k may be 0 (shared expert alone: E may
 * then be 0, and expert_ids, probs and the routed weights may be NULL);
 * base (fp16 [T, H]) may be NULL.  Scratch: act_buf fp16 [T*(k+1), I], y_buf
 * fp16 [T*(k+1), H], sort_buf int32 [E + 2 + 2*T*(k+1)].  Replaces
 * metal_marlin/kernels/moe.py:742-856 (moe_fused_dispatch_shared_fp4),
 * :442-582 (moe_shared_expert_fp4), :858-930 (moe_add_shared_expert_fp4) and
 * the forward of metal_marlin/moe_dispatch.py:1111-1238 (FusedMoEDispatcher). */
int mm_moe_mlp_shared_fp4(const uint16_t* X, const void* expert_ids, int ids_i64,
                          const float* probs, int T, int k, int E, int H, int I,
                          const uint32_t* Bgu, const uint16_t* Sgu, const uint32_t* Bdn,
                          const uint16_t* Sdn, const uint32_t* Bsgu, const uint16_t* Ssgu,
                          const uint32_t* Bsdn, const uint16_t* Ssdn, float shared_weight,
                          const uint16_t* base, int group_size, uint16_t* act_buf,
                          uint16_t* y_buf, int32_t* sort_buf, uint16_t* out, void* stream);

/* Shared + routed aggregation of one FP4 projection (no MLP):
 *   out[t] = X[t] . W_sh + sum_j probs[t, j] * (X[t] . W_routed[e(t, j)])
 * W_sh [K/8, N] packed (scales Ssh [K/g, N]); W_routed [E, K/8, N] (scales
 * [E, K/g, N]); expert_ids [T, k] int32 (ids_i64 = 0) or int64 (ids_i64 = 1),
 * probs fp32 [T, k]; fp32 sums in slot order, fp16 out [T, N].  Ids outside
 * [0, E) contribute nothing.  N % 8 == 0.  Scratch: y_buf fp16 [T*(k+1), N],
 * sort_buf int32 [E + 2 + 2*T*(k+1)].  Three launches (sort, one grouped
 * launch over the routed and shared groups, combine).  Replaces
 * metal_marlin/kernels/moe.py:182-329 (moe_shared_expert_fused_fp4, kernel
 * src/moe_shared_expert.metal:604-). */
int mm_moe_gemm_shared_fp4(const uint16_t* X, const void* expert_ids, int ids_i64,
                           const float* probs, int T, int k, int E, int K, int N,
                           const uint32_t* Bsh, const uint16_t* Ssh, const uint32_t* B,
                           const uint16_t* S, int group_size, uint16_t* y_buf, int32_t* sort_buf,
                           uint16_t* out, void* stream);

/* ------------------------------------------- flat-group FP4 (FP4Metal) */

/* Quantizes n values (dtype 0 f32, 1 fp16, 2 bf16) in flat groups of
 * group_size over the flattened tensor, the last group padded with zeros:
 * scales[i] = max(max|x| / 6, 1e-8) in f32 (NaN when the group holds a NaN),
 * codes[j] = (v < 0 ? 8 : 0) | nearest positive E2M1 index of |v| (ties to the
 * lower index) for v = x[j] / scales[j / group_size].  codes: n bytes;
 * scales: ceil(n / group_size) floats.  Replaces metal_marlin/fp4_metal.py:
 * 130-190 (FP4Metal.quantize). */
int mm_fp4_flat_quantize(const void* x, size_t n, int dtype, int group_size, uint8_t* codes,
                         float* scales, void* stream);

/* out[j] = E2M1[codes[j] & 15] * scales[j / group_size] in f32; requires
 * nscales * group_size >= n.  Replaces metal_marlin/fp4_metal.py:192-276
 * (FP4Metal.dequantize). */
int mm_fp4_flat_dequantize(const uint8_t* codes, const float* scales, size_t n, size_t nscales,
                           int group_size, float* out, void* stream);

/* out[j] = (lo[j] & 15) | ((hi[j] & 15) << 4).  Replaces
 * metal_marlin/fp4_metal.py:278-300 (FP4Metal.pack_pair). */
int mm_fp4_pack_pair(const uint8_t* lo, const uint8_t* hi, size_t n, uint8_t* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MMFP4_H */
