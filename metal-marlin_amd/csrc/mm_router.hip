// Fused MoE router for gfx950: router GEMM (fp16 MFMA, fp32 accumulate) ->
// fp32 softmax over the experts -> top-k (descending, lower expert id first
// on ties) -> optional renormalisation, one launch; plus the softmax/top-k
// part alone for callers that already hold the logits.
//
// Reference: metal_marlin/moe_dispatch.py:178-219 (_fused_router_topk: the
// gate nn.Linear, then _router_softmax_fusion :99-151), :328-449
// (_fused_router_topk_metal / the moe_fused_router_sorted kernel),
// metal_marlin/kernels/moe.py:729-740 (moe_router_topk), and
// metal_marlin/kernels_core.py:966-1100 (the mmfp4_softmax_topk kernel).
// As in the reference's torch path, the logits are rounded to the gate's
// output dtype (fp16) before the softmax.
#include "mm_common.h"

namespace {

constexpr int RT_TOK = 16;       // tokens per block (one MFMA row tile)
constexpr int RT_WAVES = 4;
constexpr int RT_MAXK = 64;      // top-k limit (one lane per selected expert)

// Wave-wide argmax of (value, index), ties to the lower index.
MM_DEV void wave_argmax(float& v, int& i) {
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) {
    const float ov = __shfl_xor(v, d);
    const int oi = __shfl_xor(i, d);
    if (ov > v || (ov == v && oi < i)) {
      v = ov;
      i = oi;
    }
  }
}

MM_DEV float wave_max(float v) {
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) v = fmaxf(v, __shfl_xor(v, d));
  return v;
}

MM_DEV float wave_sum(float v) {
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) v += __shfl_xor(v, d);
  return v;
}

// One wave: softmax + top-k of one token's logits row `lg` (fp32, E
// entries, already rounded as the reference rounds them) -> ids / probs.
MM_DEV void softmax_topk_row(const float* lg, int E, int k, int renorm, int64_t* ids,
                             float* probs) {
  const int lane = threadIdx.x & 63;
  float mx = -INFINITY;
  for (int e = lane; e < E; e += 64) mx = fmaxf(mx, lg[e]);
  mx = wave_max(mx);
  float sum = 0.0f;
  for (int e = lane; e < E; e += 64) sum += expf(lg[e] - mx);
  sum = wave_sum(sum);
  // Candidates: each lane keeps its slice of the experts; the k rounds pick
  // the largest remaining probability across the wave.
  // Round r's winner is kept by lane r; the owner lane of an expert marks it
  // taken.
  float taken_sum = 0.0f, my_p = 0.0f;
  int my_i = 0;
  uint64_t used = 0;                   // this lane's taken slots e = lane + 64*slot (E <= 4096)
  for (int r = 0; r < k; ++r) {
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    int slot = 0;
    for (int e = lane; e < E; e += 64, ++slot) {
      if ((used >> slot) & 1ull) continue;
      const float p = expf(lg[e] - mx) / sum;
      if (p > bv || (p == bv && e < bi)) {
        bv = p;
        bi = e;
      }
    }
    wave_argmax(bv, bi);
    if ((bi & 63) == lane) used |= 1ull << (bi >> 6);
    if (lane == r) {
      my_p = bv;
      my_i = bi;
    }
    taken_sum += bv;
  }
  if (lane < k) {
    ids[lane] = my_i;
    probs[lane] = renorm ? my_p / taken_sum : my_p;
  }
}

// grid = ceil(T / 16) blocks of 4 waves.  X [T, H] fp16 row-major, W [E, H]
// fp16 row-major (nn.Linear weight), bias [E] fp32 or null.  Wave w computes
// the logits of the block's 16 tokens for expert tiles w, w+4, ... (16
// experts each) with MFMA 16x16x32; the logits go through LDS; then each wave
// runs softmax + top-k for 4 of the tokens.
__global__ void __launch_bounds__(RT_WAVES * 64)
k_moe_router(const f16* __restrict__ X, const f16* __restrict__ W, const float* __restrict__ bias,
             int T, int H, int E, int k, int renorm, int64_t* __restrict__ ids,
             float* __restrict__ probs) {
  extern __shared__ float lg[];                 // [RT_TOK][E]
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int c = lane & 15, q = lane >> 4;
  const int t0 = blockIdx.x * RT_TOK;
  const int ntile = (E + 15) / 16;
  const f16* xrow = X + (size_t)min(t0 + c, T - 1) * H;     // A operand row of this lane
  for (int tile = wave; tile < ntile; tile += RT_WAVES) {
    const int e = min(tile * 16 + c, E - 1);                // B operand column (expert)
    const f16* wrow = W + (size_t)e * H;
    f32x4 acc = {0, 0, 0, 0};
    for (int k0 = 0; k0 < H; k0 += 32) {
      const f16x8 a = *(const f16x8*)(xrow + k0 + 8 * q);
      const f16x8 b = *(const f16x8*)(wrow + k0 + 8 * q);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc, 0, 0, 0);
    }
    // acc[j]: token 4*q + j, expert tile*16 + c.
    const int ec = tile * 16 + c;
    if (ec < E) {
      const float bb = bias != nullptr ? bias[ec] : 0.0f;
#pragma unroll
      for (int j = 0; j < 4; ++j) lg[(4 * q + j) * E + ec] = (float)(f16)(acc[j] + bb);
    }
  }
  __syncthreads();
  for (int r = wave; r < RT_TOK; r += RT_WAVES) {
    const int t = t0 + r;
    if (t >= T) break;
    softmax_topk_row(lg + r * E, E, k, renorm, ids + (size_t)t * k, probs + (size_t)t * k);
  }
}

// Softmax + top-k of given logits [T, E] (fp16 or fp32): one wave per token.
__global__ void __launch_bounds__(RT_WAVES * 64)
k_softmax_topk(const void* __restrict__ logits, int logits_f32, int T, int E, int k, int renorm,
               int64_t* __restrict__ ids, float* __restrict__ probs) {
  extern __shared__ float lg[];                 // [RT_WAVES][E]
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int t = blockIdx.x * RT_WAVES + wave;
  if (t >= T) return;
  float* row = lg + wave * E;
  for (int e = lane; e < E; e += 64)
    row[e] = logits_f32 ? ((const float*)logits)[(size_t)t * E + e]
                        : (float)((const f16*)logits)[(size_t)t * E + e];
  softmax_topk_row(row, E, k, renorm, ids + (size_t)t * k, probs + (size_t)t * k);
}

}  // namespace

// ===========================================================================
// C ABI
// ===========================================================================
extern "C" int mm_moe_router(const uint16_t* X, const uint16_t* W, const float* bias, int T, int H,
                             int E, int k, int renorm, int64_t* ids, float* probs, void* stream) {
  MM_CHECK_ARG(T >= 0 && H > 0 && E > 0, "mm_moe_router: bad shape T=%d H=%d E=%d", T, H, E);
  MM_CHECK_ARG(H % 32 == 0, "mm_moe_router: hidden size %d must be divisible by 32", H);
  MM_CHECK_ARG(E <= 64 * 64, "mm_moe_router: num_experts=%d must be <= 4096", E);
  MM_CHECK_ARG(k >= 1 && k <= RT_MAXK && k <= E, "mm_moe_router: top_k=%d must be in [1, %d]",
               k, E < RT_MAXK ? E : RT_MAXK);
  MM_CHECK_ARG(((uintptr_t)X & 15) == 0 && ((uintptr_t)W & 15) == 0,
               "mm_moe_router: hidden states and router weight must be 16-byte aligned");
  if (T == 0) return 0;
  const size_t lds = (size_t)RT_TOK * E * sizeof(float);
  MM_CHECK_ARG(lds <= 64 * 1024, "mm_moe_router: num_experts=%d too large for one block", E);
  hipLaunchKernelGGL(k_moe_router, dim3(mm_cdiv(T, RT_TOK)), dim3(RT_WAVES * 64), lds,
                     (hipStream_t)stream, (const f16*)X, (const f16*)W, bias, T, H, E, k, renorm,
                     ids, probs);
  MM_CHECK_LAUNCH("mm_moe_router");
  return 0;
}

extern "C" int mm_softmax_topk(const void* logits, int logits_f32, int T, int E, int k,
                               int renorm, int64_t* ids, float* probs, void* stream) {
  MM_CHECK_ARG(T >= 0 && E > 0, "mm_softmax_topk: bad shape T=%d E=%d", T, E);
  MM_CHECK_ARG(E <= 64 * 64, "mm_softmax_topk: num_experts=%d must be <= 4096", E);
  MM_CHECK_ARG(k >= 1 && k <= RT_MAXK && k <= E, "mm_softmax_topk: top_k=%d must be in [1, %d]",
               k, E < RT_MAXK ? E : RT_MAXK);
  if (T == 0) return 0;
  const size_t lds = (size_t)RT_WAVES * E * sizeof(float);
  hipLaunchKernelGGL(k_softmax_topk, dim3(mm_cdiv(T, RT_WAVES)), dim3(RT_WAVES * 64), lds,
                     (hipStream_t)stream, logits, logits_f32, T, E, k, renorm, ids, probs);
  MM_CHECK_LAUNCH("mm_softmax_topk");
  return 0;
}
