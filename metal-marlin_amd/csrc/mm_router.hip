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
constexpr int RT_WAVES = 4;      // softmax/top-k kernel: waves (tokens) per block
constexpr int RT_NW = 4;         // router kernel: waves (tasks) per block
constexpr int RT_MAXSL = 4;      // router kernel: max slices of H per expert tile
constexpr int RT_MAX_TB = 16384; // router kernel: token blocks (arrival counters)
constexpr int RT_FIN = 4;        // router kernel: logits per thread per hand-off batch
constexpr int RT_UNROLL = 8;     // loads issued ahead of their MFMAs
constexpr int RT_MAXK = 64;      // top-k limit (one lane per selected expert)

// Wave reductions without LDS round trips: DPP steps inside each row of 16
// lanes (xor 1, xor 2, mirror within 8, mirror within 16 -- each lane is
// combined with a lane of the other half, so after the four steps every
// lane holds its row's result), then the four row results are read into
// scalars and combined in row order, which leaves the result wave-uniform.
template <int CTRL>
MM_DEV uint32_t dpp_u32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}
template <int CTRL>
MM_DEV float dpp_f(float v) {
  return __uint_as_float(dpp_u32<CTRL>(__float_as_uint(v)));
}
constexpr int DPP_XOR1 = 0xB1, DPP_XOR2 = 0x4E, DPP_HALF_MIRROR = 0x141, DPP_MIRROR = 0x140;

MM_DEV float rowlane_f(float v, int l) {
  return __uint_as_float((uint32_t)__builtin_amdgcn_readlane((int)__float_as_uint(v), l));
}

MM_DEV float wave_max(float v) {
  v = fmaxf(v, dpp_f<DPP_XOR1>(v));
  v = fmaxf(v, dpp_f<DPP_XOR2>(v));
  v = fmaxf(v, dpp_f<DPP_HALF_MIRROR>(v));
  v = fmaxf(v, dpp_f<DPP_MIRROR>(v));
  return fmaxf(fmaxf(rowlane_f(v, 0), rowlane_f(v, 16)), fmaxf(rowlane_f(v, 32), rowlane_f(v, 48)));
}

MM_DEV float wave_sum(float v) {
  v += dpp_f<DPP_XOR1>(v);
  v += dpp_f<DPP_XOR2>(v);
  v += dpp_f<DPP_HALF_MIRROR>(v);
  v += dpp_f<DPP_MIRROR>(v);
  return ((rowlane_f(v, 0) + rowlane_f(v, 16)) + rowlane_f(v, 32)) + rowlane_f(v, 48);
}

// (value, index) as one 64-bit key whose unsigned order is: larger value
// first, then lower index (the float bits are made order-preserving).
MM_DEV uint64_t argmax_key(float v, int i) {
  const uint32_t b = __float_as_uint(v);
  const uint32_t u = b ^ ((uint32_t)((int32_t)b >> 31) | 0x80000000u);
  return ((uint64_t)u << 32) | (uint32_t)~(uint32_t)i;
}
MM_DEV float key_value(uint64_t k) {
  const uint32_t u = (uint32_t)(k >> 32);
  return __uint_as_float((u & 0x80000000u) ? (u ^ 0x80000000u) : ~u);
}
MM_DEV int key_index(uint64_t k) { return (int)~(uint32_t)k; }

template <int CTRL>
MM_DEV uint64_t dpp_keymax(uint64_t k) {
  const uint64_t o = ((uint64_t)dpp_u32<CTRL>((uint32_t)(k >> 32)) << 32) | dpp_u32<CTRL>((uint32_t)k);
  return o > k ? o : k;
}
MM_DEV uint64_t readlane_key(uint64_t k, int l) {
  return ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(k >> 32), l) << 32) |
         (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)k, l);
}
MM_DEV uint64_t wave_keymax(uint64_t k) {
  k = dpp_keymax<DPP_XOR1>(k);
  k = dpp_keymax<DPP_XOR2>(k);
  k = dpp_keymax<DPP_HALF_MIRROR>(k);
  k = dpp_keymax<DPP_MIRROR>(k);
  uint64_t m = readlane_key(k, 0);
  const uint64_t k1 = readlane_key(k, 16), k2 = readlane_key(k, 32), k3 = readlane_key(k, 48);
  m = k1 > m ? k1 : m;
  m = k2 > m ? k2 : m;
  return k3 > m ? k3 : m;
}

// Wave-wide argmax of (value, index), ties to the lower index.
MM_DEV void wave_argmax(float& v, int& i) {
  const uint64_t k = wave_keymax(argmax_key(v, i));
  v = key_value(k);
  i = key_index(k);
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

// NR rows at once (NR independent shuffle chains hide each other's latency):
// softmax + top-k of rows lg + j*rstride, j < NR, each E <= 64*SL entries.
// The probabilities are formed once per expert (exp(l - max) / sum, the same
// expression and summation order as softmax_topk_row) and kept in registers;
// a round is then one register scan and one wave arg-max per row.  Rows
// j >= nvalid are computed but not stored.
template <int NR, int SL>
MM_DEV void softmax_topk_rows(const float* lg, int rstride, int nvalid, int E, int k, int renorm,
                              int64_t* ids, float* probs) {
  const int lane = threadIdx.x & 63;
  float p[NR][SL], mx[NR], sm[NR];
#pragma unroll
  for (int j = 0; j < NR; ++j) {
    mx[j] = -INFINITY;
#pragma unroll
    for (int sl = 0; sl < SL; ++sl) {
      const int e = lane + 64 * sl;
      p[j][sl] = e < E ? lg[j * rstride + e] : -INFINITY;
      mx[j] = fmaxf(mx[j], p[j][sl]);
    }
  }
#pragma unroll
  for (int j = 0; j < NR; ++j) mx[j] = wave_max(mx[j]);
#pragma unroll
  for (int j = 0; j < NR; ++j) {
    sm[j] = 0.0f;
#pragma unroll
    for (int sl = 0; sl < SL; ++sl) {
      if (lane + 64 * sl < E) {
        p[j][sl] = expf(p[j][sl] - mx[j]);
        sm[j] += p[j][sl];
      }
    }
  }
#pragma unroll
  for (int j = 0; j < NR; ++j) sm[j] = wave_sum(sm[j]);
#pragma unroll
  for (int j = 0; j < NR; ++j)
#pragma unroll
    for (int sl = 0; sl < SL; ++sl)          // -1: below every probability, never taken
      p[j][sl] = lane + 64 * sl < E ? p[j][sl] / sm[j] : -1.0f;

  uint32_t used[NR];
  float my_p[NR], taken[NR];
  int my_i[NR];
#pragma unroll
  for (int j = 0; j < NR; ++j) {
    used[j] = 0;
    taken[j] = 0.0f;
    my_p[j] = 0.0f;
    my_i[j] = 0;
  }
  for (int r = 0; r < k; ++r) {
    float bv[NR];
    int bi[NR];
#pragma unroll
    for (int j = 0; j < NR; ++j) {
      bv[j] = -2.0f;
      bi[j] = 0x7fffffff;
#pragma unroll
      for (int sl = 0; sl < SL; ++sl) {
        const float v = p[j][sl];
        if (!((used[j] >> sl) & 1u) && v > bv[j]) {   // slots ascend in e: ties keep the lower
          bv[j] = v;
          bi[j] = lane + 64 * sl;
        }
      }
    }
#pragma unroll
    for (int j = 0; j < NR; ++j) wave_argmax(bv[j], bi[j]);
#pragma unroll
    for (int j = 0; j < NR; ++j) {
      if ((bi[j] & 63) == lane) used[j] |= 1u << (bi[j] >> 6);
      if (lane == r) {
        my_p[j] = bv[j];
        my_i[j] = bi[j];
      }
      taken[j] += bv[j];
    }
  }
  if (lane < k) {
#pragma unroll
    for (int j = 0; j < NR; ++j) {
      if (j >= nvalid) break;
      ids[j * k + lane] = my_i[j];
      probs[j * k + lane] = renorm ? my_p[j] / taken[j] : my_p[j];
    }
  }
}

// Four rows per wave, one per row of 16 lanes (E <= 16*SL): the reductions
// stay inside a DPP row (four steps, no cross-row traffic), so a round of the
// top-k is one register scan and four key-max steps for all four rows.  Lane
// l of row j holds experts (l & 15) + 16*s.  Rows j >= nvalid are computed
// but not stored.
MM_DEV uint64_t row_keymax(uint64_t k) {
  k = dpp_keymax<DPP_XOR1>(k);
  k = dpp_keymax<DPP_XOR2>(k);
  k = dpp_keymax<DPP_HALF_MIRROR>(k);
  return dpp_keymax<DPP_MIRROR>(k);
}
MM_DEV float row_max(float v) {
  v = fmaxf(v, dpp_f<DPP_XOR1>(v));
  v = fmaxf(v, dpp_f<DPP_XOR2>(v));
  v = fmaxf(v, dpp_f<DPP_HALF_MIRROR>(v));
  return fmaxf(v, dpp_f<DPP_MIRROR>(v));
}
MM_DEV float row_sum(float v) {
  v += dpp_f<DPP_XOR1>(v);
  v += dpp_f<DPP_XOR2>(v);
  v += dpp_f<DPP_HALF_MIRROR>(v);
  return v + dpp_f<DPP_MIRROR>(v);
}

// ld(j, e): logit e of row j (e < E).
template <int SL, class Ld>
MM_DEV void softmax_topk_rows16(Ld ld, int nvalid, int E, int k, int renorm, int64_t* ids,
                                float* probs) {
  const int lane = threadIdx.x & 63;
  const int j = lane >> 4, l = lane & 15;
  float p[SL];
  float mx = -INFINITY;
#pragma unroll
  for (int sl = 0; sl < SL; ++sl) {
    const int e = l + 16 * sl;
    p[sl] = e < E ? ld(j, e) : -INFINITY;
    mx = fmaxf(mx, p[sl]);
  }
  mx = row_max(mx);
  float sm = 0.0f;
#pragma unroll
  for (int sl = 0; sl < SL; ++sl)
    if (l + 16 * sl < E) {
      p[sl] = expf(p[sl] - mx);
      sm += p[sl];
    }
  sm = row_sum(sm);
#pragma unroll
  for (int sl = 0; sl < SL; ++sl)          // -1: below every probability, never taken
    p[sl] = l + 16 * sl < E ? p[sl] / sm : -1.0f;

  uint32_t used = 0;
  float taken = 0.0f;
  float my_p[RT_MAXK / 16];                 // round r is kept by lane r & 15, slot r >> 4
  int my_i[RT_MAXK / 16];
#pragma unroll
  for (int s = 0; s < RT_MAXK / 16; ++s) {
    my_p[s] = 0.0f;
    my_i[s] = 0;
  }
  for (int r = 0; r < k; ++r) {
    float bv = -2.0f;
    int bi = 0x7fffffff;
#pragma unroll
    for (int sl = 0; sl < SL; ++sl)
      if (!((used >> sl) & 1u) && p[sl] > bv) {   // slots ascend in e: ties keep the lower
        bv = p[sl];
        bi = l + 16 * sl;
      }
    const uint64_t key = row_keymax(argmax_key(bv, bi));
    bv = key_value(key);
    bi = key_index(key);
    if ((bi & 15) == l) used |= 1u << (bi >> 4);
#pragma unroll
    for (int s = 0; s < RT_MAXK / 16; ++s)
      if ((r >> 4) == s && (r & 15) == l) {
        my_p[s] = bv;
        my_i[s] = bi;
      }
    taken += bv;
  }
  if (j < nvalid) {
#pragma unroll
    for (int s = 0; s < RT_MAXK / 16; ++s) {
      const int r = 16 * s + l;
      if (r < k) {
        ids[j * k + r] = my_i[s];
        probs[j * k + r] = renorm ? my_p[s] / taken : my_p[s];
      }
    }
  }
}

// Slots per lane of the 16-lanes-per-row layout (E <= 256), or 0.
inline int rt16_slots(int E) {
  return E <= 16 ? 1 : E <= 32 ? 2 : E <= 64 ? 4 : E <= 128 ? 8 : E <= 256 ? 16 : 0;
}

// Slots per lane for E experts (E <= 1024), or 0 above that.
inline int rt_slots(int E) {
  return E <= 64 ? 1 : E <= 128 ? 2 : E <= 256 ? 4 : E <= 512 ? 8 : E <= 1024 ? 16 : 0;
}

// Router GEMM + softmax + top-k in one launch, spread over many CUs (one CU
// streams only a few tens of GB/s, so the gate weight must be read by many
// blocks).  grid = (blocks per token block, token blocks of 16).  A task is
// (expert tile of 16, slice of `spl` 32-k steps); block b's wave w runs task
// 4b + w, issuing RT_UNROLL A/W loads ahead of their MFMA 16x16x32s.  X
// [T, H] fp16, W [E, H] fp16 (nn.Linear weight), bias [E] fp32 or null.
// Slice partials go to the workspace with agent-scope stores; the last block
// of a token block to arrive sums them in slice order, adds the bias, rounds
// the logits to fp16 in LDS and runs softmax + top-k, one wave per token.
template <bool R16, int SL>
__global__ void __launch_bounds__(RT_NW * 64)
k_moe_router(const f16* __restrict__ X, const f16* __restrict__ W, const float* __restrict__ bias,
             int T, int H, int E, int k, int renorm, int spl, int nsl, float* __restrict__ part,
             uint32_t* __restrict__ counters, int64_t* __restrict__ ids, float* __restrict__ probs) {
  extern __shared__ float lg[];                 // [RT_TOK][E]
  __shared__ uint32_t s_last;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int c = lane & 15, q = lane >> 4;
  const int tb = blockIdx.y, t0 = tb * RT_TOK;
  const int ntile = (E + 15) / 16;
  const int nsteps = H / 32;
  float* pt = part + (size_t)tb * nsl * RT_TOK * E;           // [nsl][RT_TOK][E]
  const int task = blockIdx.x * RT_NW + wave;
  if (task < ntile * nsl) {
    const int tile = task % ntile, sl = task / ntile;
    const f16* xrow = X + (size_t)min(t0 + c, T - 1) * H + 8 * q;   // A operand row of this lane
    const f16* wrow = W + (size_t)min(tile * 16 + c, E - 1) * H + 8 * q;
    const int s1 = min(nsteps, (sl + 1) * spl);
    int st = sl * spl;
    f32x4 acc = {0, 0, 0, 0};
    for (; st + RT_UNROLL <= s1; st += RT_UNROLL) {
      f16x8 a[RT_UNROLL], b[RT_UNROLL];
#pragma unroll
      for (int u = 0; u < RT_UNROLL; ++u) {
        a[u] = *(const f16x8*)(xrow + 32 * (st + u));
        b[u] = *(const f16x8*)(wrow + 32 * (st + u));
      }
#pragma unroll
      for (int u = 0; u < RT_UNROLL; ++u)
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[u], b[u], acc, 0, 0, 0);
    }
    for (; st < s1; ++st)
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(*(const f16x8*)(xrow + 32 * st),
                                                   *(const f16x8*)(wrow + 32 * st), acc, 0, 0, 0);
    // acc[j]: token 4*q + j, expert tile*16 + c.
    const int ec = tile * 16 + c;
    if (ec < E) {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        __hip_atomic_store(pt + ((size_t)sl * RT_TOK + 4 * q + j) * E + ec, acc[j],
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  // The partials are agent-scope (write-through) stores: wait for their
  // acknowledgement before the arrival counter can publish them.
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t prev = __hip_atomic_fetch_add(&counters[tb], 1u, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT);
    s_last = (prev == gridDim.x - 1u) ? 1u : 0u;
  }
  __syncthreads();
  if (!s_last) return;
  // Every partial of RT_FIN items per thread is loaded before any is summed,
  // so the hand-off costs one memory round trip rather than one per slice.
  constexpr int NT = RT_NW * 64;
  const int n = RT_TOK * E;
  for (int i0 = threadIdx.x; i0 < n; i0 += RT_FIN * NT) {
    float v[RT_FIN][RT_MAXSL];
#pragma unroll
    for (int u = 0; u < RT_FIN; ++u)
#pragma unroll
      for (int sl = 0; sl < RT_MAXSL; ++sl) {
        const int i = i0 + u * NT;
        v[u][sl] = (i < n && sl < nsl)
                       ? __hip_atomic_load(pt + (size_t)sl * n + i, __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT)
                       : 0.0f;
      }
#pragma unroll
    for (int u = 0; u < RT_FIN; ++u) {
      const int i = i0 + u * NT;
      if (i >= n) break;
      float acc = v[u][0];
#pragma unroll
      for (int sl = 1; sl < RT_MAXSL; ++sl) acc += v[u][sl];   // zero past nsl: exact
      const float bb = bias != nullptr ? bias[i % E] : 0.0f;
      lg[i] = (float)(f16)(acc + bb);
    }
  }
  __syncthreads();
  constexpr int NR = RT_TOK / RT_NW;          // rows per wave
  static_assert(NR == 4, "four rows per wave (one per DPP row in the 16-lane layout)");
  const int r0 = wave * NR;
  if (t0 + r0 < T) {
    if constexpr (R16)
      softmax_topk_rows16<SL>([&](int j, int e) { return lg[(r0 + j) * E + e]; },
                              min(NR, T - t0 - r0), E, k, renorm, ids + (size_t)(t0 + r0) * k,
                              probs + (size_t)(t0 + r0) * k);
    else
      softmax_topk_rows<NR, SL>(lg + r0 * E, E, min(NR, T - t0 - r0), E, k, renorm,
                                ids + (size_t)(t0 + r0) * k, probs + (size_t)(t0 + r0) * k);
  }
  if (threadIdx.x == 0)
    __hip_atomic_store(&counters[tb], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Router plan: 32-k steps per slice and slice count (at most RT_MAXSL
// slices, each a multiple of RT_UNROLL steps), blocks per token block.
struct RouterPlan {
  int spl, nsl, nbx;
};
RouterPlan plan_router(int H, int E) {
  RouterPlan p;
  const int nsteps = H / 32;
  p.spl = mm_cdiv(mm_cdiv(nsteps, RT_MAXSL), RT_UNROLL) * RT_UNROLL;
  p.nsl = mm_cdiv(nsteps, p.spl);
  p.nbx = mm_cdiv(mm_cdiv(E, 16) * p.nsl, RT_NW);
  return p;
}

// Softmax + top-k of given logits [T, E] (fp16 or fp32).  SL > 0 (E <= 1024):
// RT_WAVES waves x NR tokens per block, NR rows per wave at once; SL == 0:
// one token per wave, probabilities recomputed per round.
template <int NR, int SL, bool R16>
__global__ void __launch_bounds__(RT_WAVES * 64)
k_softmax_topk(const void* __restrict__ logits, int logits_f32, int T, int E, int k, int renorm,
               int64_t* __restrict__ ids, float* __restrict__ probs) {
  extern __shared__ float lg[];                 // [RT_WAVES][NR][E]
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int t0 = (blockIdx.x * RT_WAVES + wave) * NR;
  if (t0 >= T) return;
  const int nv = min(NR, T - t0);
  if constexpr (R16) {
    // 16 lanes per row: each lane loads its own logits, no LDS staging.
    // Rows past T read the last row (their results are not stored).
    const size_t base = (size_t)t0 * E;
    const int jmax = nv - 1;
    if (logits_f32)
      softmax_topk_rows16<SL>(
          [&](int j, int e) { return ((const float*)logits)[base + (size_t)min(j, jmax) * E + e]; },
          nv, E, k, renorm, ids + (size_t)t0 * k, probs + (size_t)t0 * k);
    else
      softmax_topk_rows16<SL>(
          [&](int j, int e) {
            return (float)((const f16*)logits)[base + (size_t)min(j, jmax) * E + e];
          },
          nv, E, k, renorm, ids + (size_t)t0 * k, probs + (size_t)t0 * k);
    return;
  }
  float* rows = lg + (size_t)wave * NR * E;
  for (int j = 0; j < nv; ++j)
    for (int e = lane; e < E; e += 64)
      rows[j * E + e] = logits_f32 ? ((const float*)logits)[(size_t)(t0 + j) * E + e]
                                   : (float)((const f16*)logits)[(size_t)(t0 + j) * E + e];
  if constexpr (SL == 0) {
    softmax_topk_row(rows, E, k, renorm, ids + (size_t)t0 * k, probs + (size_t)t0 * k);
  } else {
    softmax_topk_rows<NR, SL>(rows, E, nv, E, k, renorm, ids + (size_t)t0 * k,
                              probs + (size_t)t0 * k);
  }
}

}  // namespace

// ===========================================================================
// C ABI
// ===========================================================================
extern "C" size_t mm_moe_router_workspace_bytes(int T, int H, int E) {
  if (T <= 0 || H <= 0 || E <= 0) return (size_t)RT_MAX_TB * sizeof(uint32_t);
  const RouterPlan p = plan_router(H, E);
  return (size_t)RT_MAX_TB * sizeof(uint32_t) +
         (size_t)mm_cdiv(T, RT_TOK) * p.nsl * RT_TOK * E * sizeof(float);
}

extern "C" int mm_moe_router(const uint16_t* X, const uint16_t* W, const float* bias, int T, int H,
                             int E, int k, int renorm, int64_t* ids, float* probs, void* ws,
                             size_t ws_bytes, void* stream) {
  MM_CHECK_ARG(T >= 0 && H > 0 && E > 0, "mm_moe_router: bad shape T=%d H=%d E=%d", T, H, E);
  MM_CHECK_ARG(H % 32 == 0, "mm_moe_router: hidden size %d must be divisible by 32", H);
  MM_CHECK_ARG(E <= 1024, "mm_moe_router: num_experts=%d must be <= 1024", E);
  MM_CHECK_ARG(k >= 1 && k <= RT_MAXK && k <= E, "mm_moe_router: top_k=%d must be in [1, %d]",
               k, E < RT_MAXK ? E : RT_MAXK);
  MM_CHECK_ARG(((uintptr_t)X & 15) == 0 && ((uintptr_t)W & 15) == 0,
               "mm_moe_router: hidden states and router weight must be 16-byte aligned");
  if (T == 0) return 0;
  MM_CHECK_ARG(mm_cdiv(T, RT_TOK) <= RT_MAX_TB, "mm_moe_router: T=%d exceeds %d tokens", T,
               RT_MAX_TB * RT_TOK);
  const size_t need = mm_moe_router_workspace_bytes(T, H, E);
  MM_CHECK_ARG(ws != nullptr && ws_bytes >= need,
               "mm_moe_router: workspace of %zu bytes is smaller than the %zu required", ws_bytes,
               need);
  const RouterPlan p = plan_router(H, E);
  const size_t lds = (size_t)RT_TOK * E * sizeof(float);
  float* part = (float*)((char*)ws + (size_t)RT_MAX_TB * sizeof(uint32_t));
#define MM_LAUNCH_RT(R16, SLV)                                                                 \
  hipLaunchKernelGGL((k_moe_router<R16, SLV>), dim3(p.nbx, mm_cdiv(T, RT_TOK)), dim3(RT_NW * 64), \
                     lds, (hipStream_t)stream, (const f16*)X, (const f16*)W, bias, T, H, E, k,     \
                     renorm, p.spl, p.nsl, part, (uint32_t*)ws, ids, probs)
  switch (rt16_slots(E)) {
    case 1: MM_LAUNCH_RT(true, 1); break;
    case 2: MM_LAUNCH_RT(true, 2); break;
    case 4: MM_LAUNCH_RT(true, 4); break;
    case 8: MM_LAUNCH_RT(true, 8); break;
    case 16: MM_LAUNCH_RT(true, 16); break;
    default:
      if (E <= 512) MM_LAUNCH_RT(false, 8);
      else MM_LAUNCH_RT(false, 16);
  }
#undef MM_LAUNCH_RT
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
  const int sl = rt_slots(E), sl16 = rt16_slots(E);
  const int nr = sl == 0 ? 1 : 4;               // tokens per wave
  // The 16-lanes-per-row layout (sl16 > 0) reads the logits into registers.
  const size_t lds = sl16 > 0 ? 0 : (size_t)RT_WAVES * nr * E * sizeof(float);
  const dim3 grid(mm_cdiv(T, RT_WAVES * nr));
#define MM_LAUNCH_ST(NRV, SLV, R16)                                                              \
  hipLaunchKernelGGL((k_softmax_topk<NRV, SLV, R16>), grid, dim3(RT_WAVES * 64), lds,             \
                     (hipStream_t)stream, logits, logits_f32, T, E, k, renorm, ids, probs)
  switch (sl16) {
    case 1: MM_LAUNCH_ST(4, 1, true); break;
    case 2: MM_LAUNCH_ST(4, 2, true); break;
    case 4: MM_LAUNCH_ST(4, 4, true); break;
    case 8: MM_LAUNCH_ST(4, 8, true); break;
    case 16: MM_LAUNCH_ST(4, 16, true); break;
    default:
      if (sl == 8) MM_LAUNCH_ST(4, 8, false);
      else if (sl == 16) MM_LAUNCH_ST(4, 16, false);
      else MM_LAUNCH_ST(1, 0, false);
  }
#undef MM_LAUNCH_ST
  MM_CHECK_LAUNCH("mm_softmax_topk");
  return 0;
}
