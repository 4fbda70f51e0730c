// MoE grouped-expert FP4 path for gfx950: device counting sort of the
// (token, slot) assignments, a grouped expert GEMM over the expert-sorted rows
// (optionally gathering token rows and applying SwiGLU in the epilogue), and
// a deterministic probability-weighted combine.
//
// Reference: metal_marlin/moe_dispatch.py:493-555 (group_tokens_by_expert),
// :789-809 (gather_for_experts), :812-925 (scatter/aggregate),
// :1241-1431 (_fused_expert_mlp); metal_marlin/kernels/moe.py:583-727
// (moe_expert_gemm_fp4); Metal src/moe_expert_gemm.metal:557-782.  The
// reference's grouped kernel accumulates out[token] += p*y with a
// non-atomic read-modify-write; here every output row is owned by exactly one
// writer and the combine sums the k slots in fixed order.
#include "mm_common.h"
#include "mm_skinny.h"
#include "mm_prefill.h"

namespace {
using namespace mmsk;
using namespace mmpf;

#define MM_MOE_DEC_NW 4      // waves per block of the grouped decode kernel (busy launches)
#define MM_MOE_DEC_SPW 4     // 32-k steps per wave per round there
// Grouped prefill kernel: a 2-stage LDS ring (loads one chunk ahead) and at
// most 168 VGPRs, so three 4-wave blocks fit per CU (3 waves per SIMD).
// Measured on MI355X at the Qwen3-30B-A3B shapes: the more resident waves hide
// latency better than the deeper ring did (3 stages, 204 VGPRs, 2 blocks per
// CU): gate_up at T=1024 111-113 -> 93-99 us, at T=512 78 -> 64 us, at T=4096
// 282 -> 264 us; down at T=512 40 -> 33 us.
constexpr int MOE_PF_STAGES = 2;
constexpr int MOE_PF_WAVES_PER_SIMD = 3;
#define MM_MOE_PF_ROWS 24   // average rows per expert above which the MFMA tile kernel runs

// Expert weights: experts e < Er are slices of the stacked [Er, K/8, N]
// words and [Er, K/g, N] scales; expert Er (when a shared expert is run as an
// extra group) has its own [K/8, N] / [K/g, N] tensors.
struct ExpertW {
  const uint32_t* B;
  const f16* S;
  const uint32_t* Bsh;
  const f16* Ssh;
  int Er;
  MM_DEV const uint32_t* b(int e, int K, int N) const {
    return e < Er ? B + (size_t)e * (K / 8) * N : Bsh;
  }
  MM_DEV const f16* s(int e, int K, int N, int g) const {
    return e < Er ? S + (size_t)e * (K / g) * N : Ssh;
  }
};

constexpr int SORT_THREADS = 1024;
constexpr int MOE_MAX_EXPERTS = SORT_THREADS;   // the sort holds one expert per thread
constexpr int SORT_WAVES = SORT_THREADS / 64;
constexpr int SORT_KC = 8;          // 64-key chunks fetched together per wave
// Inputs above MM_MOE_SORT_ONE_BLOCK assignments (when the caller has scratch
// for the per-block counts) sort in blocks of MM_MOE_SORT_SEG.  Measured on
// MI355X, whole Qwen3-30B-A3B MLP call, one block / two launches: T*k = 4096
// 121 / 126 us, 8192 171 / 178 us, 16384 292 / 288 us, 32768 474 / 460 us.
#define MM_MOE_SORT_ONE_BLOCK 8192
#define MM_MOE_SORT_SEG 1024
// The single-launch multi-block sort (k_moe_sort_mb) serves MB_MIN < n <= MB_MAX
// assignments with E <= MB_EXPERTS (its LDS holds (2 + 16) * E counters);
// n > 0 always (an empty input takes the one-block kernel).  Measured on
// MI355X, whole Qwen3-30B-A3B MLP call against the one-block sort: T = 8 / 32
// / 128 / 256 / 1024 / 2048 43.1 -> 41.2, 66.3 -> 64.5, 78.4 -> 75.3, 117.0
// -> 113.5, 155.4 -> 151.1, 269.3 -> 253.8 us (sort alone at T = 1024:
// 14-17 -> 7.3 us).
#define MM_MOE_SORT_MB_MIN 0
#define MM_MOE_SORT_MB_MAX 32768
#define MM_MOE_SORT_MB_EXPERTS 512

// Stable counting sort in one block.  Wave w owns the w-th contiguous
// segment of the flat assignments (whole 64-element chunks), so segment order
// is index order.  Within a chunk, the lanes holding the same expert are found
// with one ballot per key bit (log2(E) ballots, independent of how many
// distinct experts the chunk holds); the lowest such lane is the group's
// leader.  Pass 1 counts per (wave, expert); a scan turns the counts into
// expert offsets and each wave's first position per expert; pass 2 places
// every assignment at its wave's running position plus its rank among the
// equal lanes below it.  Dynamic LDS: wpos[SORT_WAVES][E] ints.
// Ids outside [0, E) (the reference requires them in range) are dropped:
// they are placed after every expert's rows, in index order, so sorted_idx
// and inverse stay permutations of the T*k assignments and offsets[E] counts
// the valid ones only; no grouped GEMM reads the dropped rows.
// SH: every token has one more slot (index kin of kin + 1) whose key is the
// shared-expert group E - 1; n = T * (kin + 1) then, and flat indices run
// over the kin + 1 slots.
// MODE 0: one block sorts all n.  Larger inputs use two launches over
// blocks of bseg assignments each (segment order is again index order):
// MODE 1 counts block b's segment per expert into cnt[b][E + 1] (entry E:
// its dropped ids); MODE 2 places block b's segment, starting each expert at
// its offset plus the counts of the blocks before b (block 0 writes
// offsets).
template <typename IdT, bool SH, int MODE = 0>
__global__ void __launch_bounds__(SORT_THREADS)
k_moe_sort(const IdT* __restrict__ ids, int n, int E, int kin, int32_t* __restrict__ offsets,
           int32_t* __restrict__ sorted_idx, int32_t* __restrict__ inverse,
           int32_t* __restrict__ cnt, int bseg) {
  extern __shared__ int wpos[];
  __shared__ int wsum[SORT_WAVES];
  __shared__ int winv[SORT_WAVES];    // dropped (out-of-range) ids per wave
  __shared__ int s_valid;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nbits = E > 1 ? 32 - __clz(E - 1) : 0;
  const int b0 = MODE ? blockIdx.x * bseg : 0, b1 = MODE ? min(n, b0 + bseg) : n;
  const int per = mm_cdiv(mm_cdiv(b1 - b0, 64), SORT_WAVES) * 64;
  const int seg0 = min(b1, b0 + wave * per), seg1 = min(b1, seg0 + per);
  const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
  int* mine = wpos + wave * E;

  for (int x = tid; x < SORT_WAVES * E; x += SORT_THREADS) wpos[x] = 0;
  int ninv = 0;                       // this wave's dropped ids (wave-uniform)
  __syncthreads();

  // Keys past the segment read a clamped index (the load is unconditional, so
  // the SORT_KC loads of a batch stay in flight together) and become -2; an
  // out-of-range id inside the segment becomes -1.
  auto key_at = [&](int i) {
    if constexpr (SH) {
      const int t = i / (kin + 1), j = i - t * (kin + 1);
      if (i >= seg1) return -2;
      if (j == kin) return E - 1;
      const long long v = (long long)ids[min(t * kin + j, n / (kin + 1) * kin - 1)];
      return (v >= 0 && v < E - 1) ? (int)v : -1;
    } else {
      const long long v = (long long)ids[min(i, n - 1)];
      return i >= seg1 ? -2 : ((v >= 0 && v < E) ? (int)v : -1);
    }
  };
  auto match = [&](int key) {
    const bool valid = key >= 0;
    uint64_t m = __ballot(valid);
    for (int bit = 0; bit < nbits; ++bit) {
      const bool on = valid && ((key >> bit) & 1);
      const uint64_t bb = __ballot(on);
      m &= on ? bb : ~bb;
    }
    return valid ? m : 0ull;
  };

  // Keys are fetched SORT_KC chunks at a time so their loads overlap.  When
  // the wave's segment is one such batch (n <= SORT_WAVES*64*SORT_KC), its
  // keys, in-group ranks and group sizes stay in registers for pass 2.
  const bool single = seg1 - seg0 <= 64 * SORT_KC;
  int skey[SORT_KC], srank[SORT_KC], sgrp[SORT_KC];
#pragma unroll
  for (int c = 0; c < SORT_KC; ++c) skey[c] = -2, srank[c] = 0, sgrp[c] = 0;   // empty segment
  for (int s0 = seg0; s0 < seg1; s0 += 64 * SORT_KC) {       // pass 1: counts
#pragma unroll
    for (int c = 0; c < SORT_KC; ++c) skey[c] = key_at(s0 + 64 * c + lane);
#pragma unroll
    for (int c = 0; c < SORT_KC; ++c) {
      const int e = skey[c];
      const uint64_t same = match(e);
      srank[c] = __popcll(same & below);
      sgrp[c] = (e >= 0 && srank[c] == 0) ? __popcll(same) : 0;   // set on the group's leader
      if (sgrp[c]) mine[e] += sgrp[c];
      ninv += __popcll(__ballot(e == -1));
    }
  }
  if (lane == 0) winv[wave] = ninv;
  __syncthreads();

  if constexpr (MODE == 1) {   // this block's counts per expert, then its dropped ids
    int32_t* const row = cnt + (size_t)blockIdx.x * (E + 1);
    if (tid < E) {
      int c = 0;
      for (int w = 0; w < SORT_WAVES; ++w) c += wpos[w * E + tid];
      row[tid] = c;
    }
    if (tid == SORT_THREADS - 1) {
      int d = 0;
      for (int w = 0; w < SORT_WAVES; ++w) d += winv[w];
      row[E] = d;
    }
    return;
  }
  // Expert totals -> exclusive offsets (wave scans, then a scan of the wave
  // sums), and each wave's first position per expert.  MODE 2: the totals
  // are over every block, and this block starts past the blocks before it.
  int tot = 0, pre = 0, dpre = 0;
  if constexpr (MODE == 2) {
    if (tid < E)
      for (int b = 0; b < (int)gridDim.x; ++b) {
        const int c = cnt[(size_t)b * (E + 1) + tid];
        tot += c;
        if (b < (int)blockIdx.x) pre += c;
      }
    for (int b = 0; b < (int)blockIdx.x; ++b) dpre += cnt[(size_t)b * (E + 1) + E];
  } else {
    if (tid < E)
      for (int w = 0; w < SORT_WAVES; ++w) tot += wpos[w * E + tid];
  }
  int incl = tot;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int o = __shfl_up(incl, d);
    if (lane >= d) incl += o;
  }
  if (lane == 63) wsum[wave] = incl;
  __syncthreads();
  int wbase = 0;
  for (int w = 0; w < wave; ++w) wbase += wsum[w];
  if (tid < E) {
    int run = wbase + incl - tot;
    if (MODE == 0 || blockIdx.x == 0) offsets[tid] = run;
    run += pre;
    for (int w = 0; w < SORT_WAVES; ++w) {
      const int c = wpos[w * E + tid];
      wpos[w * E + tid] = run;
      run += c;
    }
  }
  if (tid == SORT_THREADS - 1) {
    if (MODE == 0 || blockIdx.x == 0) offsets[E] = wbase + incl;
    s_valid = wbase + incl;
  }
  __syncthreads();
  // Dropped ids: this wave's first position after all valid assignments.
  int tail = s_valid + dpre;
  for (int w = 0; w < wave; ++w) tail += winv[w];
  auto place_dropped = [&](int e, int i) {
    const uint64_t m = __ballot(e == -1);
    if (e == -1) {
      const int pos = tail + __popcll(m & below);
      sorted_idx[pos] = i;
      inverse[i] = pos;
    }
    tail += __popcll(m);
  };

  // Pass 2: placement.  Every lane reads its group's running position before
  // the leader advances it past the group (LDS ops of a wave complete in
  // order).
  if (single) {
#pragma unroll
    for (int c = 0; c < SORT_KC; ++c) {
      const int e = skey[c];
      const int i = seg0 + 64 * c + lane;
      if (e >= 0) {
        const int pos = mine[e] + srank[c];
        sorted_idx[pos] = i;
        inverse[i] = pos;
      }
      if (sgrp[c]) mine[e] += sgrp[c];
      place_dropped(e, i);
    }
    return;
  }
  for (int s0 = seg0; s0 < seg1; s0 += 64 * SORT_KC) {
#pragma unroll
    for (int c = 0; c < SORT_KC; ++c) skey[c] = key_at(s0 + 64 * c + lane);
#pragma unroll
    for (int c = 0; c < SORT_KC; ++c) {
      const int i = s0 + 64 * c + lane;
      const int e = skey[c];
      const uint64_t same = match(e);
      if (e >= 0) {
        const int pos = mine[e] + __popcll(same & below);
        sorted_idx[pos] = i;
        inverse[i] = pos;
      }
      if (e >= 0 && (same & below) == 0) mine[e] += __popcll(same);
      place_dropped(e, i);
    }
  }
}

// Stable counting sort over several blocks in ONE launch, with no
// communication between blocks: block b owns the b-th SORT_THREADS-long
// segment of the flat assignments (one per thread) and first counts, in LDS
// with integer atomics, every expert's assignments over ALL n ids and over the
// ids before its segment (all blocks read all ids, from L2).  From those it
// knows each expert's offset and where its own segment's rows of that expert
// start, and places its segment with the in-wave ranks of the one-block sort
// (ballot matching) and per-wave counts.  The result is the one-block sort's
// (same order, same dropped-id handling); block 0 writes the offsets.  The
// per-block cost grows with n (every block counts all ids), so the host uses
// it for mid-sized inputs only.  Dynamic LDS: (2 + SORT_WAVES) * E ints.
template <typename IdT, bool SH>
__global__ void __launch_bounds__(SORT_THREADS)
k_moe_sort_mb(const IdT* __restrict__ ids, int n, int E, int kin, int32_t* __restrict__ offsets,
              int32_t* __restrict__ sorted_idx, int32_t* __restrict__ inverse) {
  extern __shared__ int sm[];
  int* const tot = sm;              // [E] assignments per expert, all ids
  int* const pre = sm + E;          // [E] the same over ids before this segment
  int* const wpos = sm + 2 * E;     // [SORT_WAVES][E] per-wave counts -> start positions
  __shared__ int wsum[SORT_WAVES];
  __shared__ int winv[SORT_WAVES];  // dropped ids per wave of this segment
  __shared__ int s_drop;            // dropped ids before this segment
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nbits = E > 1 ? 32 - __clz(E - 1) : 0;
  const int seg0 = blockIdx.x * SORT_THREADS;
  const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
  for (int x = tid; x < (2 + SORT_WAVES) * E; x += SORT_THREADS) sm[x] = 0;
  if (tid == 0) s_drop = 0;
  __syncthreads();

  // Key of flat assignment i: its expert, -1 for an id outside the range
  // (dropped), -2 past the end.
  auto key_at = [&](int i) {
    if constexpr (SH) {
      const int t = i / (kin + 1), j = i - t * (kin + 1);
      if (i >= n) return -2;
      if (j == kin) return E - 1;
      const long long v = (long long)ids[min(t * kin + j, n / (kin + 1) * kin - 1)];
      return (v >= 0 && v < E - 1) ? (int)v : -1;
    } else {
      const long long v = (long long)ids[min(i, n - 1)];
      return i >= n ? -2 : ((v >= 0 && v < E) ? (int)v : -1);
    }
  };

  // Pass A: histograms of all ids and of the ids before the segment.  The
  // keys of SORT_KC rounds are loaded together so their loads overlap.
  int dpre = 0;
  for (int i0 = 0; i0 < n; i0 += SORT_THREADS * SORT_KC) {
    int key[SORT_KC];
#pragma unroll
    for (int u = 0; u < SORT_KC; ++u) key[u] = key_at(i0 + u * SORT_THREADS + tid);
#pragma unroll
    for (int u = 0; u < SORT_KC; ++u) {
      const int i = i0 + u * SORT_THREADS + tid;
      const int e = key[u];
      if (e >= 0) {
        __hip_atomic_fetch_add(&tot[e], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        if (i < seg0)
          __hip_atomic_fetch_add(&pre[e], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      } else if (e == -1) {
        dpre += i < seg0;
      }
    }
  }
  // Own assignment: rank among the equal keys of lower lanes in the wave, and
  // the wave's count per expert (by the group's leader lane).
  const int i = seg0 + tid;
  const int e = key_at(i);
  uint64_t same = 0;
  {
    const bool valid = e >= 0;
    uint64_t m = __ballot(valid);
    for (int bit = 0; bit < nbits; ++bit) {
      const bool on = valid && ((e >> bit) & 1);
      const uint64_t bb = __ballot(on);
      m &= on ? bb : ~bb;
    }
    same = valid ? m : 0ull;
  }
  const int rank = __popcll(same & below);
  if (e >= 0 && rank == 0) wpos[wave * E + e] = __popcll(same);
  const uint64_t dm = __ballot(e == -1);
  if (lane == 0) winv[wave] = __popcll(dm);
  // dropped ids before the segment: one LDS add per wave
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) dpre += __shfl_xor(dpre, d);
  if (lane == 0)
    __hip_atomic_fetch_add(&s_drop, dpre, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  __syncthreads();

  // Exclusive offsets over experts (wave scans, then the wave sums), then each
  // wave's first position per expert: offset + ids of the expert before the
  // segment + those of the earlier waves of the segment.
  const int c = tid < E ? tot[tid] : 0;
  int incl = c;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int o = __shfl_up(incl, d);
    if (lane >= d) incl += o;
  }
  if (lane == 63) wsum[wave] = incl;
  __syncthreads();
  int wbase = 0;
  for (int w = 0; w < wave; ++w) wbase += wsum[w];
  int nvalid = 0;
  for (int w = 0; w < SORT_WAVES; ++w) nvalid += wsum[w];
  if (tid < E) {
    const int off = wbase + incl - c;
    if (blockIdx.x == 0) offsets[tid] = off;
    int run = off + pre[tid];
    for (int w = 0; w < SORT_WAVES; ++w) {
      const int cw = wpos[w * E + tid];
      wpos[w * E + tid] = run;
      run += cw;
    }
  }
  if (blockIdx.x == 0 && tid == 0) offsets[E] = nvalid;
  __syncthreads();
  if (e >= 0) {
    const int pos = wpos[wave * E + e] + rank;
    sorted_idx[pos] = i;
    inverse[i] = pos;
  } else if (e == -1) {
    int tail = nvalid + s_drop;
    for (int w = 0; w < wave; ++w) tail += winv[w];
    const int pos = tail + __popcll(dm & below);
    sorted_idx[pos] = i;
    inverse[i] = pos;
  }
}

// Grouped expert GEMM.  grid = (column tiles, 1, E); block = NW waves which
// split K; the block walks its expert's rows in chunks of MT*16.
//   act == 0: NT=2 tiles of 64 columns at n0 and n0+64.
//   act == 1: tile 0 = gate columns [n0, n0+64), tile 1 = up columns
//             [N/2 + n0, ...); output silu(gate) * up, width N/2.
// NW waves split K, each taking SPW 32-k steps per round; the host picks
// (NW, SPW) per launch from the expert's K so that few rounds remain and no
// wave idles.
template <int MT, int NW, int SPW, int FL>
__global__ void __launch_bounds__(NW * 64)
k_moe_grouped(const f16* __restrict__ X, const int32_t* __restrict__ sorted_idx,
              const int32_t* __restrict__ offsets, int gather, int topk, ExpertW W, int K,
              int N, int g, int act, f16* __restrict__ Y) {
  constexpr int NT = 2;
  constexpr int MOE_NW = NW, MOE_SPW = SPW;
  __shared__ __attribute__((aligned(16))) float red[row_items_lds_floats<MT, NT, MOE_NW>()];
  const int e = blockIdx.z;
  const int r0 = offsets[e], r1 = offsets[e + 1];
  if (r1 <= r0) return;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int c = lane & 15, q = lane >> 4;
  const uint32_t* B = W.b(e, K, N);
  const f16* S = W.s(e, K, N, g);
  const int nout = act ? N / 2 : N;
  const int n0 = act ? blockIdx.x * SK_COLS : blockIdx.x * NT * SK_COLS;
  const int coloff = act ? N / 2 : SK_COLS;
  const int nsteps = (K / 8 + 3) / 4;
  const int nrounds = (nsteps + MOE_NW * MOE_SPW - 1) / (MOE_NW * MOE_SPW);

  for (int mb = r0; mb < r1; mb += MT * 16) {
    const int mrows = min(MT * 16, r1 - mb);
    f32x4 acc[MT][NT][4];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[mt][t][j] = f32x4{0, 0, 0, 0};
    const f16* A = gather ? X : X + (size_t)mb * K;
    const SkTile tl[NT] = {SkTile{B, S, nullptr, n0}, SkTile{B, S, nullptr, n0 + coloff}};
    skinny_wave<false, MT, NT, MOE_SPW, FL>(A, K, gather ? sorted_idx + mb : nullptr, topk, mrows,
                                            tl, N, K, g, wave * MOE_SPW, nrounds,
                                            MOE_NW * MOE_SPW, acc);
    // Row items (mt, rr): lane (c, q) of the owning wave holds row
    // 16*mt + 4*q + rr, columns 4*c .. 4*c + 3 of both tiles.
    constexpr int IPW = row_items_per_wave<MT, MOE_NW>();
    f32x4 rv[IPW][NT];
    block_reduce_items<MT, NT, MOE_NW>(red, acc, mrows, rv);
#pragma unroll
    for (int k = 0; k < IPW; ++k) {
      const int it = wave + k * MOE_NW;
      const int row = it < MT * 4 ? 16 * (it >> 2) + 4 * q + (it & 3) : mrows;
      if (row >= mrows) continue;
      f16* yrow = Y + (size_t)(mb + row) * nout;
      if (act) {
        const int col = n0 + 4 * c;
        if (col < nout) {
          f16x4 o;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const float gt = rv[k][0][j], up = rv[k][1][j];
            o[j] = (f16)(gt / (1.0f + __expf(-gt)) * up);
          }
          *(f16x4*)(yrow + col) = o;
        }
      } else {
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          const int col = n0 + t * SK_COLS + 4 * c;
          if (col < nout)
            *(f16x4*)(yrow + col) =
                f16x4{(f16)rv[k][t][0], (f16)rv[k][t][1], (f16)rv[k][t][2], (f16)rv[k][t][3]};
        }
      }
    }
    __syncthreads();   // every wave has read `red` before the next chunk overwrites it
  }
}

// ---------------------------------------------------------------------------
// Grouped expert GEMM, prefill-sized groups: the pipelined MFMA main loop of
// the dense prefill kernel (mm_prefill.h) over one (expert, row tile,
// column tile) per block.  grid.y enumerates row tiles of BM rows over all
// experts in expert order; each block finds its expert with one wave scan of
// the offsets (grid.y is an upper bound; surplus blocks exit).  A rows are
// gathered through sorted_idx (gather=1) or read in sorted order.  Column
// map (tile-major, CW=2): each wave's 64 LDS columns are 32 output columns
// twice -- act=1: the gate columns then the matching up columns (N/2 on),
// so silu(gate)*up is formed in registers; act=0: 64 consecutive columns.
// Row blocks of a wave that lie past the expert's rows skip their MFMAs.
// ---------------------------------------------------------------------------
struct MoeSrc {
  const f16* X;
  const int32_t* sidx;
  int gather, topk, K;
  int mb, rlast;           // first sorted row of the tile, last row of the expert
  int act, half, o0;       // act=1: half = N/2, o0 = first output column
  const uint32_t* B;
  const f16* S;
  const f16* Z;
  int ld;
  MM_DEV const f16* arow(int r) const {
    const int sr = min(mb + r, rlast);
    return X + (size_t)(gather ? sidx[sr] / topk : sr) * K;
  }
  MM_DEV int col(int P, int w) const {
    if (!act) return min(o0 + P, ld - w);
    const int oc = pair_out_col(o0, P, w, half);
    return pair_is_up(P) ? half + oc : oc;
  }
  MM_DEV const uint32_t* bcol(int P, int w) const { return B + col(P, w); }
  MM_DEV const f16* scol(int P, int w) const { return S + col(P, w); }
  MM_DEV const f16* zcol(int P, int w) const { return Z + col(P, w); }
};

template <int WM, int WN, int RB, bool G64, int STAGES>
__global__ void __launch_bounds__(WM * WN * 64, MOE_PF_WAVES_PER_SIMD)
k_moe_prefill(const f16* __restrict__ X, const int32_t* __restrict__ sorted_idx,
              const int32_t* __restrict__ offsets, int gather, int topk, ExpertW W, int E,
              int K, int N, int g, int act, int gx, f16* __restrict__ Y) {
  constexpr int CW = 2;
  constexpr int SROWS = G64 ? PF2_SROWS_G64 : PF2_SROWS;
  using Sh = Pf2Shape<false, WM, WN, RB, CW, STAGES, SROWS>;
  constexpr int BM = Sh::BM, BN = Sh::BN;
  // One LDS object only: with a second __shared__ array in the kernel the
  // compiler cannot tell the operand reads from the in-flight global -> LDS
  // copies and waits for all of them (vmcnt(0)) in every chunk, which
  // serialises the load pipeline.  The row-tile prefix lives past the ring.
  __shared__ __attribute__((aligned(16))) char smem[Sh::LDS_BYTES + (MOE_MAX_EXPERTS + 1) * 4];
  int* const tp = (int*)(smem + Sh::LDS_BYTES);   // row-tile prefix over experts
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int l32 = lane & 31, h = lane >> 5;

  // tp[e] = row tiles of experts < e (one wave scan).
  if (wave == 0) {
    int base = 0;
    for (int e0 = 0; e0 < E; e0 += 64) {
      const int e = e0 + lane;
      const int t = e < E ? (offsets[e + 1] - offsets[e] + BM - 1) / BM : 0;
      int incl = t;
#pragma unroll
      for (int d = 1; d < 64; d <<= 1) {
        const int o = __shfl_up(incl, d);
        if (lane >= d) incl += o;
      }
      if (e < E) tp[e + 1] = base + incl;
      base += __shfl(incl, 63);
    }
    if (lane == 0) tp[0] = 0;
  }
  __syncthreads();
  // The grid is an upper bound on gx * (row tiles); blocks past the real
  // count exit.  Blocks are dealt round-robin to the 8 XCDs, so the linear id
  // is remapped to give each XCD one contiguous run of (row tile, column
  // tile) pairs: the column tiles of one row tile then share their A rows in
  // that XCD's L2.
  const int nreal = gx * tp[E];
  const int L = blockIdx.x;
  if (L >= nreal) return;
  const int xcd = L & 7, q = nreal >> 3, rem = nreal & 7;
  const int lin = xcd * q + min(xcd, rem) + (L >> 3);
  const int y = lin / gx, bx = lin - y * gx;
  int lo = 0, hi = E - 1;            // expert e with tp[e] <= y < tp[e + 1]
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (tp[mid] <= y) lo = mid; else hi = mid - 1;
  }
  const int e = lo;
  const int r0 = offsets[e], r1 = offsets[e + 1];
  const int mb = r0 + (y - tp[e]) * BM;
  const int rows = min(BM, r1 - mb);
  const int half = N / 2;
  const int o0 = act ? bx * (BN / 2) : bx * BN;
  const MoeSrc src{X, sorted_idx, gather, topk, K, mb, r1 - 1, act, half, o0,
                   W.b(e, K, N), W.s(e, K, N, g), nullptr, N};
  const int rb_live =
      __builtin_amdgcn_readfirstlane(min(RB, max(0, (rows - wm * 32 * RB + 31) / 32)));
  f32x16 acc[RB][CW];
  // The live row-block count is wave-uniform and fixed for the tile: one
  // switch here keeps the main loop free of per-step branches.
  static_for(
      [&](auto lc) {
        constexpr int L = decltype(lc)::value;
        if (rb_live == L)
          pf2_mainloop<false, WM, WN, RB, CW, G64, true, STAGES, SROWS, L>(src, K, g, 0,
                                                                           K / PF2_BK, smem, acc);
      },
      std::make_integer_sequence<int, RB + 1>{});

#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int r = wm * 32 * RB + rb * 32 + 8 * (v >> 2) + 4 * h + (v & 3);
      if (r >= rows) continue;
      if (act) {
        const int oc = o0 + wn * 32 + l32;
        if (oc < half) {
          const float gt = acc[rb][0][v], up = acc[rb][1][v];
          Y[(size_t)(mb + r) * half + oc] = (f16)(gt / (1.0f + __expf(-gt)) * up);
        }
      } else {
#pragma unroll
        for (int j = 0; j < CW; ++j) {
          const int c = o0 + wn * 64 + 32 * j + l32;
          if (c < N) Y[(size_t)(mb + r) * N + c] = (f16)acc[rb][j][v];
        }
      }
    }
  }
}

// out[t, :] = base[t, :] + sum_j p_j * Y[inverse[t*k + j], :] with p_j =
// probs[t, j] for the kin routed slots and p_kin = wsh for the shared slot
// (k = kin + 1 when a shared expert ran as an extra group, else k = kin);
// base may be null.  Summed in fp32 in slot order; one block per token, 8
// columns per thread.  nvalid (may be null): the sort's count of valid
// assignments; slots placed at or past it (dropped ids) contribute nothing.
__global__ void __launch_bounds__(256)
k_moe_combine(const f16* __restrict__ Y, const float* __restrict__ probs,
              const int32_t* __restrict__ inverse, int k, int kin, float wsh,
              const f16* __restrict__ base, const int32_t* __restrict__ nvalid, int H,
              f16* __restrict__ out) {
  const int t = blockIdx.x;
  const int lim = nvalid ? *nvalid : 0x7fffffff;
  for (int h8 = threadIdx.x; h8 < H / 8; h8 += 256) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    if (base) {
      const f16x8 b = *(const f16x8*)(base + (size_t)t * H + 8 * h8);
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i] = (float)b[i];
    }
    for (int j = 0; j < k; ++j) {
      const float p = j < kin ? probs[(size_t)t * kin + j] : wsh;
      const int r = inverse[(size_t)t * k + j];
      if (r >= lim) continue;
      const f16x8 y = *(const f16x8*)(Y + (size_t)r * H + 8 * h8);
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i] += p * (float)y[i];
    }
    f16x8 o;
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = (f16)acc[i];
    *(f16x8*)(out + (size_t)t * H + 8 * h8) = o;
  }
}

// shared: append the shared-expert slot (group E - 1) to every token; the
// ids are then [T, k] routed ids for the E - 1 routed experts.
template <typename IdT>
int moe_sort(const char* who, const IdT* expert_ids, int T, int k, int E, int32_t* offsets,
             int32_t* sorted_idx, int32_t* inverse, void* stream, bool shared = false,
             int32_t* cnt = nullptr) {
  MM_CHECK_ARG(T >= 0 && (k > 0 || (shared && k == 0)), "%s: bad T=%d k=%d", who, T, k);
  MM_CHECK_ARG(E > 0 && E <= SORT_THREADS, "%s: num_experts=%d must be in [1, %d]", who, E,
               SORT_THREADS);
  const int kt = k + (shared ? 1 : 0);
  MM_CHECK_ARG((long)T * kt < (1L << 30), "%s: T*k too large", who);
  const size_t lds = (size_t)SORT_WAVES * E * sizeof(int);
  const int n = T * kt;
  hipStream_t st = (hipStream_t)stream;
  if (n > MM_MOE_SORT_MB_MIN && n <= MM_MOE_SORT_MB_MAX && E <= MM_MOE_SORT_MB_EXPERTS) {
    // Mid-sized inputs: several blocks in one launch, each counting every id.
    const int nb = mm_cdiv(n, SORT_THREADS);
    const size_t lds_mb = (size_t)(2 + SORT_WAVES) * E * sizeof(int);
    if (shared)
      hipLaunchKernelGGL((k_moe_sort_mb<IdT, true>), dim3(nb), dim3(SORT_THREADS), lds_mb, st,
                         expert_ids, n, E, k, offsets, sorted_idx, inverse);
    else
      hipLaunchKernelGGL((k_moe_sort_mb<IdT, false>), dim3(nb), dim3(SORT_THREADS), lds_mb, st,
                         expert_ids, n, E, k, offsets, sorted_idx, inverse);
  } else if (cnt != nullptr && n > MM_MOE_SORT_ONE_BLOCK) {
    // Blocks of MM_MOE_SORT_SEG assignments: a count launch, then a place
    // launch (cnt: nb * (E + 1) ints of caller scratch).
    const int nb = mm_cdiv(n, MM_MOE_SORT_SEG);
#define MM_LAUNCH_SORT2(SHV)                                                                  \
  hipLaunchKernelGGL((k_moe_sort<IdT, SHV, 1>), dim3(nb), dim3(SORT_THREADS), lds, st,          \
                     expert_ids, n, E, k, offsets, sorted_idx, inverse, cnt, MM_MOE_SORT_SEG); \
  hipLaunchKernelGGL((k_moe_sort<IdT, SHV, 2>), dim3(nb), dim3(SORT_THREADS), lds, st,          \
                     expert_ids, n, E, k, offsets, sorted_idx, inverse, cnt, MM_MOE_SORT_SEG)
    if (shared) {
      MM_LAUNCH_SORT2(true);
    } else {
      MM_LAUNCH_SORT2(false);
    }
#undef MM_LAUNCH_SORT2
  } else if (shared) {
    hipLaunchKernelGGL((k_moe_sort<IdT, true>), dim3(1), dim3(SORT_THREADS), lds, st, expert_ids,
                       n, E, k, offsets, sorted_idx, inverse, nullptr, 0);
  } else {
    hipLaunchKernelGGL((k_moe_sort<IdT, false>), dim3(1), dim3(SORT_THREADS), lds, st, expert_ids,
                       n, E, k, offsets, sorted_idx, inverse, nullptr, 0);
  }
  MM_CHECK_LAUNCH(who);
  return 0;
}

// Grouped expert GEMM over E groups (W: their weights) of k*T sorted rows.
int grouped_gemm(const uint16_t* X, const int32_t* sorted_idx, const int32_t* offsets,
                 int gather, int k, int T, ExpertW W, int E, int K, int N, int g, int act,
                 uint16_t* Y, void* stream) {
  MM_CHECK_ARG(E > 0 && K > 0 && N > 0 && T >= 0 && k > 0, "mm_moe_grouped_gemm: bad shape");
  MM_CHECK_ARG(K % 8 == 0, "mm_moe_grouped_gemm: K=%d must be divisible by 8", K);
  MM_CHECK_ARG(g > 0 && g % 8 == 0 && K % g == 0,
               "mm_moe_grouped_gemm: group_size=%d must be a multiple of 8 dividing K=%d", g, K);
  MM_CHECK_ARG(act == 0 || act == 1, "mm_moe_grouped_gemm: act=%d must be 0 or 1", act);
  MM_CHECK_ARG(act ? (N % 8 == 0) : (N % 4 == 0),
               "mm_moe_grouped_gemm: N=%d must be divisible by %d", N, act ? 8 : 4);
  if (T == 0) return 0;
  MM_CHECK_ARG((size_t)(K / 8) * (size_t)N * 4 < ((size_t)1 << 32),
               "mm_moe_grouped_gemm: one expert's packed weights must be under 4 GiB");
  const int nout = act ? N / 2 : N;
  // Prefill-sized groups (more than MM_MOE_PF_ROWS rows per expert on
  // average) run the MFMA tile kernel when the shapes allow its 16-byte
  // pieces: K % 64 == 0, N % 8 == 0 (N % 16 == 0 with SwiGLU).
  if ((long)T * k > (long)MM_MOE_PF_ROWS * E && K % PF2_BK == 0 && N % (act ? 16 : 8) == 0 &&
      E <= MOE_MAX_EXPERTS) {
    const long tk = (long)T * k;
    // Row tile: 64 rows while groups average under 48 rows, else 96 (measured
    // on MI355X at the Qwen3-30B-A3B shapes, T = 256..4096: 96-row tiles beat
    // 128 and 256 once per-expert counts vary by tens of rows).
    const int cfg = tk < 48L * E ? 1 : 3;
#define MM_LAUNCH_MOE_PF(WM, WN, RB, ST)                                                         \
  do {                                                                                         \
    constexpr int BM = WM * 32 * RB, BN = WN * 64;                                             \
    const int gx = act ? mm_cdiv(nout, BN / 2) : mm_cdiv(N, BN);                               \
    const long blocks = (long)gx * ((tk + BM - 1) / BM + std::min<long>(E, tk));               \
    MM_CHECK_ARG(blocks < (1L << 30), "mm_moe_grouped_gemm: T*k=%ld too large", tk);           \
    if (g % PF2_BK == 0)                                                                       \
      hipLaunchKernelGGL((k_moe_prefill<WM, WN, RB, true, ST>), dim3((unsigned)blocks), \
                         dim3(WM * WN * 64), 0, (hipStream_t)stream, (const f16*)X, sorted_idx, \
                         offsets, gather, k, W, E, K, N, g, act, gx, (f16*)Y);  \
    else                                                                                       \
      hipLaunchKernelGGL((k_moe_prefill<WM, WN, RB, false, ST>), dim3((unsigned)blocks),\
                         dim3(WM * WN * 64), 0, (hipStream_t)stream, (const f16*)X, sorted_idx, \
                         offsets, gather, k, W, E, K, N, g, act, gx, (f16*)Y);  \
  } while (0)
    if (cfg == 1)
      MM_LAUNCH_MOE_PF(1, 4, 2, MOE_PF_STAGES);    // 64 x 256, 4 waves
    else
      MM_LAUNCH_MOE_PF(1, 4, 3, MOE_PF_STAGES);    // 96 x 256, 4 waves
#undef MM_LAUNCH_MOE_PF
    MM_CHECK_LAUNCH("mm_moe_grouped_gemm(prefill)");
    return 0;
  }
  // The decode kernel addresses gathered activation rows with 31-bit byte
  // offsets (a buffer resource whose out-of-range loads return zero).
  MM_CHECK_ARG(!gather || (size_t)T * (size_t)K * 2 < ((size_t)1 << 31),
               "mm_moe_grouped_gemm: gathered activations must be under 2 GiB");
  const int tiles = act ? mm_cdiv(nout, SK_COLS) : mm_cdiv(N, 2 * SK_COLS);
  dim3 grid(tiles, 1, E);
  // Blocks the launch can keep busy: column tiles x experts that can hold a
  // row.  Few blocks (a handful of tokens): 8 waves x 8 steps per block so
  // each block pulls more bytes; otherwise 4 waves x 4 steps, which keeps
  // more blocks resident per CU (measured best from 8 to 8192 rows).
  const long busy = (long)tiles * (long)std::min<long>(E, (long)T * k);
  const int cfg = busy < 512 ? 0 : 1;
#define MM_LAUNCH_MOE(MTV, NWV, SPWV, FLV)                                                     \
  hipLaunchKernelGGL((k_moe_grouped<MTV, NWV, SPWV, FLV>), grid, dim3(NWV * 64), 0,               \
                     (hipStream_t)stream, (const f16*)X, sorted_idx, offsets, gather, k, W, K, N, g, \
                     act, (f16*)Y)
#define MM_LAUNCH_MOE_FL(MTV, NWV, SPWV)                                                       \
  switch (flush_steps(g, SPWV)) {                                                              \
    case 1: MM_LAUNCH_MOE(MTV, NWV, SPWV, 1); break;                                           \
    case 2: MM_LAUNCH_MOE(MTV, NWV, SPWV, 2); break;                                           \
    case 4: MM_LAUNCH_MOE(MTV, NWV, SPWV, 4); break;                                           \
    case 8: MM_LAUNCH_MOE(MTV, NWV, SPWV, (SPWV % 8 == 0 ? 8 : 0)); break;                     \
    default: MM_LAUNCH_MOE(MTV, NWV, SPWV, 0); break;                                          \
  }
  if (cfg == 0) {
    MM_LAUNCH_MOE_FL(1, 8, 8);
  } else {
    MM_LAUNCH_MOE_FL(1, MM_MOE_DEC_NW, MM_MOE_DEC_SPW);
  }
#undef MM_LAUNCH_MOE_FL
#undef MM_LAUNCH_MOE
  MM_CHECK_LAUNCH("mm_moe_grouped_gemm");
  return 0;
}


int combine(const uint16_t* Y, const float* probs, const int32_t* inverse, int T, int k, int kin,
            float wsh, const uint16_t* base, const int32_t* nvalid, int H, uint16_t* out,
            void* stream) {
  MM_CHECK_ARG(T >= 0 && k > 0 && H > 0, "mm_moe_combine: bad shape");
  MM_CHECK_ARG(H % 8 == 0, "mm_moe_combine: H=%d must be divisible by 8", H);
  if (T == 0) return 0;
  hipLaunchKernelGGL(k_moe_combine, dim3(T), dim3(256), 0, (hipStream_t)stream, (const f16*)Y,
                     probs, inverse, k, kin, wsh, (const f16*)base, nvalid, H, (f16*)out);
  MM_CHECK_LAUNCH("mm_moe_combine");
  return 0;
}

// Routed-expert SwiGLU MLP: stable sort -> gate_up (token gather + SwiGLU
// epilogue) -> down -> probability-weighted combine, four launches on one
// stream with no host synchronisation.  (Deriving each expert's rows from the
// ids inside the GEMM blocks instead of sorting was measured and rejected: no
// faster at T=32 and 20% slower at T=128, since every block then scans all
// T*k ids before its first load.)
// With a shared expert (Bsgu != null) it is one more group, E, that every
// token visits with weight wsh: its rows share the two grouped launches with
// the routed experts' rows, and the combine adds it as slot k.  k may then be
// 0 (the shared expert alone).  base (may be null) is added in the combine.
template <typename IdT>
int moe_mlp(const char* who, const uint16_t* X, const IdT* ids, const float* probs, int T, int k,
            int E, int H, int I, const uint32_t* Bgu, const uint16_t* Sgu, const uint32_t* Bdn,
            const uint16_t* Sdn, const uint32_t* Bsgu, const uint16_t* Ssgu, const uint32_t* Bsdn,
            const uint16_t* Ssdn, float wsh, const uint16_t* base, int g, uint16_t* act_buf,
            uint16_t* y_buf, int32_t* sort_buf, uint16_t* out, void* stream) {
  const bool sh = Bsgu != nullptr;
  MM_CHECK_ARG(T >= 0 && (k > 0 || (sh && k == 0)) && E >= 0 && H > 0 && I > 0 &&
                   (E > 0 || sh),
               "%s: bad shape", who);
  MM_CHECK_ARG(!sh || (Ssgu != nullptr && Bsdn != nullptr && Ssdn != nullptr),
               "%s: the shared expert needs all four of its tensors", who);
  if (T == 0) return 0;
  MM_CHECK_ARG(act_buf != nullptr && y_buf != nullptr && sort_buf != nullptr && out != nullptr,
               "%s: scratch and output buffers are required", who);
  const int G = E + (sh ? 1 : 0), kt = k + (sh ? 1 : 0);
  const long tk = (long)T * kt;
  int32_t* offsets = sort_buf;
  int32_t* sorted_idx = sort_buf + G + 1;
  int32_t* inverse = sorted_idx + tk;
  // y_buf is free until the down launch: it holds the sort's per-block counts.
  int rc = moe_sort(who, ids, T, k, G, offsets, sorted_idx, inverse, stream, sh,
                    (int32_t*)y_buf);
  if (rc) return rc;
  const ExpertW wgu{Bgu, (const f16*)Sgu, Bsgu, (const f16*)Ssgu, E};
  const ExpertW wdn{Bdn, (const f16*)Sdn, Bsdn, (const f16*)Ssdn, E};
  rc = grouped_gemm(X, sorted_idx, offsets, 1, kt, T, wgu, G, H, 2 * I, g, 1, act_buf, stream);
  if (rc) return rc;
  rc = grouped_gemm(act_buf, sorted_idx, offsets, 0, kt, T, wdn, G, I, H, g, 0, y_buf, stream);
  if (rc) return rc;
  return combine(y_buf, probs, inverse, T, kt, k, wsh, base, offsets + G, H, out, stream);
}

// Shared + routed aggregation of one FP4 projection (no MLP): every token
// runs the shared matrix with weight 1 and its k routed matrices with their
// probabilities, all as groups of one grouped launch (act = 0), then the
// combine.  y_buf [T*(k+1), N] fp16, sort_buf [E + 2 + 2*T*(k+1)] int32.
template <typename IdT>
int moe_gemm_shared(const char* who, const uint16_t* X, const IdT* ids, const float* probs,
                    int T, int k, int E, int K, int N, const uint32_t* Bsh, const uint16_t* Ssh,
                    const uint32_t* B, const uint16_t* S, int g, uint16_t* y_buf,
                    int32_t* sort_buf, uint16_t* out, void* stream) {
  MM_CHECK_ARG(T >= 0 && k >= 0 && E >= 0 && K > 0 && N > 0 && (E > 0 || k == 0),
               "%s: bad shape", who);
  MM_CHECK_ARG(Bsh != nullptr && Ssh != nullptr, "%s: the shared matrix is required", who);
  MM_CHECK_ARG(N % 8 == 0, "%s: N=%d must be divisible by 8", who, N);
  if (T == 0) return 0;
  MM_CHECK_ARG(y_buf != nullptr && sort_buf != nullptr && out != nullptr,
               "%s: scratch and output buffers are required", who);
  const int G = E + 1, kt = k + 1;
  const long tk = (long)T * kt;
  int32_t* offsets = sort_buf;
  int32_t* sorted_idx = sort_buf + G + 1;
  int32_t* inverse = sorted_idx + tk;
  // y_buf is free until the grouped launch: it holds the sort's per-block counts.
  int rc = moe_sort(who, ids, T, k, G, offsets, sorted_idx, inverse, stream, true,
                    (int32_t*)y_buf);
  if (rc) return rc;
  const ExpertW w{B, (const f16*)S, Bsh, (const f16*)Ssh, E};
  rc = grouped_gemm(X, sorted_idx, offsets, 1, kt, T, w, G, K, N, g, 0, y_buf, stream);
  if (rc) return rc;
  return combine(y_buf, probs, inverse, T, kt, k, 1.0f, nullptr, offsets + G, N, out, stream);
}

}  // namespace

// ===========================================================================
// C ABI
// ===========================================================================
extern "C" int mm_moe_sort(const int32_t* expert_ids, int T, int k, int E, int32_t* offsets,
                           int32_t* sorted_idx, int32_t* inverse, void* stream) {
  return moe_sort("mm_moe_sort", expert_ids, T, k, E, offsets, sorted_idx, inverse, stream);
}

extern "C" int mm_moe_sort_i64(const int64_t* expert_ids, int T, int k, int E, int32_t* offsets,
                               int32_t* sorted_idx, int32_t* inverse, void* stream) {
  return moe_sort("mm_moe_sort_i64", expert_ids, T, k, E, offsets, sorted_idx, inverse, stream);
}

extern "C" int mm_moe_grouped_gemm(const uint16_t* X, const int32_t* sorted_idx,
                                   const int32_t* offsets, int gather, int k, int T,
                                   const uint32_t* B, const uint16_t* S, int E, int K, int N,
                                   int g, int act, uint16_t* Y, void* stream) {
  return grouped_gemm(X, sorted_idx, offsets, gather, k, T,
                      ExpertW{B, (const f16*)S, nullptr, nullptr, E}, E, K, N, g, act, Y, stream);
}

extern "C" int mm_moe_combine(const uint16_t* Y, const float* probs, const int32_t* inverse,
                              int T, int k, int H, uint16_t* out, void* stream) {
  return combine(Y, probs, inverse, T, k, k, 0.0f, nullptr, nullptr, H, out, stream);
}

extern "C" int mm_moe_mlp_fp4(const uint16_t* X, const void* expert_ids, int ids_i64,
                              const float* probs, int T, int k, int E, int H, int I,
                              const uint32_t* Bgu, const uint16_t* Sgu, const uint32_t* Bdn,
                              const uint16_t* Sdn, int g, uint16_t* act_buf, uint16_t* y_buf,
                              int32_t* sort_buf, uint16_t* out, void* stream) {
  const char* who = "mm_moe_mlp_fp4";
  if (ids_i64)
    return moe_mlp(who, X, (const int64_t*)expert_ids, probs, T, k, E, H, I, Bgu, Sgu, Bdn, Sdn,
                   nullptr, nullptr, nullptr, nullptr, 0.0f, nullptr, g, act_buf, y_buf, sort_buf,
                   out, stream);
  return moe_mlp(who, X, (const int32_t*)expert_ids, probs, T, k, E, H, I, Bgu, Sgu, Bdn, Sdn,
                 nullptr, nullptr, nullptr, nullptr, 0.0f, nullptr, g, act_buf, y_buf, sort_buf,
                 out, stream);
}

extern "C" int mm_moe_mlp_shared_fp4(const uint16_t* X, const void* expert_ids, int ids_i64,
                                     const float* probs, int T, int k, int E, int H, int I,
                                     const uint32_t* Bgu, const uint16_t* Sgu,
                                     const uint32_t* Bdn, const uint16_t* Sdn,
                                     const uint32_t* Bsgu, const uint16_t* Ssgu,
                                     const uint32_t* Bsdn, const uint16_t* Ssdn,
                                     float shared_weight, const uint16_t* base, int g,
                                     uint16_t* act_buf, uint16_t* y_buf, int32_t* sort_buf,
                                     uint16_t* out, void* stream) {
  const char* who = "mm_moe_mlp_shared_fp4";
  MM_CHECK_ARG(Bsgu != nullptr, "%s: the shared expert's gate_up weights are required", who);
  if (ids_i64 || k == 0)
    return moe_mlp(who, X, (const int64_t*)expert_ids, probs, T, k, E, H, I, Bgu, Sgu, Bdn, Sdn,
                   Bsgu, Ssgu, Bsdn, Ssdn, shared_weight, base, g, act_buf, y_buf, sort_buf, out,
                   stream);
  return moe_mlp(who, X, (const int32_t*)expert_ids, probs, T, k, E, H, I, Bgu, Sgu, Bdn, Sdn,
                 Bsgu, Ssgu, Bsdn, Ssdn, shared_weight, base, g, act_buf, y_buf, sort_buf, out,
                 stream);
}

extern "C" int mm_moe_gemm_shared_fp4(const uint16_t* X, const void* expert_ids, int ids_i64,
                                      const float* probs, int T, int k, int E, int K, int N,
                                      const uint32_t* Bsh, const uint16_t* Ssh,
                                      const uint32_t* B, const uint16_t* S, int g,
                                      uint16_t* y_buf, int32_t* sort_buf, uint16_t* out,
                                      void* stream) {
  const char* who = "mm_moe_gemm_shared_fp4";
  if (ids_i64 || k == 0)
    return moe_gemm_shared(who, X, (const int64_t*)expert_ids, probs, T, k, E, K, N, Bsh, Ssh,
                           B, S, g, y_buf, sort_buf, out, stream);
  return moe_gemm_shared(who, X, (const int32_t*)expert_ids, probs, T, k, E, K, N, Bsh, Ssh, B,
                         S, g, y_buf, sort_buf, out, stream);
}
