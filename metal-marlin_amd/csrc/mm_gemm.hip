// Fused FP4 (E2M1) / INT4 dequant-GEMM for gfx950:  C[M,N] = A[M,K] . dequant(B, S[, Z])
//
// Reference path: metal_marlin/kernels_core.py:1830-1937 (marlin_gemm_fp4),
// :1959-2066 (marlin_gemm_int4), metal_dispatch.py:4045-4181 (dispatch_gemm_fp4)
// and the Metal kernels src/marlin_gemm.metal:938-1150, 2053-2532,
// src/decode_gemv.metal:204-266.  Numerics: each weight is dequantised to the
// reference's fp16 value (mm_common.h), products accumulate in fp32 on the
// matrix cores, and the result is rounded once to fp16.
//
// Two kernels:
//  * skinny (M <= 32, decode): weights stream HBM -> registers -> MFMA with no
//    LDS staging; the M rows ride in a 16-row MFMA operand (zero padded).  A
//    block holds NW waves that split its K range; the block reduces the waves
//    in LDS, and a K split across blocks is reduced by the last-arriving block
//    (deterministic order, counter left at zero for the next call).
//  * prefill (M > 32): 32x32x16 MFMA tiles, A double-buffered through LDS,
//    B loaded as packed words one chunk ahead and dequantised in registers.
#include <algorithm>
#include <mutex>
#include <type_traits>

#include "mm_common.h"
#include "mm_skinny.h"
#include "mm_prefill.h"

// ===========================================================================
// Skinny path
// ===========================================================================
namespace {
using namespace mmsk;
using namespace mmpf;

constexpr int SK_RED_BATCH = 8;   // partial-sum loads in flight per thread

// SiLU(gate) * up in fp32 (the gate/up sums are never rounded to fp16 first).
MM_DEV float swiglu(float gate, float up) { return gate / (1.0f + __expf(-gate)) * up; }

// Epilogue modes of the dense skinny kernel.
//   SK_PLAIN : C[:, n] = A . W[:, n]                          (one matrix)
//   SK_SWIGLU: C[:, n] = silu(A . Wg[:, n]) * (A . Wu[:, n])   (gate, up; C is [M, N])
//   SK_PAIR  : C[:, n] = A . Wg[:, n], C[:, N + n] = A . Wu[:, n]   (C is [M, 2N])
//   SK_MULTI : up to three independent products sharing A and K (Q, K, V):
//              the grid's column tiles are the three matrices' tiles in turn.
enum { SK_PLAIN = 0, SK_SWIGLU = 1, SK_PAIR = 2, SK_MULTI = 3 };

// SK_MULTI problem table: matrix p owns column tiles [tile0[p], tile0[p+1])
// and partial-sum columns [cbase[p], cbase[p] + N[p]) of a [ksplit][M][ntot]
// buffer; C[p] is [M, N[p]].
struct SkMulti {
  const uint32_t* B[3];
  const f16* S[3];
  const f16* Z[3];
  f16* C[3];
  int N[3];
  int tile0[4];
  int cbase[3];
  int ntot;
};

// Dense skinny kernel.  grid = (column tiles, ksplit).  SK_PLAIN / SK_MULTI:
// a block covers NT adjacent 64-column tiles of one matrix.  SK_SWIGLU /
// SK_PAIR (NT = 2): tile 0 is columns [n0, n0+64) of (B, S, Z) and tile 1
// the same columns of (B2, S2, Z2).  Split-K partials are [ksplit][M][PW]
// fp32 with PW = N, 2N for the pair modes (gate at n, up at N + n), or ntot.
// ROWP: 0 Marlin-layout weights; 1, 2 row-packed [N, K/8] weights with
// scales [N, K/g] (1) or [K/g, N] (2), transposed through LDS into the
// Marlin operand order (skinny_wave RT); 3 Marlin-layout weights with scales
// [N, K/g].
// Row-packed single-tile blocks: the RT staging takes a few registers over
// the 128 that keep two 8-wave blocks resident per CU; at that limit the
// flush intervals listed here compile without spills (the others keep the
// default).  Measured at M=1, 14336 -> 4096 split 7 ways: 11.9 us with the
// as-loaded staging this replaced, 10.7 us; 4096 -> 28672 15.3 -> 14.5 us.
template <int ROWP, int NT, int FL>
constexpr int sk_min_waves() {
  return NT == 1 && ((ROWP == 2 && (FL == 0 || FL >= 4)) || (ROWP == 1 && (FL == 0 || FL >= 8)))
             ? 4
             : 1;
}
template <int INT4, int MT, int NT, int SPW, int NW, int FL, int ACT, int ROWP = 0>
__global__ void __launch_bounds__(NW * 64, (sk_min_waves<ROWP, NT, FL>()))
k_skinny(const f16* __restrict__ A, int lda, const uint32_t* __restrict__ B,
         const f16* __restrict__ S, const f16* __restrict__ Z, const uint32_t* __restrict__ B2,
         const f16* __restrict__ S2, const f16* __restrict__ Z2, f16* __restrict__ C, int ldc,
         int M, int N, int K, int g, int nrounds, float* __restrict__ part,
         uint32_t* __restrict__ counters, SkMulti mp) {
  static_assert(ACT == SK_PLAIN || ACT == SK_MULTI || NT == 2,
                "pair modes use one tile of each matrix");
  constexpr bool ONE = ACT == SK_PLAIN || ACT == SK_MULTI;   // one matrix per block
  // Row-packed weights are staged through 8 KiB of LDS per wave and tile in
  // the main loop; the block reduction reuses the same memory afterwards.
  constexpr bool STAGE = ROWP == 1 || ROWP == 2;
  // 9..32 rows, one column tile: each wave's activation slab (16*MT rows x
  // 32*SPW k, 8 KiB) goes through LDS too, when every round lies inside K
  // (measured on MI355X, per Llama layer: M=16 46.6 -> 44.6 us, M=32
  // 69.7 -> 66.4 us; two-tile blocks, e.g. 4096 x 28672 at M=32, were slower
  // with it, 21.0 -> 22.0 us).
  constexpr bool ASTG = !STAGE && NT == 1 && 16 * MT * 4 * SPW == 512;
  constexpr int RED = row_items_lds_floats<MT, NT, NW>();
  constexpr int STG = STAGE ? NW * NT * 2048 : (ASTG ? NW * 2048 : 0);
  constexpr int LDSF = STG > RED ? STG : RED;   // floats
  __shared__ __attribute__((aligned(16))) float red[LDSF];
  __shared__ uint32_t s_last;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int c = lane & 15, q = lane >> 4;
  int tile = blockIdx.x, cbase = 0, PW = ONE ? N : 2 * N;
  if constexpr (ACT == SK_MULTI) {
    const int p = tile >= mp.tile0[2] ? 2 : (tile >= mp.tile0[1] ? 1 : 0);
    B = mp.B[p];
    S = mp.S[p];
    Z = mp.Z[p];
    C = mp.C[p];
    N = mp.N[p];
    ldc = N;
    tile -= mp.tile0[p];
    cbase = mp.cbase[p];
    PW = mp.ntot;
  }
  const int n0 = tile * (ONE ? NT : 1) * SK_COLS;
  const int ksplit = gridDim.y;
  // First column (lane group c) of tile t in C and in the partial-sum row.
  auto ccol = [&](int t) {
    return ONE ? n0 + t * SK_COLS + 4 * c : n0 + 4 * c + (ACT == SK_PAIR ? t * N : 0);
  };
  auto pcol = [&](int t) { return ONE ? cbase + n0 + t * SK_COLS + 4 * c : t * N + n0 + 4 * c; };
  // Steps owned by this block: NW*SPW*nrounds consecutive 32-k steps; waves
  // take interleaved SPW-step slabs so each round reads adjacent word rows.
  const int blk_st0 = blockIdx.y * NW * SPW * nrounds;
  f32x4 acc[MT][NT][4];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[mt][t][j] = f32x4{0, 0, 0, 0};

  SkTile tl[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t)
    tl[t] = ONE ? SkTile{B, S, Z, n0 + t * SK_COLS}
                : (t == 0 ? SkTile{B, S, Z, n0} : SkTile{B2, S2, Z2, n0});
  if constexpr (STAGE) {
    static_assert(!INT4 && ACT != SK_MULTI, "row-packed: FP4 product or gate/up pair");
    skinny_wave<false, MT, NT, SPW, FL, false, ROWP == 1, false, true>(
        A, lda, nullptr, 1, M, tl, N, K, g, blk_st0 + wave * SPW, nrounds, NW * SPW, acc,
        nullptr, (char*)red + wave * NT * 8192);
    __syncthreads();   // every wave is done with its staging area
  } else if (ASTG && M > 8 && K % (32 * SPW) == 0) {
    skinny_wave<INT4, MT, NT, SPW, FL, false, ROWP == 3, ASTG>(
        A, lda, nullptr, 1, M, tl, N, K, g, blk_st0 + wave * SPW, nrounds, NW * SPW, acc,
        (char*)red + wave * 8192);
    __syncthreads();   // every wave is done with its staging area
  } else {
    skinny_wave<INT4, MT, NT, SPW, FL, false, ROWP == 3>(A, lda, nullptr, 1, M, tl, N, K, g,
                                                         blk_st0 + wave * SPW, nrounds, NW * SPW,
                                                         acc);
  }
  // Row items (mt, rr): lane (c, q) of the owning wave holds row
  // 16*mt + 4*q + rr, columns 4*c .. 4*c + 3 of each tile.
  constexpr int IPW = row_items_per_wave<MT, NW>();
  f32x4 rv[IPW][NT];
  block_reduce_items<MT, NT, NW>(red, acc, M, rv);
  auto item_row = [&](int k) {
    const int it = wave + k * NW;
    return it < MT * 4 ? 16 * (it >> 2) + 4 * q + (it & 3) : M;
  };

  if (ksplit == 1) {
#pragma unroll
    for (int k = 0; k < IPW; ++k) {
      const int row = item_row(k);
      if (row >= M) continue;
      if constexpr (ACT == SK_SWIGLU) {
        const int col = n0 + 4 * c;
        if (col < N)
          *(f16x4*)(C + (size_t)row * ldc + col) =
              f16x4{(f16)swiglu(rv[k][0][0], rv[k][1][0]), (f16)swiglu(rv[k][0][1], rv[k][1][1]),
                    (f16)swiglu(rv[k][0][2], rv[k][1][2]), (f16)swiglu(rv[k][0][3], rv[k][1][3])};
      } else {
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          const int col = ONE ? n0 + t * SK_COLS + 4 * c : n0 + 4 * c;
          if (col < N)
            *(f16x4*)(C + (size_t)row * ldc + ccol(t)) =
                f16x4{(f16)rv[k][t][0], (f16)rv[k][t][1], (f16)rv[k][t][2], (f16)rv[k][t][3]};
        }
      }
    }
    return;
  }
  // K split across blocks: publish this block's partial tile, then the last
  // block of the column tile sums all partials in split order.  Partials are
  // moved with 16-byte sc1 buffer accesses (the agent-scope policy: coherent
  // across the XCDs' L2s without writing back whole caches) and the counter
  // with an agent-scope atomic; waiting for each wave's stores orders them
  // before the counter bump.
  const __amdgpu_buffer_rsrc_t prs = mm_rsrc(part);
#pragma unroll
  for (int k = 0; k < IPW; ++k) {
    const int row = item_row(k);
    if (row >= M) continue;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int col = ONE ? n0 + t * SK_COLS + 4 * c : n0 + 4 * c;
      if (col < N)
        store_agent_x4(prs, 4u * (uint32_t)((blockIdx.y * M + row) * PW + pcol(t)), rv[k][t]);
    }
  }
  // Hand-off.  The partials are sc1 stores (coherent across the XCDs' L2s);
  // each wave's s_waitcnt(0) waits until its stores are performed at that
  // coherence point before it reaches the barrier, after which thread 0 bumps
  // the arrival counter; the last block reads them with sc1 loads.
  // This is the ordering the ISA gives a wave's memory operations.  The
  // language-level form (release increment, acquire read) was measured: the
  // agent-scope release writes back the whole L2 (buffer_wbl2) and took the
  // 14336 -> 4096 GEMM at M=1 from 9.4 to 22.4 us.
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t prev = __hip_atomic_fetch_add(&counters[blockIdx.x], 1u, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT);
    s_last = (prev == (uint32_t)ksplit - 1u) ? 1u : 0u;
  }
  __syncthreads();
  if (!s_last) return;
  // One thread per (row, 4-column) item sums the splits in order; the loads of
  // SK_RED_BATCH splits are issued together so the chain is ksplit/8 trips.
  // SK_SWIGLU items carry the gate and the up columns of one 4-column group.
  auto sum_splits = [&](int row, int pc) {
    f32x4 v = {0, 0, 0, 0};
    for (int y0 = 0; y0 < ksplit; y0 += SK_RED_BATCH) {
      f32x4 ld[SK_RED_BATCH];
#pragma unroll
      for (int i = 0; i < SK_RED_BATCH; ++i) {
        const int y = min(y0 + i, ksplit - 1);
        ld[i] = load_agent_x4(prs, 4u * (uint32_t)((y * M + row) * PW + pc));
      }
#pragma unroll
      for (int i = 0; i < SK_RED_BATCH; ++i)
        if (y0 + i < ksplit) v += ld[i];
    }
    return v;
  };
  constexpr int GROUPS = (ACT == SK_SWIGLU ? 1 : NT) * SK_COLS / 4;   // 4-column items per row
  const int nitems = min(M, MT * 16) * GROUPS;
  for (int e = threadIdx.x; e < nitems; e += NW * 64) {
    const int row = e / GROUPS, gi = e % GROUPS;
    if constexpr (ACT == SK_SWIGLU) {
      const int col = n0 + 4 * gi;
      if (col >= N) continue;
      const f32x4 gt = sum_splits(row, col), up = sum_splits(row, N + col);
      *(f16x4*)(C + (size_t)row * ldc + col) =
          f16x4{(f16)swiglu(gt[0], up[0]), (f16)swiglu(gt[1], up[1]),
                (f16)swiglu(gt[2], up[2]), (f16)swiglu(gt[3], up[3])};
    } else {
      const int t = gi / (SK_COLS / 4);
      const int col = (ONE ? n0 + t * SK_COLS : n0) + 4 * (gi % (SK_COLS / 4));
      if (col >= N) continue;
      const int oc = ONE ? col : t * N + col;
      const f32x4 v = sum_splits(row, ONE ? cbase + col : oc);
      *(f16x4*)(C + (size_t)row * ldc + oc) = f16x4{(f16)v[0], (f16)v[1], (f16)v[2], (f16)v[3]};
    }
  }
  if (threadIdx.x == 0)
    __hip_atomic_store(&counters[blockIdx.x], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Two-slab skinny kernel (M <= 8, K % 64 == 0, group size % 64 == 0): one
// block per 32 columns over the whole K, no split-K hand-off.  Each MFMA
// 16x16x32 step covers 64 k: rows 0..7 of the operand carry the activations
// of the first 32-k slab against columns 0..7 (weights of that slab), rows
// 8..15 the second slab against columns 8..15, so D[m][c] + D[8+m][8+c] is
// row m of the product for column group c.  Half-width tiles double the
// grid of narrow layers without a K split.
// ROWP: row-packed FP4 words [N, K/8] (K % 512 == 0), transposed through
// LDS into the Marlin operand order (skinny_wave RT); scales [N, K/g] when
// SROW, else [K/g, N].
template <int INT4, int SPW, int NW, int FL, bool SROW = false, bool ROWP = false>
__global__ void __launch_bounds__(NW * 64)
k_skinny_dual(const f16* __restrict__ A, const uint32_t* __restrict__ B,
              const f16* __restrict__ S, const f16* __restrict__ Z, f16* __restrict__ C, int M,
              int N, int K, int g, int nrounds) {
  // ROWP: each wave stages its weights through 8 KiB of LDS in the main
  // loop; the block reduction reuses the same memory afterwards.
  constexpr int RED = row_items_lds_floats<1, 1, NW>();
  constexpr int LDSF = ROWP && NW * 2048 > RED ? NW * 2048 : RED;   // floats
  __shared__ __attribute__((aligned(16))) float red[LDSF];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int c = lane & 15, q = lane >> 4;
  const int n0 = blockIdx.x * 32;
  f32x4 acc[1][1][4];
#pragma unroll
  for (int j = 0; j < 4; ++j) acc[0][0][j] = f32x4{0, 0, 0, 0};
  const SkTile tl[1] = {SkTile{B, S, Z, n0}};
  if constexpr (ROWP) {
    skinny_wave<false, 1, 1, SPW, FL, true, SROW, false, true>(
        A, K, nullptr, 1, M, tl, N, K, g, wave * SPW, nrounds, NW * SPW, acc, nullptr,
        (char*)red + wave * 8192);
    __syncthreads();   // every wave is done with its staging area
  } else
    skinny_wave<INT4, 1, 1, SPW, FL, true, SROW>(A, K, nullptr, 1, M, tl, N, K, g, wave * SPW,
                                                 nrounds, NW * SPW, acc);
  // Lanes q >= 2 hold the second slab's sums of the same rows (4*(q & 1) + rr):
  // items of rows < M are reduced over the waves, then lane (q, c) with
  // q < 2, c < 8 of the owning wave adds lane (q + 2, c + 8) = lane + 40.
  constexpr int IPW = row_items_per_wave<1, NW>();
  f32x4 rv[IPW][1];
  block_reduce_items<1, 1, NW, true>(red, acc, M, rv);
#pragma unroll
  for (int k = 0; k < IPW; ++k) {
    const int rr = wave + k * NW;   // wave-uniform
    if (rr >= 4 || rr >= M) continue;
    f32x4 v;
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = rv[k][0][j] + __shfl_down(rv[k][0][j], 40);
    const int row = 4 * q + rr, col = n0 + 4 * c;
    if (q < 2 && c < 8 && row < M && col < N)
      *(f16x4*)(C + (size_t)row * N + col) = f16x4{(f16)v[0], (f16)v[1], (f16)v[2], (f16)v[3]};
  }
}

// Column-strip kernel (M <= 16, group size a multiple of 32): one block per
// NS*16 columns over the whole K; no split-K and no workspace.
template <int INT4, int NS, int SPW, int NW, int FL>
__global__ void __launch_bounds__(NW * 64)
k_strip(const f16* __restrict__ A, int lda, const uint32_t* __restrict__ B,
        const f16* __restrict__ S, const f16* __restrict__ Z, f16* __restrict__ C, int ldc,
        int M, int N, int K, int g, int nrounds) {
  __shared__ float red[(NW - 1) * NS * 4 * 64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n0 = xcd_strip(blockIdx.x, gridDim.x) * 16 * NS;
  f32x4 acc[NS];
#pragma unroll
  for (int t = 0; t < NS; ++t) acc[t] = f32x4{0, 0, 0, 0};
  strip_wave<INT4, NS, SPW, FL>(A, lda, nullptr, 1, M, B, S, Z, N, K, g, n0, wave * SPW,
                                nrounds, NW * SPW, acc);
  strip_block_reduce<NS, NW>(red, acc, M);
  if (wave != 0) return;
  const int m = lane & 15, kb = lane >> 4;
  if (m >= M) return;
#pragma unroll
  for (int t = 0; t < NS; ++t) {
    const int col = n0 + 16 * t + 4 * kb;
    if (col < N)
      *(f16x4*)(C + (size_t)m * ldc + col) =
          f16x4{(f16)acc[t][0], (f16)acc[t][1], (f16)acc[t][2], (f16)acc[t][3]};
  }
}

// ===========================================================================
// Prefill path
// ===========================================================================
constexpr int PF_BK = 64;             // k per LDS chunk (4 MFMA k-steps of 16)
constexpr int PF_LDS_STRIDE = PF_BK + 8;  // halves; +16 B per row breaks bank aliasing

template <bool INT4, int WM, int WN, int RB>
__global__ void __launch_bounds__(WM * WN * 64)
k_prefill(const f16* __restrict__ A, int lda, const uint32_t* __restrict__ B,
          const f16* __restrict__ S, const f16* __restrict__ Z, f16* __restrict__ C, int ldc,
          int M, int N, int K, int g) {
  constexpr int NTHR = WM * WN * 64;
  constexpr int BM = WM * 32 * RB;
  constexpr int BN = WN * 128;
  constexpr int AVEC = BM * (PF_BK / 8);        // 16-byte A vectors per chunk
  static_assert(AVEC % NTHR == 0, "A chunk must split evenly over the block");
  constexpr int AV_PER_THR = AVEC / NTHR;
  __shared__ f16 As[2][BM * PF_LDS_STRIDE];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int l32 = lane & 31, h = lane >> 5;
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
  const int KP = K >> 3;
  const int nch = (K + PF_BK - 1) / PF_BK;
  const int ncol = n0 + wn * 128 + 4 * l32;
  const bool nok = ncol < N;

  f32x16 acc[RB][4];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[rb][j][v] = 0.0f;

  f16x8 areg[AV_PER_THR];
  u32x4 bcur[4], bnext[4];
  f16x4 scur[4], snext[4], zcur[4], znext[4];

  auto load_a = [&](int ch) {
#pragma unroll
    for (int i = 0; i < AV_PER_THR; ++i) {
      const int v = threadIdx.x + i * NTHR;
      const int row = v / (PF_BK / 8), c8 = v % (PF_BK / 8);
      const int m = m0 + row, k = ch * PF_BK + c8 * 8;
      areg[i] = (m < M && k < K) ? *(const f16x8*)(A + (size_t)m * lda + k)
                                 : f16x8{0, 0, 0, 0, 0, 0, 0, 0};
    }
  };
  auto store_a = [&](int buf) {
#pragma unroll
    for (int i = 0; i < AV_PER_THR; ++i) {
      const int v = threadIdx.x + i * NTHR;
      const int row = v / (PF_BK / 8), c8 = v % (PF_BK / 8);
      *(f16x8*)(&As[buf][row * PF_LDS_STRIDE + c8 * 8]) = areg[i];
    }
  };
  auto load_b = [&](int ch, u32x4 (&w)[4], f16x4 (&s)[4], f16x4 (&z)[4]) {
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int kp = ch * (PF_BK / 8) + 2 * t + h;
      const bool ok = nok && kp < KP;
      const int gi = (kp * 8) / g;
      w[t] = ok ? *(const u32x4*)(B + (size_t)kp * N + ncol) : u32x4{0, 0, 0, 0};
      s[t] = ok ? *(const f16x4*)(S + (size_t)gi * N + ncol) : f16x4{0, 0, 0, 0};
      if constexpr (INT4)
        z[t] = ok ? *(const f16x4*)(Z + (size_t)gi * N + ncol) : f16x4{0, 0, 0, 0};
    }
  };

  load_a(0);
  store_a(0);
  load_b(0, bcur, scur, zcur);

  for (int ch = 0; ch < nch; ++ch) {
    const int buf = ch & 1;
    const bool more = ch + 1 < nch;
    if (more) {
      load_a(ch + 1);
      load_b(ch + 1, bnext, snext, znext);
    }
    __syncthreads();
    const f16* as = &As[buf][(wm * 32 * RB + l32) * PF_LDS_STRIDE + 8 * h];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      f16x8 af[RB];
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
        af[rb] = *(const f16x8*)(as + rb * 32 * PF_LDS_STRIDE + 16 * t);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        f16 nz = 0;
        if constexpr (INT4) nz = -clamp_zero(zcur[t][j]);
        const f16x8 b = WordDq<INT4>::run(bcur[t][j], sanitize_scale(scur[t][j]), nz);
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
          acc[rb][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[rb], b, acc[rb][j], 0, 0, 0);
      }
    }
    if (more) {
      store_a(buf ^ 1);
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        bcur[t] = bnext[t];
        scur[t] = snext[t];
        if constexpr (INT4) zcur[t] = znext[t];
      }
    }
  }

  // Epilogue: lane holds column 4*l32 + j of tile j, rows 8*(v/4) + 4*h + v%4.
  if (!nok) return;
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int row = m0 + wm * 32 * RB + rb * 32 + 8 * (v >> 2) + 4 * h + (v & 3);
      if (row < M)
        *(f16x4*)(C + (size_t)row * ldc + ncol) =
            f16x4{(f16)acc[rb][0][v], (f16)acc[rb][1][v], (f16)acc[rb][2][v], (f16)acc[rb][3][v]};
    }
  }
}


// ===========================================================================
// Pipelined prefill path (main loop in mm_prefill.h)
// ===========================================================================
struct DenseSrc {
  const f16* A;
  int lda, M, m0, N, n0;
  const uint32_t* B;
  const f16* S;
  const f16* Z;
  int ld;
  MM_DEV const f16* arow(int r) const { return A + (size_t)min(m0 + r, M - 1) * lda; }
  MM_DEV const uint32_t* bcol(int P, int w) const { return B + min(n0 + P, N - w); }
  MM_DEV const f16* scol(int P, int w) const { return S + min(n0 + P, N - w); }
  MM_DEV const f16* zcol(int P, int w) const { return Z + min(n0 + P, N - w); }
};

// Row-packed FP4 weights B [N, K/8] (kp = K/8 words per column), scales
// [K/g, N] as DenseSrc.
struct DenseRowSrc {
  static constexpr bool kRowPacked = true;
  const f16* A;
  int lda, M, m0, N, n0;
  const uint32_t* B;
  const f16* S;
  const f16* Z;
  int ld, kp;
  MM_DEV const f16* arow(int r) const { return A + (size_t)min(m0 + r, M - 1) * lda; }
  MM_DEV const uint32_t* brow(int P) const { return B + (size_t)min(n0 + P, N - 1) * kp; }
  MM_DEV const f16* scol(int P, int w) const { return S + min(n0 + P, N - w); }
  MM_DEV const f16* zcol(int P, int w) const { return Z + min(n0 + P, N - w); }
};

// Gate/up pair: (B, S, Z) gate and (B2, S2, Z2) up matrices, both [.., N];
// n0 is the block's first output column.
struct PairSrc {
  const f16* A;
  int lda, M, m0, N, n0;
  const uint32_t *B, *B2;
  const f16 *S, *S2, *Z, *Z2;
  int ld;
  MM_DEV const f16* arow(int r) const { return A + (size_t)min(m0 + r, M - 1) * lda; }
  MM_DEV const uint32_t* bcol(int P, int w) const {
    return (pair_is_up(P) ? B2 : B) + pair_out_col(n0, P, w, N);
  }
  MM_DEV const f16* scol(int P, int w) const {
    return (pair_is_up(P) ? S2 : S) + pair_out_col(n0, P, w, N);
  }
  MM_DEV const f16* zcol(int P, int w) const {
    return (pair_is_up(P) ? Z2 : Z) + pair_out_col(n0, P, w, N);
  }
};

// Gate/up pair over row-packed [N, K/8] words (kp = K/8 words per column).
struct PairRowSrc {
  static constexpr bool kRowPacked = true;
  const f16* A;
  int lda, M, m0, N, n0;
  const uint32_t *B, *B2;
  const f16 *S, *S2, *Z, *Z2;
  int ld, kp;
  MM_DEV const f16* arow(int r) const { return A + (size_t)min(m0 + r, M - 1) * lda; }
  MM_DEV const uint32_t* brow(int P) const {
    return (pair_is_up(P) ? B2 : B) + (size_t)pair_out_col(n0, P, 1, N) * kp;
  }
  MM_DEV const f16* scol(int P, int w) const {
    return (pair_is_up(P) ? S2 : S) + pair_out_col(n0, P, w, N);
  }
  MM_DEV const f16* zcol(int P, int w) const {
    return (pair_is_up(P) ? Z2 : Z) + pair_out_col(n0, P, w, N);
  }
};

// ROWS: B (and B2) are row-packed [N, K/8] FP4 words.
template <bool INT4, int WM, int WN, int RB, int CW, bool G64, int ACT, bool ROWS = false>
__global__ void __launch_bounds__(WM * WN * 64)
k_prefill2(const f16* __restrict__ A, int lda, const uint32_t* __restrict__ B,
           const f16* __restrict__ S, const f16* __restrict__ Z, const uint32_t* __restrict__ B2,
           const f16* __restrict__ S2, const f16* __restrict__ Z2, f16* __restrict__ C, int ldc,
           int M, int N, int K, int g, float* __restrict__ part, int grp) {
  // Wave tile: (32*RB) rows x (32*CW) LDS columns.  SK_PLAIN: lane l32 owns
  // CW adjacent columns (CW packed words of one word row feed CW column
  // tiles).  Pair modes (CW = 2, tile-major): column tile 0 is 32 gate
  // columns and tile 1 the same 32 up columns, so a block covers BN/2 output
  // columns.  Requires K % 64 == 0 and N % 8 == 0 (checked by the host).
  static_assert(ACT == SK_PLAIN || CW == 2, "pair modes pair two column tiles");
  static_assert(!ROWS || !INT4, "row-packed weights: FP4");
  constexpr int SROWS = G64 ? PF2_SROWS_G64 : PF2_SROWS;
  using Sh = Pf2Shape<INT4, WM, WN, RB, CW, PF2_STAGES, SROWS>;
  __shared__ __attribute__((aligned(16))) char smem[Sh::LDS_BYTES];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int l32 = lane & 31, h = lane >> 5;
  // Tile placement.  Blocks are dealt round-robin to the 8 XCDs by linear id,
  // so the linear id is first remapped to give XCD x one contiguous run of
  // tile indices, and a tile index then walks groups of `grp` row tiles
  // column by column.  One XCD's run is about grp row tiles x (run / grp)
  // column tiles: an A row tile and a B column tile are each fetched by a
  // few XCDs instead of by all eight (the grid's x and y only count tiles).
  const int nx = gridDim.x, ny = gridDim.y;
  const int ntile = nx * ny * gridDim.z;
  const int L = blockIdx.x + nx * (blockIdx.y + ny * blockIdx.z);
  const int xq = ntile >> 3, xr = ntile & 7, xcd = L & 7;
  const int lin = xcd * xq + min(xcd, xr) + (L >> 3);
  const int bz = lin / (nx * ny), lt = lin - bz * (nx * ny);
  const int gi = lt / (grp * nx), gw = lt - gi * (grp * nx);
  const int gr = min(grp, ny - gi * grp);
  const int by = gi * grp + gw % gr, bx = gw / gr;
  const int m0 = by * Sh::BM;
  const int n0 = bx * (ACT == SK_PLAIN ? Sh::BN : Sh::BN / 2);
  // K split: split bz owns chunks [c_beg, c_end); with gridDim.z > 1 the
  // tile is written as an fp32 partial to part[z][M][PW] instead of C.
  const int nch_all = K / PF2_BK;
  const int cps = (nch_all + gridDim.z - 1) / gridDim.z;
  const int c_beg = bz * cps;
  const int c_end = min(nch_all, c_beg + cps);
  f32x16 acc[RB][CW];
  if constexpr (ROWS && ACT == SK_PLAIN) {
    const DenseRowSrc src{A, lda, M, m0, N, n0, B, S, Z, N, K / 8};
    pf2_mainloop<INT4, WM, WN, RB, CW, G64, false, PF2_STAGES, SROWS>(src, K, g, c_beg, c_end,
                                                                  smem, acc);
  } else if constexpr (ROWS) {
    const PairRowSrc src{A, lda, M, m0, N, n0, B, B2, S, S2, Z, Z2, N, K / 8};
    pf2_mainloop<INT4, WM, WN, RB, CW, G64, true, PF2_STAGES, SROWS>(src, K, g, c_beg, c_end,
                                                                 smem, acc);
  } else if constexpr (ACT == SK_PLAIN) {
    const DenseSrc src{A, lda, M, m0, N, n0, B, S, Z, N};
    pf2_mainloop<INT4, WM, WN, RB, CW, G64, false, PF2_STAGES, SROWS>(src, K, g, c_beg, c_end,
                                                                  smem, acc);
  } else {
    const PairSrc src{A, lda, M, m0, N, n0, B, B2, S, S2, Z, Z2, N};
    pf2_mainloop<INT4, WM, WN, RB, CW, G64, true, PF2_STAGES, SROWS>(src, K, g, c_beg, c_end,
                                                                  smem, acc);
  }

  typedef f16 svec __attribute__((ext_vector_type(CW)));
  typedef float fvec __attribute__((ext_vector_type(CW)));
  const int PW = ACT == SK_PLAIN ? N : 2 * N;
  const int ncol = ACT == SK_PLAIN ? n0 + wn * 32 * CW + CW * l32 : n0 + wn * 32 + l32;
  if (ncol >= N) return;
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int row = m0 + wm * 32 * RB + rb * 32 + 8 * (v >> 2) + 4 * h + (v & 3);
      if (row >= M) continue;
      if constexpr (ACT == SK_PLAIN) {
        if (gridDim.z == 1) {
          svec o;
#pragma unroll
          for (int j = 0; j < CW; ++j) o[j] = (f16)acc[rb][j][v];
          *(svec*)(C + (size_t)row * ldc + ncol) = o;
        } else {
          fvec o;
#pragma unroll
          for (int j = 0; j < CW; ++j) o[j] = acc[rb][j][v];
          *(fvec*)(part + ((size_t)bz * M + row) * PW + ncol) = o;
        }
      } else if (gridDim.z > 1) {
        float* prow = part + ((size_t)bz * M + row) * PW;
        prow[ncol] = acc[rb][0][v];
        prow[N + ncol] = acc[rb][1][v];
      } else if constexpr (ACT == SK_SWIGLU) {
        C[(size_t)row * ldc + ncol] = (f16)swiglu(acc[rb][0][v], acc[rb][1][v]);
      } else {
        C[(size_t)row * ldc + ncol] = (f16)acc[rb][0][v];
        C[(size_t)row * ldc + N + ncol] = (f16)acc[rb][1][v];
      }
    }
  }
}

// Sum the K-split partials of the prefill kernel in split order -> fp16 C.
// Partials are [ks][M][PW]; PW = N, or 2N for the pair modes (gate at n, up
// at N + n).  SK_SWIGLU writes silu(gate) * up to C [M, N]; the others copy
// the PW sums to C.
template <int ACT>
__global__ void __launch_bounds__(256)
k_splitk_reduce(const float* __restrict__ part, int ks, int M, int N, f16* __restrict__ C,
                int ldc) {
  const int PW = ACT == SK_PLAIN ? N : 2 * N;
  const int OW = ACT == SK_SWIGLU ? N : PW;                       // output columns
  const size_t i4 = (size_t)blockIdx.x * 256 + threadIdx.x;     // 4-column item
  const size_t items = (size_t)M * (OW / 4);
  if (i4 >= items) return;
  const int row = (int)(i4 / (OW / 4)), col = 4 * (int)(i4 % (OW / 4));
  f32x4 v = {0, 0, 0, 0}, u = {0, 0, 0, 0};
  for (int z = 0; z < ks; ++z) {
    const float* prow = part + ((size_t)z * M + row) * PW;
    v += *(const f32x4*)(prow + col);
    if constexpr (ACT == SK_SWIGLU) u += *(const f32x4*)(prow + N + col);
  }
  if constexpr (ACT == SK_SWIGLU)
    v = f32x4{swiglu(v[0], u[0]), swiglu(v[1], u[1]), swiglu(v[2], u[2]), swiglu(v[3], u[3])};
  *(f16x4*)(C + (size_t)row * ldc + col) = f16x4{(f16)v[0], (f16)v[1], (f16)v[2], (f16)v[3]};
}

// ===========================================================================
// Host-side planning.  The MM_SK_* / MM_ST_* / MM_PF_* constants are
// compile-time tunables (overridable with -D for tuning builds).
// ===========================================================================
#ifndef MM_SK_NW1
#define MM_SK_NW1 8         // waves per skinny block, M <= 16 (power of two)
#endif
#ifndef MM_SK_NW2
#define MM_SK_NW2 8         // waves per skinny block, 16 < M <= 32
#endif
#ifndef MM_SK_SPW1
#define MM_SK_SPW1 8        // 32-k steps per wave per round, M <= 16
#endif
#ifndef MM_SK_SPW2
#define MM_SK_SPW2 4        // 32-k steps per wave per round, 16 < M <= 32
#endif
// Max K split for 16 < M <= 32 (bounds partial traffic; 4 -> 8 measured on
// MI355X: 14336x4096 at M=17/24/32 13.9/14.5/15.0 -> 13.2/14.1/14.8 us,
// others unchanged).
#ifndef MM_SK_KS2
#define MM_SK_KS2 8
#endif
#ifndef MM_SK_NOSPLIT_TILES
#define MM_SK_NOSPLIT_TILES 200   // column tiles from which the K range is not split
#endif
#ifndef MM_SK_NOSPLIT_TILES1
#define MM_SK_NOSPLIT_TILES1 96   // the same for M <= 16
#endif
#ifndef MM_SK_MAXBLOCKS
#define MM_SK_MAXBLOCKS 2048
#endif
template <int MT> constexpr int sk_nw() { return MT == 1 ? MM_SK_NW1 : MM_SK_NW2; }
template <int MT> constexpr int sk_spw() { return MT == 1 ? MM_SK_SPW1 : MM_SK_SPW2; }
// The Marlin-layout gate/up pair (two column tiles per wave) at M <= 16 takes
// half-length slabs: twice the blocks along K for the same bytes.  Measured
// on MI355X, 4096 -> 2 x 14336, M=1: 13.7 -> 13.0 us; M=8 and M=16 within 1%.
// The row-packed pair keeps 8 steps (4 steps: M=1 16.7 -> 18.5 us).
#ifndef MM_SK_PAIR_SPW1
#define MM_SK_PAIR_SPW1 4
#endif
template <int MT, int ACT, int ROWP> constexpr int sk_spw_act() {
  return (ACT == SK_SWIGLU || ACT == SK_PAIR) && MT == 1 && ROWP == 0 ? MM_SK_PAIR_SPW1
                                                                      : sk_spw<MT>();
}
// One 64-column virtual-tile quad per block: more column tiles means fewer
// K splits (less partial-sum traffic) for the same parallelism.
template <int MT> constexpr int sk_nt() { return 1; }

struct SkinnyPlan {
  int ksplit;
  int nrounds;
  int ntiles;
};

SkinnyPlan plan_skinny(int M, int N, int K, int spw = 0) {
  SkinnyPlan p;
  const int nt = 1;
  if (spw == 0) spw = M <= 16 ? sk_spw<1>() : sk_spw<2>();
  const int nsteps = (K / 8 + 3) / 4;                  // 32-k steps
  const int slab = (M <= 16 ? sk_nw<1>() : sk_nw<2>()) * spw;   // steps per block round
  const int blocks_k = mm_cdiv(nsteps, slab);          // block-rounds along K
  p.ntiles = mm_cdiv(N, nt * SK_COLS);
  // One round per block (every load of a wave in flight at once) unless that
  // makes more than ~2048 blocks; for M > 16 cap the split at 8 to bound the
  // partial-sum traffic (ksplit * M * N * 4 bytes each way).
  int ks = blocks_k;
  if ((long)ks * p.ntiles > MM_SK_MAXBLOCKS) ks = mm_cdiv(MM_SK_MAXBLOCKS, p.ntiles);
  // With this many column tiles the grid already spreads over the CUs: a K
  // split would only add the hand-off and a second round of blocks (two
  // 8-wave blocks are resident per CU).  Measured on MI355X at M=1:
  // 4096x28672 16.8 -> 13.3 us, 4096x14336 10.0 -> 8.3 us; for M <= 16
  // from 96 tiles: 4096x6144 6.6 -> 5.6 us (two rounds per wave cost less
  // than the split-K hand-off).
  if (p.ntiles >= (M <= 16 ? MM_SK_NOSPLIT_TILES1 : MM_SK_NOSPLIT_TILES)) ks = 1;
  if (M > 16 && ks > MM_SK_KS2) ks = MM_SK_KS2;
  if (ks < 1) ks = 1;
  p.nrounds = mm_cdiv(blocks_k, ks);
  p.ksplit = mm_cdiv(blocks_k, p.nrounds);
  return p;
}

// The workspace starts with a fixed, shape-independent block of split-K
// arrival counters (one per column tile); partial sums follow it.
constexpr int SK_MAX_TILES = 16384;
constexpr size_t SK_COUNTER_BYTES = (size_t)SK_MAX_TILES * sizeof(uint32_t);

// Sized for the larger of the plain plan and the pair plan (its shorter
// slabs can split K further), so one figure serves both entry points.
size_t skinny_ws_bytes(int M, int N, int K) {
  int ks = plan_skinny(M, N, K).ksplit;
  if (M <= 16) ks = std::max(ks, plan_skinny(M, N, K, MM_SK_PAIR_SPW1).ksplit);
  if (ks == 1) return SK_COUNTER_BYTES;
  return SK_COUNTER_BYTES + (size_t)ks * M * N * sizeof(float);
}

// ACT = SK_PLAIN: C = A . B.  Pair modes: B/S/Z is the gate matrix and
// B2/S2/Z2 the up matrix, both [.., N]; the split and workspace are those of
// the unfused [K, 2N] product (plan_skinny(M, 2N, K)).
// SK_MULTI: `mp` describes the matrices (N is then mp->ntot, B..Z2 unused).
#define MM_ROWP_TILES 1      // 64-column tiles per block of the plain row-packed product; 2
                             // measured slower at M=1 (4096x6144 10.1 -> 18.8 us)
template <int INT4, int MT, int ACT, int ROWP = 0>
int launch_skinny(const f16* A, int lda, const uint32_t* B, const f16* S, const f16* Z,
                  const uint32_t* B2, const f16* S2, const f16* Z2, f16* C, int ldc, int M,
                  int N, int K, int g, void* ws, size_t ws_bytes, hipStream_t st,
                  const SkMulti* mp = nullptr) {
  const int PW = ACT == SK_PLAIN || ACT == SK_MULTI ? N : 2 * N;
  constexpr int SPW = sk_spw_act<MT, ACT, ROWP>();
  const SkinnyPlan p = plan_skinny(M, PW, K, SPW);
  constexpr int NT =
      ACT == SK_PLAIN || ACT == SK_MULTI ? (ROWP == 1 || ROWP == 2 ? MM_ROWP_TILES : sk_nt<MT>())
                                         : 2;
  const int gx = ACT == SK_PLAIN ? mm_cdiv(N, NT * SK_COLS)
                                 : (ACT == SK_MULTI ? mp->tile0[3] : mm_cdiv(N, SK_COLS));
  const SkMulti none{};
  MM_CHECK_ARG(gx <= SK_MAX_TILES, "gemm: N=%d exceeds the supported %d columns", N,
               SK_MAX_TILES * SK_COLS);
  uint32_t* counters = (uint32_t*)ws;
  float* part = nullptr;
  if (p.ksplit > 1) {
    const size_t need = skinny_ws_bytes(M, PW, K);
    MM_CHECK_ARG(ws != nullptr && ws_bytes >= need,
                 "gemm: workspace of %zu bytes is smaller than the %zu required", ws_bytes, need);
    part = (float*)((char*)ws + SK_COUNTER_BYTES);
  }
  dim3 grid(gx, p.ksplit);
  const int fl = flush_steps(g, SPW);
#define MM_LAUNCH_SK(FLV, RP)                                                               \
  hipLaunchKernelGGL((k_skinny<INT4, MT, NT, SPW, sk_nw<MT>(), FLV, ACT, RP>), grid,          \
                     dim3(sk_nw<MT>() * 64), 0, st, A, lda, B, S, Z, B2, S2, Z2, C, ldc, M, N, \
                     K, g, p.nrounds, part, counters, mp ? *mp : none)
#define MM_LAUNCH_SK_FL(RP)                                                                 \
  switch (fl) {                                                                             \
    case 1: MM_LAUNCH_SK(1, RP); break;                                                     \
    case 2: MM_LAUNCH_SK(2, RP); break;                                                     \
    case 4: MM_LAUNCH_SK(4 <= SPW ? 4 : 0, RP); break;                                      \
    case 8: MM_LAUNCH_SK(8 <= SPW ? 8 : 0, RP); break;                                      \
    default: MM_LAUNCH_SK(0, RP); break;                                                    \
  }
  MM_LAUNCH_SK_FL(ROWP)
#undef MM_LAUNCH_SK_FL
#undef MM_LAUNCH_SK
  MM_CHECK_LAUNCH("gemm(skinny)");
  return 0;
}

// Plain skinny product with two 64-column tiles per block and the whole K
// range per block (no split, so no workspace is touched).  The caller
// guarantees at least MM_SK_NOSPLIT_TILES blocks.  NW: waves per block; the
// dispatcher takes 4 from 24 rows up (measured on MI355X, 4096 x 28672:
// M=32 21.3 -> 19.8 us, M=24 20.3 -> 19.6 us with 4 waves; M=17 18.6 ->
// 19.9 us, so 8 below).
template <int INT4, int MT, int NW = sk_nw<MT>()>
int launch_skinny_nt2(const f16* A, const uint32_t* B, const f16* S, const f16* Z, f16* C, int M,
                      int N, int K, int g, hipStream_t st) {
  constexpr int NT = 2, SPW = sk_spw<MT>();
  const int nrounds = mm_cdiv((K / 8 + 3) / 4, NW * SPW);
  const dim3 grid(mm_cdiv(N, NT * SK_COLS), 1);
  const SkMulti none{};
#define MM_LAUNCH_SKN(FLV)                                                                    \
  hipLaunchKernelGGL((k_skinny<INT4, MT, NT, SPW, NW, FLV, SK_PLAIN, 0>), grid, dim3(NW * 64), \
                     0, st, A, K, B, S, Z, nullptr, nullptr, nullptr, C, N, M, N, K, g,         \
                     nrounds, nullptr, nullptr, none)
  switch (flush_steps(g, SPW)) {
    case 1: MM_LAUNCH_SKN(1); break;
    case 2: MM_LAUNCH_SKN(2); break;
    case 4: MM_LAUNCH_SKN(4 <= SPW ? 4 : 0); break;
    case 8: MM_LAUNCH_SKN(8 <= SPW ? 8 : 0); break;
    default: MM_LAUNCH_SKN(0); break;
  }
#undef MM_LAUNCH_SKN
  MM_CHECK_LAUNCH("gemm(skinny, 128-column blocks)");
  return 0;
}

#ifndef MM_SK_DUAL_NW
#define MM_SK_DUAL_NW 8
#endif
// 64-k steps per wave per round.  Measured at M=1 (qkv / o): 8 waves x 8
// steps 5.51 / 5.25 us, 8 x 4 5.46 / 5.12, 16 x 4 5.89 / 5.54, 4 x 8
// 6.12 / 5.79, 4 x 16 5.99 / 5.69.  With the row-item block reduction:
// 8 x 8 5.10-5.19 / 4.77-4.84, 16 x 4 5.01-5.03 / 4.65-4.68, 4 x 16
// 5.82 / 5.45, and the whole layer within run-to-run noise of 8 x 8.
#ifndef MM_SK_DUAL_SPW
#define MM_SK_DUAL_SPW MM_SK_SPW1
#endif
// The two-slab kernel serves M <= 8 layers whose 64-column plan runs unsplit
// on fewer than MM_SK_DUAL_BELOW blocks, when 32-column tiles give at least
// MM_SK_DUAL_MIN_TILES blocks (measured on MI355X at M=1: 4096 -> 6144
// 6.6 -> 5.3 us; 14336 -> 4096, which the 64-column plan splits 7 ways, is
// slower as 128 unsplit blocks, 9.3 -> 11.1 us, and keeps the split).  Small
// layers (K*N <= 4096^2) take it even where the 64-column plan would split:
// 4096 -> 4096 4.9 us against 5.2-5.3 us for the column-strip kernel.
#ifndef MM_SK_DUAL_BELOW
#define MM_SK_DUAL_BELOW 128
#endif
#ifndef MM_SK_DUAL_MIN_TILES
#define MM_SK_DUAL_MIN_TILES 96
#endif

bool use_dual(int M, int N, int K, int g) {
  if (M > 8 || K % 64 != 0 || g % 64 != 0 || N % 4 != 0) return false;
  if (flush_steps(g / 2, MM_SK_DUAL_SPW) == 0) return false;
  return (plan_skinny(M, N, K).ksplit == 1 || (long)K * N <= 4096L * 4096) &&
         mm_cdiv(N, SK_COLS) < MM_SK_DUAL_BELOW && mm_cdiv(N, 32) >= MM_SK_DUAL_MIN_TILES;
}

template <int INT4, bool SROW = false>
int launch_dual(const f16* A, const uint32_t* B, const f16* S, const f16* Z, f16* C, int M, int N,
                int K, int g, hipStream_t st) {
  constexpr int SPW = MM_SK_DUAL_SPW, NW = MM_SK_DUAL_NW;
  const int nsteps = K / 64;                           // 64-k steps
  const int nrounds = mm_cdiv(nsteps, NW * SPW);
  const int fl = flush_steps(g / 2, SPW);              // 64-k steps per scale group
#define MM_LAUNCH_DU(FLV)                                                                      \
  hipLaunchKernelGGL((k_skinny_dual<INT4, SPW, NW, FLV, SROW>), dim3(mm_cdiv(N, 32)), dim3(NW * 64), 0, \
                     st, A, B, S, Z, C, M, N, K, g, nrounds)
  switch (fl) {
    case 1: MM_LAUNCH_DU(1); break;
    case 2: MM_LAUNCH_DU(2); break;
    case 4: MM_LAUNCH_DU(4); break;
    case 8: MM_LAUNCH_DU(8 <= SPW ? 8 : 4); break;
    default: MM_CHECK_ARG(false, "gemm(dual): unsupported group size %d", g);
  }
#undef MM_LAUNCH_DU
  MM_CHECK_LAUNCH("gemm(dual)");
  return 0;
}

// The row-packed product takes the two-slab kernel on the shapes use_dual
// picks (measured slower on the others at M=1: 4096x28672 18.7 -> 20.9 us,
// 14336x4096 12.4 -> 16.7 us).

#ifndef MM_ST_NW
#define MM_ST_NW 8
#endif
#ifndef MM_ST_SPW
#define MM_ST_SPW 8
#endif

template <int INT4, int NS>
int launch_strip(const f16* A, int lda, const uint32_t* B, const f16* S, const f16* Z, f16* C,
                 int ldc, int M, int N, int K, int g, hipStream_t st) {
  constexpr int NW = MM_ST_NW, SPW = MM_ST_SPW;
  const int nsl = (K / 8 + 3) / 4;
  const int nrounds = mm_cdiv(nsl, NW * SPW);
  const int fl = flush_steps(g, SPW);
#define MM_LAUNCH_ST(FLV)                                                                     \
  hipLaunchKernelGGL((k_strip<INT4, NS, SPW, NW, FLV>), dim3(mm_cdiv(N, 16 * NS)), dim3(NW * 64), \
                     0, st, A, lda, B, S, Z, C, ldc, M, N, K, g, nrounds)
  switch (fl) {
    case 1: MM_LAUNCH_ST(1); break;
    case 2: MM_LAUNCH_ST(2); break;
    case 4: MM_LAUNCH_ST(4); break;
    case 8: MM_LAUNCH_ST(8 <= SPW ? 8 : 4); break;
    default: MM_CHECK_ARG(false, "gemm(strip): unsupported group size %d", g);
  }
#undef MM_LAUNCH_ST
  MM_CHECK_LAUNCH("gemm(strip)");
  return 0;
}

template <bool INT4, int WM, int WN, int RB>
int launch_prefill(const f16* A, int lda, const uint32_t* B, const f16* S, const f16* Z, f16* C,
                   int ldc, int M, int N, int K, int g, hipStream_t st) {
  constexpr int BM = WM * 32 * RB, BN = WN * 128;
  dim3 grid(mm_cdiv(N, BN), mm_cdiv(M, BM));
  hipLaunchKernelGGL((k_prefill<INT4, WM, WN, RB>), grid, dim3(WM * WN * 64), 0, st, A, lda, B, S,
                     Z, C, ldc, M, N, K, g);
  MM_CHECK_LAUNCH("gemm(prefill)");
  return 0;
}


// (WM, WN, RB, CW) of the pipelined prefill tiles.
#define PF2_BIG 2, 4, 4, 2       // 256 x 256, 8 waves of 128 x 64
#define PF2_MID 2, 4, 2, 2       // 128 x 256, 8 waves of 64 x 64
#define PF2_SMALL 1, 4, 2, 2     // 64 x 256, 4 waves of 64 x 64

#ifndef MM_PF_KS_BLOCKS
#define MM_PF_KS_BLOCKS 200   // split K while the grid has fewer blocks than this
#endif
// Prefill plan: tile config (0: 256x256, 1: 128x256, 2: 64x256) and K split.
struct PrefillPlan {
  int cfg;
  int ksplit;
};

PrefillPlan plan_prefill(int M, int N, int K) {
  PrefillPlan p;
  static const int BMs[3] = {256, 128, 64};
  const long t256 = (long)mm_cdiv(M, 256) * mm_cdiv(N, 256);
  p.cfg = (M > 128 && t256 >= 240) ? 0 : (M > 64 ? 1 : 2);
  const long blocks = (long)mm_cdiv(M, BMs[p.cfg]) * mm_cdiv(N, 256);
  // Split K when the grid cannot fill the 256 CUs; every split keeps >= 8
  // chunks of 64 k so the pipeline stays full.
  const int nch = K / PF2_BK;
  int ks = 1;
  while (blocks * ks < MM_PF_KS_BLOCKS && nch / (ks * 2) >= 8) ks *= 2;
  p.ksplit = ks;
  return p;
}

size_t prefill_ws_bytes(int M, int N, int K) {
  const PrefillPlan p = plan_prefill(M, N, K);
  return p.ksplit > 1 ? (size_t)p.ksplit * M * N * sizeof(float) : 0;
}

// Row-group height of k_prefill2's tile walk.  One XCD's run of tiles
// covers about grp row tiles x (run / grp) column tiles; each of its row
// tiles costs BM x 2 bytes of A per k and each column tile BN x 0.5 bytes of
// B (+ INT4 zeros: BN x ~0.03), so pick the power of two that minimises the
// XCD's A + B fetch.
int prefill_row_group(int nx, int ny, int nz, int BM, int BN, bool int4) {
  const int run = std::max(1, nx * ny * nz / 8);
  const double bcost = BN * (int4 ? 0.53 : 0.5);
  int best = 1;
  double best_cost = 1e300;
  for (int r = 1; r <= ny; r *= 2) {
    const int rows = std::min(ny, std::max(r, (run + nx - 1) / nx));
    const int cols = std::min(nx, (run + rows - 1) / rows);
    const double cost = rows * BM * 2.0 + cols * bcost;
    if (cost < best_cost) { best_cost = cost; best = r; }
  }
  return best;
}

template <bool INT4, int ACT, int WM, int WN, int RB, int CW, bool ROWS = false>
int launch_prefill2(const f16* A, int lda, const uint32_t* B, const f16* S, const f16* Z,
                    const uint32_t* B2, const f16* S2, const f16* Z2, f16* C, int ldc, int M,
                    int N, int K, int g, int ks, float* part, hipStream_t st) {
  constexpr int BM = WM * 32 * RB, BN = WN * 32 * CW;
  dim3 grid(mm_cdiv(N, ACT == SK_PLAIN ? BN : BN / 2), mm_cdiv(M, BM), ks);
  const int grp = prefill_row_group((int)grid.x, (int)grid.y, (int)grid.z, BM, BN, INT4);
  if (g % PF2_BK == 0)
    hipLaunchKernelGGL((k_prefill2<INT4, WM, WN, RB, CW, true, ACT, ROWS>), grid,
                       dim3(WM * WN * 64), 0, st, A, lda, B, S, Z, B2, S2, Z2, C, ldc, M, N, K, g,
                       part, grp);
  else if constexpr (!ROWS)
    hipLaunchKernelGGL((k_prefill2<INT4, WM, WN, RB, CW, false, ACT>), grid, dim3(WM * WN * 64),
                       0, st, A, lda, B, S, Z, B2, S2, Z2, C, ldc, M, N, K, g, part, grp);
  MM_CHECK_LAUNCH("gemm(prefill2)");
  if (ks > 1) {
    const int OW = ACT == SK_PLAIN ? N : (ACT == SK_SWIGLU ? N : 2 * N);
    const size_t items = (size_t)M * (OW / 4);
    hipLaunchKernelGGL(k_splitk_reduce<ACT>, dim3((unsigned)((items + 255) / 256)), dim3(256), 0,
                       st, part, ks, M, N, C, ldc);
    MM_CHECK_LAUNCH("gemm(prefill split-K reduce)");
  }
  return 0;
}

template <int INT4>
// INT4 == 2: SZ holds the scales and zero points interleaved ([K/g, N/4, 8],
// see load_sz4) for the decode kernels; the prefill kernels read S and Z.
int gemm_dispatch(const char* who, const f16* A, const uint32_t* B, const f16* S, const f16* Z,
                  f16* C, int M, int N, int K, int g, void* ws, size_t ws_bytes,
                  hipStream_t st, const f16* SZ = nullptr) {
  constexpr bool U4 = INT4 != 0;
  // the decode kernels' scale operand: SZ for the interleaved form
  const f16* Sd = INT4 == 2 ? SZ : S;
  MM_CHECK_ARG(M >= 0 && N > 0 && K > 0, "%s: bad shape M=%d N=%d K=%d", who, M, N, K);
  MM_CHECK_ARG(K % 8 == 0, "%s: K=%d must be divisible by 8", who, K);
  MM_CHECK_ARG(N % 4 == 0, "%s: N=%d must be divisible by 4", who, N);
  MM_CHECK_ARG(g > 0 && g % 8 == 0 && K % g == 0,
               "%s: group_size=%d must be a multiple of 8 dividing K=%d", who, g, K);
  MM_CHECK_ARG(((uintptr_t)A & 15) == 0 && ((uintptr_t)B & 15) == 0 && ((uintptr_t)S & 7) == 0 &&
                   ((uintptr_t)C & 7) == 0 && (!INT4 || ((uintptr_t)Z & 7) == 0) &&
                   (INT4 != 2 || ((uintptr_t)SZ & 15) == 0),
               "%s: operands must be 16-byte (A, B, interleaved scales/zeros) / 8-byte "
               "(scales, zeros, C) aligned", who);
  if (M == 0) return 0;
  // The decode kernels address one weight matrix with 32-bit byte offsets;
  // larger matrices take the prefill kernels (64-bit addressing) at any M.
  const bool off32 = (size_t)(K / 8) * (size_t)N * 4 < ((size_t)1 << 32);
  if (off32 && use_dual(M, N, K, g)) return launch_dual<INT4>(A, B, Sd, Z, C, M, N, K, g, st);
  if (off32 && M <= 16 && flush_steps(g, MM_ST_SPW) > 0) {
    // Column strips (no split-K hand-off) win for small layers, where the
    // hand-off is a large share of the launch; split-K wins from ~13 MB up
    // (measured on MI355X: 4096x4096 5.8 vs 7.0 us, 4096x6144 8.0 vs 7.2 us).
    if ((long)K * N <= 4096L * 4096 && N / 16 >= 128)
      return launch_strip<INT4, 1>(A, K, B, Sd, Z, C, N, M, N, K, g, st);
  }
  // Wide layers at 9..32 rows: 128-column blocks (NT = 2) with no K split.  The
  // activation rows each block reads are then shared by twice the weight
  // columns (measured on MI355X, 4096 x 28672: M=16 16.5 -> 15.0 us, M=32
  // 24.6 -> 20.4 us; at M <= 8 and on narrower layers the 64-column plan wins).
  if (off32 && M > 8 && M <= 32 && mm_cdiv(N, 2 * SK_COLS) >= MM_SK_NOSPLIT_TILES) {
    if (M <= 16) return launch_skinny_nt2<INT4, 1>(A, B, Sd, Z, C, M, N, K, g, st);
    if (M >= 24) return launch_skinny_nt2<INT4, 2, 4>(A, B, Sd, Z, C, M, N, K, g, st);
    return launch_skinny_nt2<INT4, 2>(A, B, Sd, Z, C, M, N, K, g, st);
  }
  if (off32 && M <= 16)
    return launch_skinny<INT4, 1, SK_PLAIN>(A, K, B, Sd, Z, nullptr, nullptr, nullptr, C, N, M, N,
                                            K, g, ws, ws_bytes, st);
  if (off32 && M <= 32)
    return launch_skinny<INT4, 2, SK_PLAIN>(A, K, B, Sd, Z, nullptr, nullptr, nullptr, C, N, M, N,
                                            K, g, ws, ws_bytes, st);
  // The pipelined kernel stages scale rows in 8-column pieces (N % 8 == 0)
  // and whole 64-k chunks (K % 64 == 0).
  if (N % 8 == 0 && K % PF2_BK == 0) {
    const PrefillPlan p = plan_prefill(M, N, K);
    float* part = nullptr;
    if (p.ksplit > 1) {
      const size_t need = SK_COUNTER_BYTES + prefill_ws_bytes(M, N, K);
      MM_CHECK_ARG(ws != nullptr && ws_bytes >= need,
                   "%s: workspace of %zu bytes is smaller than the %zu required", who, ws_bytes,
                   need);
      part = (float*)((char*)ws + SK_COUNTER_BYTES);
    }
    switch (p.cfg) {
      case 0:
        return launch_prefill2<U4, SK_PLAIN, PF2_BIG>(A, K, B, S, Z, nullptr, nullptr, nullptr,
                                                        C, N, M, N, K, g, p.ksplit, part, st);
      case 1:
        return launch_prefill2<U4, SK_PLAIN, PF2_MID>(A, K, B, S, Z, nullptr, nullptr, nullptr,
                                                        C, N, M, N, K, g, p.ksplit, part, st);
      default:
        return launch_prefill2<U4, SK_PLAIN, PF2_SMALL>(A, K, B, S, Z, nullptr, nullptr,
                                                          nullptr, C, N, M, N, K, g, p.ksplit,
                                                          part, st);
    }
  }
  // Prefill tiles: the largest tile that still gives about one block per CU.
  const long t256 = (long)mm_cdiv(M, 256) * mm_cdiv(N, 256);
  if (M > 128 && t256 >= 240)
    return launch_prefill<U4, 2, 2, 4>(A, K, B, S, Z, C, N, M, N, K, g, st);
  if (M > 64) return launch_prefill<U4, 2, 2, 2>(A, K, B, S, Z, C, N, M, N, K, g, st);
  return launch_prefill<U4, 1, 2, 2>(A, K, B, S, Z, C, N, M, N, K, g, st);
}

// Gate/up pair product (ACT = SK_SWIGLU or SK_PAIR) over two [K/8, N] packed
// matrices in one launch.  Decode sizes run the skinny kernel with one tile
// of each matrix per block; prefill sizes the pipelined kernel with
// tile-major gate/up columns.  Split-K and workspace are those of the
// unfused [K, 2N] product.
template <bool INT4, int ACT>
int pair_dispatch(const char* who, const f16* A, const uint32_t* Bg, const f16* Sg,
                  const f16* Zg, const uint32_t* Bu, const f16* Su, const f16* Zu, f16* C, int M,
                  int N, int K, int g, void* ws, size_t ws_bytes, hipStream_t st) {
  MM_CHECK_ARG(M >= 0 && N > 0 && K > 0, "%s: bad shape M=%d N=%d K=%d", who, M, N, K);
  MM_CHECK_ARG(K % 8 == 0, "%s: K=%d must be divisible by 8", who, K);
  MM_CHECK_ARG(N % 8 == 0, "%s: N=%d must be divisible by 8", who, N);
  MM_CHECK_ARG(g > 0 && g % 8 == 0 && K % g == 0,
               "%s: group_size=%d must be a multiple of 8 dividing K=%d", who, g, K);
  MM_CHECK_ARG(M <= 32 || K % PF2_BK == 0, "%s: K=%d must be divisible by %d for M > 32", who, K,
               PF2_BK);
  const uintptr_t a16 = (uintptr_t)A | (uintptr_t)Bg | (uintptr_t)Bu | (uintptr_t)Sg |
                        (uintptr_t)Su | (INT4 ? ((uintptr_t)Zg | (uintptr_t)Zu) : 0);
  MM_CHECK_ARG((a16 & 15) == 0 && ((uintptr_t)C & 7) == 0,
               "%s: A, packed weights, scales and zeros must be 16-byte aligned, C 8-byte", who);
  if (M == 0) return 0;
  const int ldc = ACT == SK_SWIGLU ? N : 2 * N;
  const bool off32 = (size_t)(K / 8) * (size_t)N * 4 < ((size_t)1 << 32);
  MM_CHECK_ARG(off32 || K % PF2_BK == 0, "%s: weights over 4 GiB need K %% %d == 0", who,
               PF2_BK);
  if (off32 && M <= 16)
    return launch_skinny<INT4, 1, ACT>(A, K, Bg, Sg, Zg, Bu, Su, Zu, C, ldc, M, N, K, g, ws,
                                       ws_bytes, st);
  if (off32 && M <= 32)
    return launch_skinny<INT4, 2, ACT>(A, K, Bg, Sg, Zg, Bu, Su, Zu, C, ldc, M, N, K, g, ws,
                                       ws_bytes, st);
  const PrefillPlan p = plan_prefill(M, 2 * N, K);
  float* part = nullptr;
  if (p.ksplit > 1) {
    const size_t need = SK_COUNTER_BYTES + prefill_ws_bytes(M, 2 * N, K);
    MM_CHECK_ARG(ws != nullptr && ws_bytes >= need,
                 "%s: workspace of %zu bytes is smaller than the %zu required", who, ws_bytes,
                 need);
    part = (float*)((char*)ws + SK_COUNTER_BYTES);
  }
  switch (p.cfg) {
    case 0:
      return launch_prefill2<INT4, ACT, PF2_BIG>(A, K, Bg, Sg, Zg, Bu, Su, Zu, C, ldc, M, N, K, g,
                                                 p.ksplit, part, st);
    case 1:
      return launch_prefill2<INT4, ACT, PF2_MID>(A, K, Bg, Sg, Zg, Bu, Su, Zu, C, ldc, M, N, K, g,
                                                 p.ksplit, part, st);
    default:
      return launch_prefill2<INT4, ACT, PF2_SMALL>(A, K, Bg, Sg, Zg, Bu, Su, Zu, C, ldc, M, N, K,
                                                   g, p.ksplit, part, st);
  }
}

// Up to three FP4 products sharing A (the Q, K and V projections): decode
// sizes run one SK_MULTI launch over all their column tiles; larger M runs
// one launch per matrix.
int multi_dispatch(const char* who, const f16* A, int nmat, const uint32_t* const* B,
                   const f16* const* S, f16* const* C, const int* N, int M, int K, int g,
                   void* ws, size_t ws_bytes, hipStream_t st) {
  MM_CHECK_ARG(nmat >= 1 && nmat <= 3, "%s: nmat=%d must be 1..3", who, nmat);
  MM_CHECK_ARG(B != nullptr && S != nullptr && C != nullptr && N != nullptr,
               "%s: null matrix table", who);
  MM_CHECK_ARG(M >= 0 && K > 0, "%s: bad shape M=%d K=%d", who, M, K);
  SkMulti mp{};
  int ntot = 0, tiles = 0;
  for (int p = 0; p < nmat; ++p) {
    MM_CHECK_ARG(N[p] > 0 && N[p] % 4 == 0, "%s: N[%d]=%d must be a positive multiple of 4",
                 who, p, N[p]);
    mp.B[p] = B[p];
    mp.S[p] = S[p];
    mp.C[p] = C[p];
    mp.N[p] = N[p];
    mp.tile0[p] = tiles;
    mp.cbase[p] = ntot;
    tiles += mm_cdiv(N[p], SK_COLS);
    ntot += N[p];
  }
  for (int p = nmat; p < 3; ++p) mp.tile0[p] = tiles;
  mp.tile0[3] = tiles;
  mp.ntot = ntot;
  bool off32 = true;
  for (int p = 0; p < nmat; ++p)
    off32 = off32 && (size_t)(K / 8) * (size_t)N[p] * 4 < ((size_t)1 << 32);
  if (!off32 || M > 16 || flush_steps(g, sk_spw<1>()) == 0 || K % 8 != 0 || g <= 0 ||
      K % g != 0) {
    // One product per launch (M > 16, or shapes the GEMM entry rejects with
    // its own message).
    for (int p = 0; p < nmat; ++p) {
      const int rc = gemm_dispatch<false>(who, A, B[p], S[p], nullptr, C[p], M, N[p], K, g, ws,
                                          ws_bytes, st);
      if (rc != 0) return rc;
    }
    return 0;
  }
  uintptr_t al = (uintptr_t)A;
  for (int p = 0; p < nmat; ++p) al |= (uintptr_t)B[p] | ((uintptr_t)S[p] & 7) | ((uintptr_t)C[p] & 7);
  MM_CHECK_ARG((al & 15) == 0, "%s: A, B 16-byte / scales, C 8-byte alignment required", who);
  MM_CHECK_ARG(tiles <= SK_MAX_TILES, "%s: too many columns", who);
  if (M == 0) return 0;
  return launch_skinny<false, 1, SK_MULTI>(A, K, nullptr, nullptr, nullptr, nullptr, nullptr,
                                           nullptr, nullptr, 0, M, ntot, K, g, ws, ws_bytes, st,
                                           &mp);
}

}  // namespace

// ===========================================================================
// C ABI
// ===========================================================================
extern "C" size_t mm_gemm_workspace_bytes(int M, int N, int K) {
  if (M <= 0 || N <= 0 || K <= 0) return SK_COUNTER_BYTES;
  if (M > 32) return SK_COUNTER_BYTES + prefill_ws_bytes(M, N, K);
  // 17..32 rows: enough for the prefill kernel too (the row-packed product
  // takes it from 17 rows).
  if (M > 16) return std::max(skinny_ws_bytes(M, N, K), SK_COUNTER_BYTES + prefill_ws_bytes(M, N, K));
  return skinny_ws_bytes(M, N, K);
}

extern "C" int mm_fp4_gemm(const uint16_t* A, const uint32_t* B, const uint16_t* S, uint16_t* C,
                           int M, int N, int K, int g, void* ws, size_t ws_bytes, void* stream) {
  return gemm_dispatch<false>("mm_fp4_gemm", (const f16*)A, B, (const f16*)S, nullptr, (f16*)C, M,
                              N, K, g, ws, ws_bytes, (hipStream_t)stream);
}

extern "C" int mm_fp4_gemm_rowpacked(const uint16_t* A, const uint32_t* B, const uint16_t* S,
                                     uint16_t* C, int M, int N, int K, int g, int scales_layout,
                                     void* ws, size_t ws_bytes, void* stream) {
  const char* who = "mm_fp4_gemm_rowpacked";
  MM_CHECK_ARG(scales_layout == 0 || scales_layout == 1,
               "%s: scales_layout=%d must be 0 ([K/g, N]) or 1 ([N, K/g])", who, scales_layout);
  MM_CHECK_ARG(M >= 0 && N > 0 && K > 0, "%s: bad shape M=%d N=%d K=%d", who, M, N, K);
  MM_CHECK_ARG(M <= 32 || scales_layout == 0,
               "%s: M=%d: above 32 rows the scales must be [K/g, N] (scales_layout 0)", who, M);
  MM_CHECK_ARG(M <= 32 || N % 8 == 0, "%s: N=%d must be divisible by 8 for M > 32", who, N);
  // The decode kernels take any multiple of 32 (one scale group per 32-k step
  // or more); the pipelined prefill kernel stages 64-k chunks of one group.
  MM_CHECK_ARG(g > 0 && g % (M <= 32 ? 32 : 64) == 0 && K % g == 0,
               "%s: group_size=%d must be a multiple of %d dividing K=%d", who, g,
               M <= 32 ? 32 : 64, K);
  MM_CHECK_ARG(N % 4 == 0, "%s: N=%d must be divisible by 4", who, N);
  MM_CHECK_ARG(M > 32 || (size_t)N * (size_t)(K / 8) * 4 < ((size_t)1 << 32),
               "%s: the packed weights must be under 4 GiB at M <= 32", who);
  // [K/g, N] scales are read as 4 adjacent columns (8 bytes) per lane.
  const uintptr_t salign = scales_layout == 0 ? 7 : 1;
  MM_CHECK_ARG(((uintptr_t)A & 15) == 0 && ((uintptr_t)B & 15) == 0 &&
                   ((uintptr_t)S & salign) == 0 && ((uintptr_t)C & 7) == 0,
               "%s: A and the packed weights must be 16-byte aligned, C 8-byte (and [K/g, N] "
               "scales 8-byte)", who);
  if (M == 0) return 0;
  hipStream_t st = (hipStream_t)stream;
  if (M > 16 && M <= 32) {
    // Two-row-block decode kernel, as the Marlin-layout path at these sizes.
    if (scales_layout == 1)
      return launch_skinny<false, 2, SK_PLAIN, 1>((const f16*)A, K, B, (const f16*)S, nullptr,
                                                  nullptr, nullptr, nullptr, (f16*)C, N, M, N,
                                                  K, g, ws, ws_bytes, st);
    return launch_skinny<false, 2, SK_PLAIN, 2>((const f16*)A, K, B, (const f16*)S, nullptr,
                                                nullptr, nullptr, nullptr, (f16*)C, N, M, N, K,
                                                g, ws, ws_bytes, st);
  }
  if (M > 32) {
    // Pipelined prefill kernel reading the row-packed words in place.
    const PrefillPlan p = plan_prefill(M, N, K);
    float* part = nullptr;
    if (p.ksplit > 1) {
      const size_t need = SK_COUNTER_BYTES + prefill_ws_bytes(M, N, K);
      MM_CHECK_ARG(ws != nullptr && ws_bytes >= need,
                   "%s: workspace of %zu bytes is smaller than the %zu required", who, ws_bytes,
                   need);
      part = (float*)((char*)ws + SK_COUNTER_BYTES);
    }
    const f16* a = (const f16*)A;
    const f16* s = (const f16*)S;
    switch (p.cfg) {
      case 0:
        return launch_prefill2<false, SK_PLAIN, PF2_BIG, true>(
            a, K, B, s, nullptr, nullptr, nullptr, nullptr, (f16*)C, N, M, N, K, g, p.ksplit,
            part, st);
      case 1:
        return launch_prefill2<false, SK_PLAIN, PF2_MID, true>(
            a, K, B, s, nullptr, nullptr, nullptr, nullptr, (f16*)C, N, M, N, K, g, p.ksplit,
            part, st);
      default:
        return launch_prefill2<false, SK_PLAIN, PF2_SMALL, true>(
            a, K, B, s, nullptr, nullptr, nullptr, nullptr, (f16*)C, N, M, N, K, g, p.ksplit,
            part, st);
    }
  }
  if (K % 512 == 0 && M <= 8 && use_dual(M, N, K, g)) {
    // Two-slab kernel, 32-column blocks over the whole K (the shapes the
    // Marlin-layout path also gives it).
    constexpr int NW = 8;
    const int nr = mm_cdiv(K / 64, NW * 8);
    // 64-k steps per scale group (0: a group size that no whole number of
    // steps matches -- use_dual excludes it -- decodes with the scale applied).
    const int fl = flush_steps(g / 2, 8);
#define MM_LAUNCH_RDU(FLV, SR)                                                                  \
  hipLaunchKernelGGL((k_skinny_dual<false, 8, NW, FLV, SR, true>), dim3(mm_cdiv(N, 32)),       \
                     dim3(NW * 64), 0, st, (const f16*)A, B, (const f16*)S, nullptr, (f16*)C, M,  \
                     N, K, g, nr)
#define MM_LAUNCH_RDU_FL(SR)                                                                    \
  switch (fl) {                                                                                \
    case 1: MM_LAUNCH_RDU(1, SR); break;                                                       \
    case 2: MM_LAUNCH_RDU(2, SR); break;                                                       \
    case 4: MM_LAUNCH_RDU(4, SR); break;                                                       \
    case 8: MM_LAUNCH_RDU(8, SR); break;                                                       \
    default: MM_LAUNCH_RDU(0, SR); break;                                                      \
  }
    if (scales_layout == 1) {
      MM_LAUNCH_RDU_FL(true)
    } else {
      MM_LAUNCH_RDU_FL(false)
    }
#undef MM_LAUNCH_RDU_FL
#undef MM_LAUNCH_RDU
    MM_CHECK_LAUNCH("gemm(rowpacked dual)");
    return 0;
  }
  if (scales_layout == 1)
    return launch_skinny<false, 1, SK_PLAIN, 1>((const f16*)A, K, B, (const f16*)S, nullptr,
                                                nullptr, nullptr, nullptr, (f16*)C, N, M, N, K,
                                                g, ws, ws_bytes, st);
  return launch_skinny<false, 1, SK_PLAIN, 2>((const f16*)A, K, B, (const f16*)S, nullptr,
                                              nullptr, nullptr, nullptr, (f16*)C, N, M, N, K, g,
                                              ws, ws_bytes, st);
}

extern "C" int mm_fp4_gemm_mmfp4(const uint16_t* A, const uint32_t* B, const uint16_t* S,
                                 uint16_t* C, int M, int N, int K, int g, void* ws,
                                 size_t ws_bytes, void* stream) {
  const char* who = "mm_fp4_gemm_mmfp4";
  MM_CHECK_ARG(M >= 0 && N > 0 && K > 0, "%s: bad shape M=%d N=%d K=%d", who, M, N, K);
  MM_CHECK_ARG(M <= 16, "%s: M=%d: decode sizes only (M <= 16); larger M: transpose the "
               "scales to [K/g, N] and call mm_fp4_gemm", who, M);
  MM_CHECK_ARG(K % 8 == 0, "%s: K=%d must be divisible by 8", who, K);
  MM_CHECK_ARG(N % 4 == 0, "%s: N=%d must be divisible by 4", who, N);
  MM_CHECK_ARG(g > 0 && g % 8 == 0 && K % g == 0,
               "%s: group_size=%d must be a multiple of 8 dividing K=%d", who, g, K);
  MM_CHECK_ARG((size_t)(K / 8) * (size_t)N * 4 < ((size_t)1 << 32),
               "%s: the packed weights must be under 4 GiB", who);
  MM_CHECK_ARG(((uintptr_t)A & 15) == 0 && ((uintptr_t)B & 15) == 0 && ((uintptr_t)S & 1) == 0 &&
                   ((uintptr_t)C & 7) == 0,
               "%s: A and the packed weights must be 16-byte aligned, C 8-byte", who);
  if (M == 0) return 0;
  if (use_dual(M, N, K, g))
    return launch_dual<false, true>((const f16*)A, B, (const f16*)S, nullptr, (f16*)C, M, N, K, g,
                                    (hipStream_t)stream);
  return launch_skinny<false, 1, SK_PLAIN, 3>((const f16*)A, K, B, (const f16*)S, nullptr,
                                              nullptr, nullptr, nullptr, (f16*)C, N, M, N, K, g,
                                              ws, ws_bytes, (hipStream_t)stream);
}

extern "C" int mm_fp4_gate_up_rowpacked(const uint16_t* A, const uint32_t* Bg, const uint16_t* Sg,
                                        const uint32_t* Bu, const uint16_t* Su, uint16_t* C,
                                        int M, int N, int K, int g, int act, void* ws,
                                        size_t ws_bytes, void* stream) {
  const char* who = "mm_fp4_gate_up_rowpacked";
  MM_CHECK_ARG(act == 0 || act == 1, "%s: act=%d must be 0 or 1", who, act);
  MM_CHECK_ARG(M >= 0 && N > 0 && K > 0, "%s: bad shape M=%d N=%d K=%d", who, M, N, K);
  // The decode kernels take any multiple of 32 (one scale group per 32-k step
  // or more); the pipelined prefill kernel stages 64-k chunks of one group.
  MM_CHECK_ARG(g > 0 && g % (M <= 32 ? 32 : 64) == 0 && K % g == 0,
               "%s: group_size=%d must be a multiple of %d dividing K=%d", who, g,
               M <= 32 ? 32 : 64, K);
  MM_CHECK_ARG(N % 8 == 0, "%s: N=%d must be divisible by 8", who, N);
  MM_CHECK_ARG(M > 32 || (size_t)N * (size_t)(K / 8) * 4 < ((size_t)1 << 32),
               "%s: each packed matrix must be under 4 GiB at M <= 32", who);
  const uintptr_t a16 = (uintptr_t)A | (uintptr_t)Bg | (uintptr_t)Bu;
  MM_CHECK_ARG((a16 & 15) == 0 && (((uintptr_t)Sg | (uintptr_t)Su) & 7) == 0 &&
                   ((uintptr_t)C & 7) == 0,
               "%s: A and the packed weights must be 16-byte aligned, scales and C 8-byte", who);
  if (M == 0) return 0;
  const int ldc = act ? N : 2 * N;
  if (M > 16 && M <= 32) {
    // Two-row-block decode kernel over both matrices, as the Marlin-layout
    // pair at these sizes.
    if (act)
      return launch_skinny<false, 2, SK_SWIGLU, 2>((const f16*)A, K, Bg, (const f16*)Sg, nullptr,
                                                   Bu, (const f16*)Su, nullptr, (f16*)C, ldc, M,
                                                   N, K, g, ws, ws_bytes, (hipStream_t)stream);
    return launch_skinny<false, 2, SK_PAIR, 2>((const f16*)A, K, Bg, (const f16*)Sg, nullptr, Bu,
                                               (const f16*)Su, nullptr, (f16*)C, ldc, M, N, K, g,
                                               ws, ws_bytes, (hipStream_t)stream);
  }
  if (M > 32) {
    // Pipelined prefill kernel reading both row-packed matrices in place;
    // split and workspace as the unfused [K, 2N] product.
    const PrefillPlan p = plan_prefill(M, 2 * N, K);
    float* part = nullptr;
    if (p.ksplit > 1) {
      const size_t need = SK_COUNTER_BYTES + prefill_ws_bytes(M, 2 * N, K);
      MM_CHECK_ARG(ws != nullptr && ws_bytes >= need,
                   "%s: workspace of %zu bytes is smaller than the %zu required", who, ws_bytes,
                   need);
      part = (float*)((char*)ws + SK_COUNTER_BYTES);
    }
    const f16 *a = (const f16*)A, *sg = (const f16*)Sg, *su = (const f16*)Su;
    hipStream_t st = (hipStream_t)stream;
#define MM_LAUNCH_ROWS_PAIR(ACTV, CFG)                                                       \
  return launch_prefill2<false, ACTV, CFG, true>(a, K, Bg, sg, nullptr, Bu, su, nullptr,       \
                                                 (f16*)C, ldc, M, N, K, g, p.ksplit, part, st)
#define MM_LAUNCH_ROWS_PAIR_CFG(ACTV)                                                        \
  switch (p.cfg) {                                                                           \
    case 0: MM_LAUNCH_ROWS_PAIR(ACTV, PF2_BIG);                                              \
    case 1: MM_LAUNCH_ROWS_PAIR(ACTV, PF2_MID);                                              \
    default: MM_LAUNCH_ROWS_PAIR(ACTV, PF2_SMALL);                                           \
  }
    if (act) MM_LAUNCH_ROWS_PAIR_CFG(SK_SWIGLU)
    MM_LAUNCH_ROWS_PAIR_CFG(SK_PAIR)
#undef MM_LAUNCH_ROWS_PAIR_CFG
#undef MM_LAUNCH_ROWS_PAIR
  }
  if (act)
    return launch_skinny<false, 1, SK_SWIGLU, 2>((const f16*)A, K, Bg, (const f16*)Sg, nullptr,
                                                 Bu, (const f16*)Su, nullptr, (f16*)C, ldc, M,
                                                 N, K, g, ws, ws_bytes, (hipStream_t)stream);
  return launch_skinny<false, 1, SK_PAIR, 2>((const f16*)A, K, Bg, (const f16*)Sg, nullptr, Bu,
                                             (const f16*)Su, nullptr, (f16*)C, ldc, M, N, K, g, ws,
                                             ws_bytes, (hipStream_t)stream);
}

extern "C" int mm_u4_gemm(const uint16_t* A, const uint32_t* B, const uint16_t* S,
                          const uint16_t* Z, uint16_t* C, int M, int N, int K, int g, void* ws,
                          size_t ws_bytes, void* stream) {
  return gemm_dispatch<1>("mm_u4_gemm", (const f16*)A, B, (const f16*)S, (const f16*)Z,
                             (f16*)C, M, N, K, g, ws, ws_bytes, (hipStream_t)stream);
}

extern "C" int mm_u4_gemm_sz(const uint16_t* A, const uint32_t* B, const uint16_t* S,
                             const uint16_t* Z, const uint16_t* SZ, uint16_t* C, int M, int N,
                             int K, int g, void* ws, size_t ws_bytes, void* stream) {
  MM_CHECK_ARG(SZ != nullptr, "mm_u4_gemm_sz: SZ (interleaved scales and zeros) is required");
  return gemm_dispatch<2>("mm_u4_gemm_sz", (const f16*)A, B, (const f16*)S, (const f16*)Z,
                          (f16*)C, M, N, K, g, ws, ws_bytes, (hipStream_t)stream,
                          (const f16*)SZ);
}

extern "C" int mm_fp4_gate_up(const uint16_t* A, const uint32_t* Bg, const uint16_t* Sg,
                              const uint32_t* Bu, const uint16_t* Su, uint16_t* C, int M, int N,
                              int K, int g, int act, void* ws, size_t ws_bytes, void* stream) {
  MM_CHECK_ARG(act == 0 || act == 1, "mm_fp4_gate_up: act=%d must be 0 or 1", act);
  if (act == 1)
    return pair_dispatch<false, SK_SWIGLU>("mm_fp4_gate_up", (const f16*)A, Bg, (const f16*)Sg,
                                           nullptr, Bu, (const f16*)Su, nullptr, (f16*)C, M, N, K,
                                           g, ws, ws_bytes, (hipStream_t)stream);
  return pair_dispatch<false, SK_PAIR>("mm_fp4_gate_up", (const f16*)A, Bg, (const f16*)Sg,
                                       nullptr, Bu, (const f16*)Su, nullptr, (f16*)C, M, N, K, g,
                                       ws, ws_bytes, (hipStream_t)stream);
}

extern "C" int mm_fp4_gemm_multi(const uint16_t* A, int nmat, const uint32_t* const* B,
                                 const uint16_t* const* S, uint16_t* const* C, const int* N, int M,
                                 int K, int g, void* ws, size_t ws_bytes, void* stream) {
  return multi_dispatch("mm_fp4_gemm_multi", (const f16*)A, nmat, B, (const f16* const*)S,
                        (f16* const*)C, N, M, K, g, ws, ws_bytes, (hipStream_t)stream);
}

// ===========================================================================
// No-allocation variant of mm_fp4_gemm: the workspace (split-K arrival
// counters and partial sums) is a file-scope device array, so a call makes no
// allocation of any kind.  Each device holds its own copy of the array for the
// life of the process; its address on a device is looked up once, with that
// device current, and kept per device.  The kernels leave the counters at zero
// after every call, so the array needs clearing only once (at set-up).  Every
// call on a device shares that device's array: calls that overlap on one
// device (several streams or threads) race.
// ===========================================================================
namespace {

constexpr size_t MM_NOALLOC_SCRATCH_BYTES = (size_t)32 << 20;   // 32 MiB
constexpr int MM_MAX_DEVICES = 64;

__device__ __align__(256) uint8_t scratch[MM_NOALLOC_SCRATCH_BYTES];

__global__ void __launch_bounds__(256) k_zero_words(uint32_t* p, size_t n) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256)
    p[i] = 0u;
}

std::mutex g_scratch_mu;
void* g_scratch_ptr[MM_MAX_DEVICES] = {};

// Address of this device's scratch array (set up on first use).
int noalloc_scratch(const char* who, hipStream_t st, void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  MM_CHECK_ARG(e == hipSuccess && dev >= 0 && dev < MM_MAX_DEVICES,
               "%s: no current HIP device (%s)", who, hipGetErrorString(e));
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    MM_CHECK_ARG(e == hipSuccess && p != nullptr,
                 "%s: hipGetSymbolAddress(scratch) failed on device %d: %s", who, dev,
                 hipGetErrorString(e));
    // Clear the counter block once (a fill kernel: no memset node for a
    // caller that captures this stream).
    hipLaunchKernelGGL(k_zero_words, dim3(64), dim3(256), 0, st, (uint32_t*)p,
                       SK_COUNTER_BYTES / sizeof(uint32_t));
    MM_CHECK_LAUNCH(who);
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return 0;
}

}  // namespace

extern "C" int mm_fp4_gemm_noalloc(const uint16_t* A, const uint32_t* B, const uint16_t* S,
                                   uint16_t* C, int M, int N, int K, int g, void* stream) {
  const char* who = "mm_fp4_gemm_noalloc";
  MM_CHECK_ARG(M >= 0 && N > 0 && K > 0, "%s: bad shape M=%d N=%d K=%d", who, M, N, K);
  const size_t need = mm_gemm_workspace_bytes(M, N, K);
  MM_CHECK_ARG(need <= MM_NOALLOC_SCRATCH_BYTES,
               "%s: M=%d N=%d K=%d needs %zu bytes of workspace, more than the %zu-byte "
               "built-in scratch (call mm_fp4_gemm with a workspace instead)",
               who, M, N, K, need, MM_NOALLOC_SCRATCH_BYTES);
  hipStream_t st = (hipStream_t)stream;
  void* ws = nullptr;
  const int rc = noalloc_scratch(who, st, &ws);
  if (rc) return rc;
  return gemm_dispatch<false>(who, (const f16*)A, B, (const f16*)S, nullptr, (f16*)C, M, N, K, g,
                              ws, MM_NOALLOC_SCRATCH_BYTES, st);
}
