// Skinny (decode-shaped, M <= 32) MFMA core shared by the dense and grouped
// GEMMs.  Weights stream HBM -> registers -> MFMA 16x16x32 with no LDS
// staging; the M rows ride in the 16-row MFMA operand.
//
// Lane l = 16*q + c of a wave, at 32-k step st:
//   B: one 16-byte load = word row kp = 4*st + q, columns n + 4c .. n + 4c + 3;
//      word j feeds "virtual" column tile j (its column c is matrix column 4c + j)
//   A: row 16*mt + c, k = 8*kp .. 8*kp + 7 (the 16x16x32 operand layout)
//   C: tile (mt, t, j), lane holds rows 16*mt + 4*q + r (r = 0..3), column 4c + j.
//
// Group scales: when the group size is a multiple of 32 (FL > 0) a group
// covers whole steps and the same group for every lane, so the MFMAs of a
// group accumulate unscaled E2M1 values and the group sum is multiplied by
// the fp32 scale once ("post-scale"); the per-word decode is then four packed
// converts.  INT4 groups accumulate a * (1024 + q) and subtract
// (1024 + z) * sum(a) (u4_magic_word below).  Other group sizes (FL == 0) scale every
// word in fp16 before the MFMA (the reference's rounding of each weight).
#pragma once
#include "mm_common.h"

// Weight words are streamed with non-temporal loads: each is read once per
// launch, and keeping them out of L2 and the Infinity Cache leaves those to
// the activations, scales and the following launches (measured on MI355X:
// Llama-3-8B layer at M=1 35.5 -> 33.8 us per step; the MoE decode MLP at
// T=32 70 -> 65 us).  Scale rows gain nothing from it and stay cached.
namespace mmsk {

constexpr int SK_COLS = 64;   // columns of one virtual-tile quad

// Pre-scaled word decode (exact reference fp16 weights).
template <bool INT4>
struct WordDq;
template <>
struct WordDq<false> {
  MM_DEV static f16x8 run(uint32_t w, f16 s, f16 /*nz*/) { return dq_fp4_word(w, f16x2{s, s}); }
};
template <>
struct WordDq<true> {
  MM_DEV static f16x8 run(uint32_t w, f16 s, f16 nz) {
    return dq_u4_word(w, f16x2{nz, nz}, f16x2{s, s});
  }
};

// Unscaled FP4 word decode: the E2M1 values.
MM_DEV f16x8 raw_fp4_word(uint32_t w) {
  const f16x2 p0 = e2m1_pair_c<0>(w), p1 = e2m1_pair_c<1>(w);
  const f16x2 p2 = e2m1_pair_c<2>(w), p3 = e2m1_pair_c<3>(w);
  return f16x8{p0.x, p0.y, p1.x, p1.y, p2.x, p2.y, p3.x, p3.y};
}

// INT4 post-scale decode.  Word w holds codes q0..q7 (nibble i = k row i).
// Each packed half is the fp16 number 1024 + q (exponent 10, q in the low
// mantissa bits), paired as (q0, q4), (q1, q5), (q2, q6), (q3, q7): one
// and-or per pair after a shift.  The MFMA then sums a * (1024 + q) exactly
// (11-bit by 11-bit products) and the group epilogue subtracts
// (1024 + z) * sum(a), with sum(a) from one extra MFMA against a ones
// operand.  The A operand is permuted to the same k order (a_k4_order).
MM_DEV f16x8 u4_magic_word(uint32_t w) {
  // (x & m) | (~m & c) is one v_bfi_b32 per pair; ~m & c == c here.  The
  // mask passes through an empty asm (no instruction) into an SGPR so the
  // compiler cannot fold ~m & c back to c -- with both constants literal it
  // emits a separate and + or (a gfx9 VOP3 takes no literal operand).
  uint32_t m = 0x000F000Fu;
  asm("" : "+s"(m));
  u32x4 p;
#pragma unroll
  for (int i = 0; i < 4; ++i) p[i] = ((w >> (4 * i)) & m) | (~m & 0x64006400u);
  return __builtin_bit_cast(f16x8, p);
}
// (a0..a7) -> (a0, a4, a1, a5, a2, a6, a3, a7): the k order of u4_magic_word.
MM_DEV f16x8 a_k4_order(f16x8 a) {
  const u32x4 d = __builtin_bit_cast(u32x4, a);
  u32x4 o;
  o[0] = __builtin_amdgcn_perm(d[2], d[0], 0x05040100u);
  o[1] = __builtin_amdgcn_perm(d[2], d[0], 0x07060302u);
  o[2] = __builtin_amdgcn_perm(d[3], d[1], 0x05040100u);
  o[3] = __builtin_amdgcn_perm(d[3], d[1], 0x07060302u);
  return __builtin_bit_cast(f16x8, o);
}
MM_DEV f16x8 f16x8_ones() {
  const f16 o = (f16)1.0f;
  return f16x8{o, o, o, o, o, o, o, o};
}

template <typename T>
MM_DEV const T* at_bytes(const void* base, uint32_t off) {
  return (const T*)((const char*)base + off);
}

// Scales (or zeros) of group gi for columns col .. col+3: [K/g, N] storage
// (one 8-byte load) or, with SROW, [N, K/g] storage of G = K/g groups per row.
template <bool SROW>
MM_DEV f16x4 load_scales4(const f16* S, uint32_t gi, uint32_t col, int N, int G) {
  if constexpr (!SROW) {
    return *at_bytes<f16x4>(S, (gi * (uint32_t)N + col) * 2u);
  } else {
    f16x4 v;
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = *at_bytes<f16>(S, ((col + j) * (uint32_t)G + gi) * 2u);
    return v;
  }
}

// INT4 == 2: scales and zero points interleaved in one array SZ [K/g, N/4, 8]
// (the 4 scales, then the 4 zero points, of each 4-column group): one 16-byte
// load per lane and group instead of two 8-byte loads.
MM_DEV void load_sz4(const f16* SZ, uint32_t gi, uint32_t col, int N, f16x4& s4, f16x4& z4) {
  const f16x8 v = *at_bytes<f16x8>(SZ, (gi * (uint32_t)N + col) * 4u);
  s4 = f16x4{v[0], v[1], v[2], v[3]};
  z4 = f16x4{v[4], v[5], v[6], v[7]};
}

// One 64-column tile of a packed weight matrix: its packed words, scales and
// (INT4) zeros, all [.., N] with row stride N, and the tile's first column.
// Tiles of one wave may come from different matrices of the same shape.
struct SkTile {
  const uint32_t* B;
  const f16* S;
  const f16* Z;
  int col0;
};

// One wave's contribution over `nrounds` rounds of SPW consecutive 32-k steps:
// round r covers steps st0 + r*ststride .. + SPW - 1, for NT column tiles.
// FL: steps per scale flush (> 0, power of two, <= SPW, and
// group_size == 32*FL*k for an integer k), or 0 for pre-scale.
// Rows >= M and columns past N compute values that are never stored: their
// addresses are clamped into the matrix so no load is predicated.
// SROW: scales (and zeros) stored [N, K/g] (the reference MMFP4 kernel's
// layout) instead of [K/g, N]: the four columns' values are four 2-byte loads.

// ASTG (16*MT rows x SPW steps = 8 KiB, no row map, every round inside K):
// each round's activation slab -- 16*MT rows x 32*SPW k (DUAL: 8 rows x
// 512 k) -- is loaded with whole lines (whole row segments per load
// instruction), written to the wave's LDS region `astage`, and the MFMA
// operands are read back from there.  Loaded directly, each operand load
// touched 16 rows' half-lines.  16-byte piece p of row r (p = word row within
// the round) lives at slot PPR * r + (p ^ sw(r)), PPR = 4*SPW (DUAL: 64)
// pieces per row, sw(r) = r % 16 (DUAL: bits 0, 1, 3 from r's bits 0, 1, 2),
// so the 16 lanes of a read pass hit 16 bank groups.
// RT (row-packed weights [N, K/8], FP4, SPW == 8 (or 4 without DUAL), every
// round inside K): each round's words -- 4*SPW word rows x 64 columns (DUAL:
// 64 x 32), 8 KiB per tile at SPW 8 -- are loaded with whole row segments (a
// column's 4*SPW*4 contiguous bytes, SPW or 16 lanes per column) and written to the wave's LDS region
// `rstage` transposed to the Marlin layout [word row][column], so the rest
// of the round (the k order, the post-scale decode, the MFMAs) is the
// Marlin-layout path's.  Word (row r, column x) lives at dword
// r * W + (x ^ 4 h(r)), W = 64 (DUAL: 32) columns, h(r) = (r >> 2) & 7: the
// four-column groups a lane reads stay contiguous, the lanes of a read pass
// hit distinct bank groups, and the transposing stores of one instruction
// hit 64 (DUAL: 32) distinct banks.
// INT4: 0 FP4, 1 INT4 (zeros in tl.Z), 2 INT4 with SZ interleaved in tl.S.
template <int INT4, int MT, int NT, int SPW, int FL, bool DUAL = false, bool SROW = false,
          bool ASTG = false, bool RT = false>
MM_DEV void skinny_wave(const f16* __restrict__ A, int lda, const int* __restrict__ rowmap,
                        int rowdiv, int M, const SkTile (&tl)[NT], int N, int K, int g,
                        int st0, int nrounds, int ststride, f32x4 (&acc)[MT][NT][4],
                        char* astage = nullptr, char* rstage = nullptr) {
  static_assert(!RT || (!INT4 && (SPW == 8 || (SPW == 4 && !DUAL)) && !ASTG),
                "row-packed staging: FP4, 8 steps (4 for single-slab blocks)");
  static_assert(FL == 0 || (SPW % FL == 0), "flush interval must divide the round");
  static_assert(!ASTG || (DUAL ? 8 * 64 : 16 * MT * 4 * SPW) == 512,
                "activation staging: an 8 KiB slab per wave");
  const int lane = threadIdx.x & 63;
  const int c = lane & 15, q = lane >> 4;
  // DUAL: a step is 64 k; lanes c < 8 take its first 32-k slab and lanes
  // c >= 8 the second, both for the 32 columns of lane group c & 7.
  constexpr int SLAB = DUAL ? 2 : 1;
  const int cl = DUAL ? (c & 7) : c, hs = DUAL ? (c >> 3) : 0;
  const int KP = K >> 3;
  const int nsteps = (KP + 4 * SLAB - 1) / (4 * SLAB);

  // Byte offset of A[row][0] in a buffer resource over A.  Operand rows past
  // M (the MFMA pads the rows to 16) get an offset past the resource's range,
  // so their loads return zeros without a memory request: at M = 1 one lane in
  // 16 fetches activations.
  const __amdgpu_buffer_rsrc_t ars = mm_rsrc(A);
  uint32_t aoff[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = min(mt * 16 + cl, M - 1);
    const int r = rowmap != nullptr ? rowmap[m] / rowdiv : m;
    aoff[mt] = mt * 16 + cl < M ? (uint32_t)r * (uint32_t)lda * 2u : MM_DEAD_OFFSET;
  }
  uint32_t coff[NT];                       // column index of this lane's first column
#pragma unroll
  for (int t = 0; t < NT; ++t) coff[t] = (uint32_t)min(tl[t].col0 + 4 * cl, N - 4);

  st0 = __builtin_amdgcn_readfirstlane(st0);   // wave-uniform: group indices stay scalar
  constexpr int NF = FL > 0 ? SPW / FL : 1;    // scale groups per round (post-scale)
  for (int r = 0; r < nrounds; ++r) {
    const int stb = st0 + r * ststride;    // wave-uniform
    if (stb >= nsteps) break;
    u32x4 w[SPW][NT];
    f16x8 a[SPW][MT];
    f16x4 s4[NF][NT], z4[NF][NT];
    // Issue every load of the round before any math: the (small) scale and
    // zero rows first, so that waiting for a step's weights never waits
    // behind a scale load issued later.
    if constexpr (FL > 0) {
#pragma unroll
      for (int f = 0; f < NF; ++f) {
        const int stg = min(stb + f * FL, nsteps - 1);
        const uint32_t gi = (uint32_t)((stg * 32 * SLAB) / g);      // scalar
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          if constexpr (INT4 == 2) {
            load_sz4(tl[t].S, gi, coff[t], N, s4[f][t], z4[f][t]);
          } else {
            s4[f][t] = load_scales4<SROW>(tl[t].S, gi, coff[t], N, K / g);
            if constexpr (INT4) z4[f][t] = load_scales4<SROW>(tl[t].Z, gi, coff[t], N, K / g);
          }
        }
      }
    }
    constexpr int PPR = DUAL ? 64 : 4 * SPW;   // ASTG: 16-byte pieces per row
    f16x8 ast[ASTG ? 8 : 1];                // ASTG: this lane's 8 slab pieces
    if constexpr (ASTG) {
      const uint32_t kb = (uint32_t)(4 * SLAB * stb);   // round's first word row
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int sl = 64 * i + lane;
        const int r = sl / PPR, pp = sl % PPR;
        const int sw = DUAL ? ((r & 3) | ((r & 4) << 1)) : (r & 15) % PPR;
        const int p = pp ^ sw;
        ast[i] = *at_bytes<f16x8>(A, (uint32_t)min(r, M - 1) * (uint32_t)lda * 2u +
                                         (kb + (uint32_t)p) * 16u);
      }
    }
    constexpr int RW = DUAL ? 32 : 64;       // RT: columns per tile (dwords per LDS row)
    constexpr int RPC = SLAB * SPW;          // RT: 16-byte pieces per column per round
    constexpr int RTB = RW * RPC * 16;       // RT: staging bytes per tile
    constexpr int RNI = RW * RPC / 64;       // RT: load instructions per tile
    u32x4 wp[RT ? NT : 1][RT ? RNI : 1];     // RT: this lane's loaded pieces per tile
    if constexpr (RT) {
      // A round overhanging K re-reads the column's last piece (its steps
      // are zeroed through the activation operand below), so every load stays
      // inside the column's KP words (KP % 4 == 0).
      const uint32_t kb = (uint32_t)(4 * SLAB * stb);   // round's first word row
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int i = 0; i < RNI; ++i) {
          const int sl = 64 * i + lane;
          const int x = sl / RPC, p = sl % RPC;
          const uint32_t cg = (uint32_t)min(tl[t].col0 + x, N - 1);
          const uint32_t kw = min(kb + 4u * (uint32_t)p, (uint32_t)KP - 4u);
          wp[t][i] = __builtin_nontemporal_load(
              at_bytes<u32x4>(tl[t].B, (cg * (uint32_t)KP + kw) * 4u));
        }
    }
#pragma unroll
    for (int i = 0; i < SPW; ++i) {
      const int kp = min(4 * (SLAB * min(stb + i, nsteps - 1) + hs) + q, KP - 1);
      if constexpr (!RT) {
#pragma unroll
        for (int t = 0; t < NT; ++t)
          w[i][t] = __builtin_nontemporal_load(
              at_bytes<u32x4>(tl[t].B, ((uint32_t)kp * (uint32_t)N + coff[t]) * 4u));
      }
      if constexpr (!ASTG) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
          a[i][mt] = __builtin_bit_cast(f16x8, __builtin_amdgcn_raw_buffer_load_b128(
                                                  ars, aoff[mt] + (uint32_t)kp * 16u, 0, 0));
      }
    }
    if constexpr (RT) {
      // Transpose through the wave's LDS region (its own: no barrier).
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int i = 0; i < RNI; ++i) {
          const int sl = 64 * i + lane;
          const int x = sl / RPC, p = sl % RPC;
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            const int row = 4 * p + k;
            *(uint32_t*)(rstage + RTB * t + (row * RW + (x ^ (4 * ((row >> 2) & 7)))) * 4) =
                wp[t][i][k];
          }
        }
#pragma unroll
      for (int i = 0; i < SPW; ++i) {
        const int row = 4 * (SLAB * i + hs) + q;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          const int x0 = (int)(coff[t] - (uint32_t)tl[t].col0);
          w[i][t] = *(const u32x4*)(rstage + RTB * t +
                                   (row * RW + (x0 ^ (4 * ((row >> 2) & 7)))) * 4);
        }
      }
    }
    if constexpr (ASTG) {
      // Through the wave's LDS region into the lanes' operand layout (the
      // region is the wave's own: no barrier).
#pragma unroll
      for (int i = 0; i < 8; ++i) *(f16x8*)(astage + 1024 * i + 16 * lane) = ast[i];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int r = 16 * mt + cl;          // rows >= M hold a duplicate of row M-1
        const int sw = DUAL ? ((r & 3) | ((r & 4) << 1)) : (r & 15) % PPR;
#pragma unroll
        for (int i = 0; i < SPW; ++i) {
          const int p = 4 * (SLAB * i + hs) + q;
          a[i][mt] = *(const f16x8*)(astage + (PPR * r + (p ^ sw)) * 16);
        }
      }
    }
    // Steps past K (a partial last step, or a round overhanging the end)
    // contribute zero through a zeroed activation operand.  (ASTG rounds lie
    // inside K.)
    if (!ASTG && (stb + SPW > nsteps || (K & (32 * SLAB - 1)) != 0)) {
#pragma unroll
      for (int i = 0; i < SPW; ++i) {
        const bool valid = stb + i < nsteps && 4 * (SLAB * (stb + i) + hs) + q < KP;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
          if (!valid) a[i][mt] = f16x8{0, 0, 0, 0, 0, 0, 0, 0};
      }
    }

    if constexpr (FL == 0) {
      // Pre-scale: each lane's own group, every step.
#pragma unroll
      for (int i = 0; i < SPW; ++i) {
        const int kp = min(4 * (SLAB * min(stb + i, nsteps - 1) + hs) + q, KP - 1);
        const uint32_t gi = (uint32_t)((kp * 8) / g);
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          f16x4 s4, z4 = {0, 0, 0, 0};
          if constexpr (INT4 == 2) {
            load_sz4(tl[t].S, gi, coff[t], N, s4, z4);
          } else {
            s4 = load_scales4<SROW>(tl[t].S, gi, coff[t], N, K / g);
            if constexpr (INT4) z4 = load_scales4<SROW>(tl[t].Z, gi, coff[t], N, K / g);
          }
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            f16 nz = 0;
            if constexpr (INT4) nz = -clamp_zero(z4[j]);
            const f16x8 b = WordDq<(INT4 != 0)>::run(w[i][t][j], sanitize_scale(s4[j]), nz);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
              acc[mt][t][j] =
                  __builtin_amdgcn_mfma_f32_16x16x32_f16(a[i][mt], b, acc[mt][t][j], 0, 0, 0);
          }
        }
      }
    } else {
      // Post-scale: one group per FL steps, uniform across the wave.
#pragma unroll
      for (int f = 0; f < NF; ++f) {
        f32x4 grp[MT][NT][4];
        f32x4 asum[MT];                     // INT4: sum of A over the group, per row
#pragma unroll
        for (int i = f * FL; i < (f + 1) * FL; ++i) {
          f16x8 ai[MT];
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            if constexpr (INT4) {
              asum[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                  a[i][mt], f16x8_ones(), i == f * FL ? f32x4{0, 0, 0, 0} : asum[mt], 0, 0, 0);
              ai[mt] = a_k4_order(a[i][mt]);
            } else {
              ai[mt] = a[i][mt];
            }
          }
#pragma unroll
          for (int t = 0; t < NT; ++t) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const f16x8 b = INT4 ? u4_magic_word(w[i][t][j]) : raw_fp4_word(w[i][t][j]);
#pragma unroll
              for (int mt = 0; mt < MT; ++mt)
                grp[mt][t][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                    ai[mt], b, i == f * FL ? f32x4{0, 0, 0, 0} : grp[mt][t][j], 0, 0, 0);
            }
          }
        }
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const float sc = (float)sanitize_scale(s4[f][t][j]);
            if constexpr (INT4) {
              const float zb = 1024.0f + (float)clamp_zero(z4[f][t][j]);
#pragma unroll
              for (int mt = 0; mt < MT; ++mt)
                acc[mt][t][j] += sc * (grp[mt][t][j] - zb * asum[mt]);
            } else {
#pragma unroll
              for (int mt = 0; mt < MT; ++mt) acc[mt][t][j] += sc * grp[mt][t][j];
            }
          }
      }
    }
  }
}

// Row-item block reduction.  A row item (mt, rr) of a lane (c, q) is its row
// 16*mt + 4*q + rr (DUALROWS: the logical row 4*(q & 1) + rr of the two-slab
// layout, whose lanes q >= 2 hold the second slab) with the four columns
// 4c + j (j = 0..3) of each tile t as one f32x4.  Every wave parks its items
// of rows < mrows in LDS (only the rows that are stored move: at one row a
// quarter of the accumulator), one barrier, then item i is summed over the
// waves by wave i % NW, in wave order (wave 0's value first, then waves 1, 2,
// ... added one at a time: a fixed order, so the sums are deterministic).  On
// return rv[k][t] holds item wave + k*NW of this wave (valid for its lanes
// whose row is < mrows).
template <int MT, int NW>
constexpr int row_items_per_wave() { return (MT * 4 + NW - 1) / NW; }
template <int MT, int NT, int NW>
constexpr int row_items_lds_floats() { return NW * MT * 4 * NT * 64 * 4; }

template <int MT, int NT, int NW, bool DUALROWS = false>
MM_DEV void block_reduce_items(float* red, const f32x4 (&acc)[MT][NT][4], int mrows,
                               f32x4 (&rv)[row_items_per_wave<MT, NW>()][NT]) {
  constexpr int NI = MT * 4, IPW = row_items_per_wave<MT, NW>();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, q = lane >> 4;
  const int qrow = DUALROWS ? 4 * (q & 1) : 4 * q;
  f32x4* slots = (f32x4*)red;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int rr = 0; rr < 4; ++rr)
      if ((DUALROWS ? 0 : 16 * mt) + qrow + rr < mrows) {
#pragma unroll
        for (int t = 0; t < NT; ++t)
          slots[((wave * NI + mt * 4 + rr) * NT + t) * 64 + lane] =
              f32x4{acc[mt][t][0][rr], acc[mt][t][1][rr], acc[mt][t][2][rr], acc[mt][t][3][rr]};
      }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < IPW; ++k) {
    const int it = wave + k * NW;   // wave-uniform
    // Items whose lowest row (q = 0) is already past mrows hold nothing.
    if (it >= NI || (DUALROWS ? 0 : 16 * (it >> 2)) + (it & 3) >= mrows) continue;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      f32x4 part[NW];
#pragma unroll
      for (int w = 0; w < NW; ++w) part[w] = slots[((w * NI + it) * NT + t) * 64 + lane];
      f32x4 v = part[0];
#pragma unroll
      for (int w = 1; w < NW; ++w) v += part[w];
      rv[k][t] = v;
    }
  }
}

// ---------------------------------------------------------------------------
// Column-strip core (M <= 16, g % 32 == 0; no split-K).  The weights are the
// MFMA A operand and the activations the B operand, so one MFMA 16x16x32
// consumes one packed word per lane:
//   lane l = 16*kb + i at slab sl (4 word rows = 32 k): weight word
//   (kp = 4*sl + kb, column n0 + 16*t + i) -- 16 lanes read 64 contiguous
//   bytes of a word row -- and activation row min(i, M-1), k = 8*kp .. +7.
//   D tile t: lane holds columns n0 + 16*t + 4*kb + r (r = 0..3), row m = i.
// Wave w takes slabs w*SPW + r*slstride + u.  Rounds are software-pipelined:
// round r+1's loads are issued before round r's math.
// ---------------------------------------------------------------------------
template <int NS, int SPW, int NF>
struct StripRound {
  uint32_t w[SPW][NS];
  f16x8 a[SPW];
  f16x4 s[NF][NS], z[NF][NS];   // scale (and INT4 zero) rows of the round's groups
};

template <int INT4, int NS, int SPW, int FL>
MM_DEV void strip_wave(const f16* __restrict__ A, int lda, const int* __restrict__ rowmap,
                       int rowdiv, int M, const uint32_t* __restrict__ B,
                       const f16* __restrict__ S, const f16* __restrict__ Z, int N, int K, int g,
                       int n0, int sl0, int nrounds, int slstride, f32x4 (&acc)[NS]) {
  static_assert(FL > 0 && SPW % FL == 0, "strip path needs a post-scale flush interval");
  const int lane = threadIdx.x & 63;
  const int i = lane & 15, kb = lane >> 4;
  const int KP = K >> 3;
  const int nsl = (KP + 3) >> 2;
  const int m = min(i, M - 1);
  // Operand rows past M fetch nothing (offset past the resource; see skinny_wave).
  const __amdgpu_buffer_rsrc_t ars = mm_rsrc(A);
  const uint32_t aoff = i < M ? (uint32_t)(rowmap != nullptr ? rowmap[m] / rowdiv : m) *
                                    (uint32_t)lda * 2u
                              : MM_DEAD_OFFSET;
  uint32_t bcol[NS], scol[NS];
#pragma unroll
  for (int t = 0; t < NS; ++t) {
    bcol[t] = (uint32_t)min(n0 + 16 * t + i, N - 1);           // weight column
    scol[t] = (uint32_t)min(n0 + 16 * t + 4 * kb, N - 4);      // output columns
  }
  constexpr int NF = SPW / FL;
  sl0 = __builtin_amdgcn_readfirstlane(sl0);   // wave-uniform: group indices stay scalar
  // Scales first: a wait for a slab's weights then never waits behind a
  // scale load issued after them.
  auto load = [&](int r, StripRound<NS, SPW, NF>& R) {
    const int slb = sl0 + r * slstride;
#pragma unroll
    for (int f = 0; f < NF; ++f) {
      const int slg = min(slb + f * FL, nsl - 1);
      const uint32_t gi = (uint32_t)((slg * 32) / g);
#pragma unroll
      for (int t = 0; t < NS; ++t) {
        if constexpr (INT4 == 2) {
          load_sz4(S, gi, scol[t], N, R.s[f][t], R.z[f][t]);
        } else {
          R.s[f][t] = *at_bytes<f16x4>(S, (gi * (uint32_t)N + scol[t]) * 2u);
          if constexpr (INT4) R.z[f][t] = *at_bytes<f16x4>(Z, (gi * (uint32_t)N + scol[t]) * 2u);
        }
      }
    }
#pragma unroll
    for (int u = 0; u < SPW; ++u) {
      const int kp = min(4 * min(slb + u, nsl - 1) + kb, KP - 1);
#pragma unroll
      for (int t = 0; t < NS; ++t)
        R.w[u][t] = __builtin_nontemporal_load(
            at_bytes<uint32_t>(B, ((uint32_t)kp * (uint32_t)N + bcol[t]) * 4u));
      R.a[u] = __builtin_bit_cast(
          f16x8, __builtin_amdgcn_raw_buffer_load_b128(ars, aoff + (uint32_t)kp * 16u, 0, 0));
    }
  };
  auto math = [&](int r, StripRound<NS, SPW, NF>& R) {
    const int slb = sl0 + r * slstride;
    if (slb + SPW > nsl) {
#pragma unroll
      for (int u = 0; u < SPW; ++u)
        if (slb + u >= nsl) R.a[u] = f16x8{0, 0, 0, 0, 0, 0, 0, 0};
    }
#pragma unroll
    for (int f = 0; f < NF; ++f) {
      // INT4: weights decode to 1024 + q (u4_magic_word); asum (every row)
      // is the activation row's sum over the group.
      f32x4 grp[NS], asum;
#pragma unroll
      for (int u = f * FL; u < (f + 1) * FL; ++u) {
        f16x8 au = R.a[u];
        if constexpr (INT4) {
          asum = __builtin_amdgcn_mfma_f32_16x16x32_f16(
              f16x8_ones(), au, u == f * FL ? f32x4{0, 0, 0, 0} : asum, 0, 0, 0);
          au = a_k4_order(au);
        }
#pragma unroll
        for (int t = 0; t < NS; ++t) {
          const f16x8 b = INT4 ? u4_magic_word(R.w[u][t]) : raw_fp4_word(R.w[u][t]);
          grp[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
              b, au, u == f * FL ? f32x4{0, 0, 0, 0} : grp[t], 0, 0, 0);
        }
      }
#pragma unroll
      for (int t = 0; t < NS; ++t)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
          float v = grp[t][rr];
          if constexpr (INT4) v -= (1024.0f + (float)clamp_zero(R.z[f][t][rr])) * asum[rr];
          acc[t][rr] += (float)sanitize_scale(R.s[f][t][rr]) * v;
        }
    }
  };
  // Rounds whose first slab is past the end are skipped (wave-uniform).
  int nr = 0;
  while (nr < nrounds && sl0 + nr * slstride < nsl) ++nr;
  if (nr == 0) return;
  StripRound<NS, SPW, NF> R0, R1;
  load(0, R0);
  for (int r = 0; r < nr; r += 2) {
    if (r + 1 < nr) load(r + 1, R1);
    math(r, R0);
    if (r + 1 >= nr) break;
    if (r + 2 < nr) load(r + 2, R0);
    math(r + 1, R1);
  }
}

// Every wave but wave 0 parks its accumulators in LDS, one barrier, then
// wave 0 adds them in wave order (deterministic).  Only lanes of rows < M
// (row = lane & 15) move data.
template <int NS, int NW>
MM_DEV void strip_block_reduce(float* red, f32x4 (&acc)[NS], int M) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const bool live = (lane & 15) < M;
  if (wave > 0 && live) {
#pragma unroll
    for (int t = 0; t < NS; ++t)
      *(f32x4*)(red + (((size_t)(wave - 1) * NS + t) * 64 + lane) * 4) = acc[t];
  }
  __syncthreads();
  if (wave == 0 && live) {
#pragma unroll
    for (int w = 0; w < NW - 1; ++w)
#pragma unroll
      for (int t = 0; t < NS; ++t)
        acc[t] += *(const f32x4*)(red + (((size_t)w * NS + t) * 64 + lane) * 4);
  }
}

// Block -> strip index keeping neighbouring strips on one XCD (blocks are
// dealt round-robin to the 8 XCDs, each with its own L2), so both 64-byte
// halves of a 128-byte line are fetched into the same L2.
MM_DEV int xcd_strip(int bid, int nblk) {
  if (nblk % 8 != 0) return bid;
  return (bid % 8) * (nblk / 8) + bid / 8;
}

// Steps per scale flush for a group size: g/32 capped at SPW when g is a
// multiple of 32 and g/32 is a power of two or a multiple of SPW; else 0.
inline int flush_steps(int g, int spw) {
  if (g % 32 != 0) return 0;
  const int gs = g / 32;
  if (gs >= spw) return gs % spw == 0 ? spw : 0;
  return (gs & (gs - 1)) == 0 ? gs : 0;
}

}  // namespace mmsk
