// Skinny (decode-shaped) MFMA core shared by the dense and grouped GEMMs.
// Weights stream HBM -> registers -> MFMA 16x16x32 with no LDS staging; the
// M rows ride in the 16-row MFMA operand (zero padded).
#pragma once
#include "mm_common.h"

namespace mmsk {

constexpr int SK_COLS = 64;   // columns covered by one 16x16 MFMA "virtual tile" quad

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

// One wave's contribution: `nst` steps of 32 k (4 word rows) starting at
// step `st0`, stepping by `ststride`, over NT column tiles of 64 columns
// (tile t starts at column n0 + t*coloff) and MT 16-row groups.
//   lane = 16*q + c: B word row 4*st + q, columns n + 4c .. n + 4c + 3,
//   A row 16*mt + c, k = 8*(4*st + q) .. +8 (the MFMA 16x16x32 operand layout).
template <bool INT4, int MT, int NT, int SPW>
MM_DEV void skinny_wave(const f16* __restrict__ A, int lda, const int* __restrict__ rowmap,
                        int rowdiv, int M, const uint32_t* __restrict__ B,
                        const f16* __restrict__ S, const f16* __restrict__ Z, int N, int K, int g,
                        int n0, int coloff, int st0, int nrounds, int ststride,
                        f32x4 (&acc)[MT][NT][4]) {
  const int lane = threadIdx.x & 63;
  const int c = lane & 15, q = lane >> 4;
  const int KP = K >> 3;

  // A row pointers are fixed for the whole K loop.
  const f16* arow[MT];
  bool mok[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = mt * 16 + c;
    mok[mt] = m < M;
    int r = m;
    if (rowmap != nullptr && mok[mt]) r = rowmap[m] / rowdiv;
    arow[mt] = A + (size_t)(mok[mt] ? r : 0) * lda;
  }
  int ncol[NT];
  bool nok[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    ncol[t] = n0 + t * coloff + 4 * c;
    nok[t] = ncol[t] < N;
  }

  for (int r = 0; r < nrounds; ++r) {
    u32x4 w[SPW][NT];
    f16x4 s[SPW][NT];
    f16x4 z[SPW][NT];
    f16x8 a[SPW][MT];
    // Issue every load of the round before any math.
#pragma unroll
    for (int i = 0; i < SPW; ++i) {
      const int st = st0 + r * ststride + i;
      const int kp = 4 * st + q;
      const bool kok = kp < KP;
      const int gi = kok ? (kp * 8) / g : 0;
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const bool ok = kok && nok[t];
        w[i][t] = ok ? *(const u32x4*)(B + (size_t)kp * N + ncol[t]) : u32x4{0, 0, 0, 0};
        s[i][t] = ok ? *(const f16x4*)(S + (size_t)gi * N + ncol[t]) : f16x4{0, 0, 0, 0};
        if constexpr (INT4)
          z[i][t] = ok ? *(const f16x4*)(Z + (size_t)gi * N + ncol[t]) : f16x4{0, 0, 0, 0};
      }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
        a[i][mt] = (kok && mok[mt]) ? *(const f16x8*)(arow[mt] + (size_t)kp * 8)
                                    : f16x8{0, 0, 0, 0, 0, 0, 0, 0};
    }
#pragma unroll
    for (int i = 0; i < SPW; ++i) {
#pragma unroll
      for (int t = 0; t < NT; ++t) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          f16 nz = 0;
          if constexpr (INT4) nz = -clamp_zero(z[i][t][j]);
          const f16x8 b = WordDq<INT4>::run(w[i][t][j], sanitize_scale(s[i][t][j]), nz);
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
            acc[mt][t][j] =
                __builtin_amdgcn_mfma_f32_16x16x32_f16(a[i][mt], b, acc[mt][t][j], 0, 0, 0);
        }
      }
    }
  }
}

// Tree-reduce the NW waves' accumulators through LDS (NW/2 tile buffers);
// on return wave 0 holds the block sum.  NW must be a power of two.
template <int MT, int NT, int NW>
MM_DEV void skinny_block_reduce(float* red, f32x4 (&acc)[MT][NT][4]) {
  constexpr int TILE = MT * NT * 16 * 64;   // floats per wave: 16 per lane per (mt, t)
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int half = NW / 2; half >= 1; half /= 2) {
    if (wave >= half && wave < 2 * half) {
      float* dst = red + (size_t)(wave - half) * TILE;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
          for (int j = 0; j < 4; ++j)
            *(f32x4*)(dst + (((mt * NT + t) * 4 + j) * 64 + lane) * 4) = acc[mt][t][j];
    }
    __syncthreads();
    if (wave < half) {
      const float* src = red + (size_t)wave * TILE;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
          for (int j = 0; j < 4; ++j)
            acc[mt][t][j] += *(const f32x4*)(src + (((mt * NT + t) * 4 + j) * 64 + lane) * 4);
    }
    __syncthreads();
  }
}

}  // namespace mmsk
