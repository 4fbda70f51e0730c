// Pipelined prefill main loop for gfx950, shared by the dense GEMM and the
// grouped-expert (MoE) GEMM.
//
// Every operand of a 64-k chunk (A tile, packed B, the scale/zero rows it
// needs) is fetched global -> LDS directly (global_load_lds_dwordx4)
// STAGES-1 chunks ahead, so the load latency hides behind that many chunks of
// MFMA work without staging registers.
//   A stage: BM rows x 64 halves, 16-byte pieces XOR-swizzled by row
//            (piece (r, c8) lives at r*8 + (c8 ^ ((r >> 1) & 7))) so the MFMA
//            operand reads of 32 consecutive rows spread over the banks;
//   B stage: 8 word rows x BN LDS columns of packed words (row-packed
//            weights: 16-byte pieces of a column's 8 words, see below);
//   S stage: up to 8 scale rows x BN fp16 (the groups the chunk touches),
//   Z stage: same for INT4 zero points.
// Every thread issues the same number of loads per chunk (addresses are
// clamped, never skipped), so a vmcnt wait counts chunks exactly.
//
// Where rows and columns come from is the caller's: a source object maps
// tile row r to an A row pointer and LDS column P to a global column.  Two
// column read patterns exist:
//   TM = false: lane l32 of wave wn reads CW adjacent LDS columns
//               wn*32*CW + CW*l32 + j (one vector read) for column tile j;
//   TM = true : it reads wn*32*CW + 32*j + l32 ("tile-major"), so column
//               tile j of a wave is 32 consecutive LDS columns.  The MoE
//               SwiGLU path uses this to put a gate column and its up column
//               in one lane.
#pragma once
#include <type_traits>
#include <utility>

#include "mm_common.h"
#include "mm_skinny.h"

#define MM_PF2_SCHED_DS 3
#define MM_PF2_SCHED_VALU 9
namespace mmpf {
using namespace mmsk;

constexpr int PF2_BK = 64;
constexpr int PF2_STAGES = 3;   // default LDS ring depth: loads run STAGES-1 chunks ahead
// Scale rows staged per chunk: the groups a 64-k chunk can touch (8 for
// g = 8); with g % 64 == 0 a chunk lies in one group and 2 rows suffice.
constexpr int PF2_SROWS = 8;
constexpr int PF2_SROWS_G64 = 2;

// A source whose weights are row-packed (`kRowPacked`, [N, K/8] words: a
// column's 8 words of a 64-k chunk are 32 contiguous bytes) provides brow(P),
// word 0 of the column behind LDS column P, in place of bcol.
template <class S, class = void>
struct is_rowpacked : std::false_type {};
template <class S>
struct is_rowpacked<S, std::void_t<decltype(S::kRowPacked)>>
    : std::integral_constant<bool, S::kRowPacked> {};

template <class F, int... I>
MM_DEV void static_for(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}

typedef __attribute__((address_space(3))) void* lds_ptr_t;

MM_DEV void gl2lds16(const void* src, void* lds_base_uniform) {
  __builtin_amdgcn_global_load_lds(src, (lds_ptr_t)lds_base_uniform, 16, 0, 0);
}

// s_waitcnt with only the vector-memory counter constrained (gfx9 encoding:
// vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt_hi[15:14]).
template <int VM>
MM_DEV void wait_vmcnt() {
  static_assert(VM >= 0 && VM < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((VM & 15) | (7 << 4) | (15 << 8) | ((VM >> 4) << 14));
}

template <bool INT4, int WM, int WN, int RB, int CW, int STAGES = PF2_STAGES,
          int SROWS = PF2_SROWS>
struct Pf2Shape {
  static constexpr int NTHR = WM * WN * 64;
  static constexpr int NWAVE = WM * WN;
  static constexpr int BM = WM * 32 * RB;
  static constexpr int BN = WN * 32 * CW;
  static constexpr int A_PIECES = BM * (PF2_BK / 8);   // 16-byte pieces per stage
  static constexpr int B_PIECES = (PF2_BK / 8) * (BN / 4);
  static constexpr int S_PIECES = SROWS * (BN / 8);
  static_assert(A_PIECES % 64 == 0 && B_PIECES % 64 == 0 && S_PIECES % 64 == 0, "split");
  static constexpr int A_IT = (A_PIECES + NTHR - 1) / NTHR;
  static constexpr int B_IT = (B_PIECES + NTHR - 1) / NTHR;
  static constexpr int S_IT = (S_PIECES + NTHR - 1) / NTHR;
  static constexpr int LOADS_PER_CHUNK = A_IT + B_IT + S_IT * (INT4 ? 2 : 1);
  static constexpr int A_BYTES = A_PIECES * 16, B_BYTES = B_PIECES * 16, S_BYTES = S_PIECES * 16;
  // LDS: [A stages][B stages][S stages][Z stages][dump].  Waves whose piece
  // range lies past a small operand still issue their load (vmcnt must count
  // the same loads in every thread) into the 1 KiB dump area.
  static constexpr int B_OFF = STAGES * A_BYTES;
  static constexpr int S_OFF = B_OFF + STAGES * B_BYTES;
  static constexpr int Z_OFF = S_OFF + STAGES * S_BYTES;
  static constexpr int D_OFF = Z_OFF + (INT4 ? STAGES * S_BYTES : 0);
  static constexpr int LDS_BYTES = D_OFF + 1024;
};

// Runs chunks [c_beg, c_end) of 64 k into acc.  Source object `src`:
//   src.arow(r)      -> const f16*, A row of tile row r (valid even past the
//                       last row: clamp), element 0 = k 0;
//   src.bcol(P, w)   -> const uint32_t*, packed word row 0 of the global
//                       column behind LDS column P, for a piece of w (4 or 8)
//                       consecutive columns starting at P (clamped in range);
//   src.scol(P, w), src.zcol(P, w) -> const f16*, the same for scales / zeros;
//   src.ld           -> row stride of B in words and of S/Z in halves.
// RBL: the wave's row blocks from RBL on hold no valid row; they skip their
// A reads and MFMAs (acc[RBL..RB) stays zero).  A compile-time count, so no
// branch splits the MFMA stream from the interleaved LDS reads and decode;
// callers with a per-wave count switch over it once, outside the loop.  The
// wave still issues its share of the loads and joins every barrier.
// Requires K % 64 == 0.
template <bool INT4, int WM, int WN, int RB, int CW, bool G64, bool TM, int STAGES, int SROWS,
          int RBL = RB, class Src>
MM_DEV void pf2_mainloop(const Src& src, int K, int g, int c_beg, int c_end, char* smem,
                         f32x16 (&acc)[RB][CW]) {
  static_assert(RBL >= 0 && RBL <= RB, "live row blocks");
  static_assert(G64 || SROWS >= PF2_SROWS, "a chunk can touch 8 groups unless g % 64 == 0");
  using Sh = Pf2Shape<INT4, WM, WN, RB, CW, STAGES, SROWS>;
  constexpr int NWAVE = Sh::NWAVE, BN = Sh::BN;
  constexpr int A_IT = Sh::A_IT, B_IT = Sh::B_IT, S_IT = Sh::S_IT;
  constexpr int A_BYTES = Sh::A_BYTES, B_BYTES = Sh::B_BYTES, S_BYTES = Sh::S_BYTES;
  constexpr int B_OFF = Sh::B_OFF, S_OFF = Sh::S_OFF, Z_OFF = Sh::Z_OFF, D_OFF = Sh::D_OFF;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int l32 = lane & 31, h = lane >> 5;
  const int nch = c_end;
  const int ngroups = K / g;
  const int ld = src.ld;

  // Each lane's source address of chunk 0 is computed once; chunk ch adds a
  // uniform offset.
  const f16* a_src[A_IT];
#pragma unroll
  for (int i = 0; i < A_IT; ++i) {
    const int p = min((i * NWAVE + wave) * 64 + lane, Sh::A_PIECES - 1);
    const int r = p >> 3, c8 = p & 7;
    a_src[i] = src.arow(r) + 8 * (c8 ^ ((r >> 1) & 7));
  }
  // Marlin-layout B: piece p is 4 columns of one word row; the stage holds
  // [8 word rows][BN columns].  Row-packed B (ROWP): piece p is 4 words (16
  // bytes) of one column, half hf = words 4hf..4hf+3, at slot 2*q + hf, where
  // q orders the columns as the lanes read them: q = P for the tile-major
  // read (column tile j of a wave is 32 consecutive columns); otherwise, with
  // column P = CW*c + j, q = j*(BN/CW) + c.  A load instruction then reads
  // both halves (32 contiguous bytes) of 32 columns, and the 16 lanes of an
  // LDS read pass read every other piece of a 512-byte span.  Both layouts
  // are loaded global -> LDS directly.
  constexpr bool ROWP = is_rowpacked<Src>::value;
  static_assert(!ROWP || G64, "row-packed B: one group per chunk");
  const uint32_t* b_src[B_IT];
#pragma unroll
  for (int i = 0; i < B_IT; ++i) {
    const int p = min((i * NWAVE + wave) * 64 + lane, Sh::B_PIECES - 1);
    if constexpr (ROWP) {
      const int hf = p % 2, q = p / 2;       // B_PIECES == 2 * BN
      const int P = TM ? q : (q % (BN / CW)) * CW + q / (BN / CW);
      b_src[i] = src.brow(P) + 4 * hf;
    } else {
      b_src[i] = src.bcol(4 * (p % (BN / 4)), 4) + (size_t)(p / (BN / 4)) * ld;
    }
  }
  int s_row[S_IT];
  const f16* s_src[S_IT];
  const f16* z_src[S_IT];
#pragma unroll
  for (int i = 0; i < S_IT; ++i) {
    const int p = min((i * NWAVE + wave) * 64 + lane, Sh::S_PIECES - 1);
    s_row[i] = p / (BN / 8);
    s_src[i] = src.scol(8 * (p % (BN / 8)), 8);
    z_src[i] = INT4 ? src.zcol(8 * (p % (BN / 8)), 8) : nullptr;
  }
  auto issue = [&](int ch, int st) {
    const int k0 = ch * PF2_BK;
#pragma unroll
    for (int i = 0; i < A_IT; ++i) {
      const int wp = i * NWAVE + wave;
      gl2lds16(a_src[i] + k0,
               wp * 64 < Sh::A_PIECES ? smem + st * A_BYTES + wp * 1024 : smem + D_OFF);
    }
#pragma unroll
    for (int i = 0; i < B_IT; ++i) {
      const int wp = i * NWAVE + wave;
      gl2lds16(b_src[i] + (ROWP ? (size_t)(k0 / 8) : (size_t)(k0 / 8) * ld),
               wp * 64 < Sh::B_PIECES ? smem + B_OFF + st * B_BYTES + wp * 1024 : smem + D_OFF);
    }
    const int gi0 = k0 / g;
#pragma unroll
    for (int i = 0; i < S_IT; ++i) {
      const int wp = i * NWAVE + wave;
      const size_t off = (size_t)min(gi0 + s_row[i], ngroups - 1) * ld;
      const bool live = wp * 64 < Sh::S_PIECES;
      gl2lds16(s_src[i] + off, live ? smem + S_OFF + st * S_BYTES + wp * 1024 : smem + D_OFF);
      if constexpr (INT4)
        gl2lds16(z_src[i] + off, live ? smem + Z_OFF + st * S_BYTES + wp * 1024 : smem + D_OFF);
    }
  };

#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int j = 0; j < CW; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[rb][j][v] = 0.0f;

#pragma unroll
  for (int c = 0; c < STAGES - 1; ++c) issue(min(c_beg + c, nch - 1), c);

  // Per-lane LDS byte offsets, fixed for the whole K loop.
  const int colw = TM ? wn * 32 * CW + l32 : wn * 32 * CW + CW * l32;   // column of tile 0
  constexpr int CSTEP = TM ? 32 : 1;                                   // tile j: + j*CSTEP
  const int arow = wm * 32 * RB + l32;               // lane's row in row block 0
  const int hx = h ^ ((arow >> 1) & 7);              // rows of all row blocks share (r>>1)&7
  // MFMA step t covers, in lane half h, the k of word row 2t + h (Marlin
  // B) or 4h + t (ROWP B: a lane's four steps then use the 4 words of one
  // piece); the A piece read is the one holding those 8 k.
  uint32_t a_off[PF2_BK / 16];                       // + st*A_BYTES + rb*32*128
#pragma unroll
  for (int t = 0; t < PF2_BK / 16; ++t)
    a_off[t] = ROWP ? arow * 128 + ((4 * h + t) ^ ((arow >> 1) & 7)) * 16
                    : arow * 128 + ((2 * t) ^ hx) * 16;
  // + st*B_BYTES, and + t*2*BN*4 (Marlin) or + j*BSTEP (ROWP)
  const uint32_t b_off = ROWP ? B_OFF + ((TM ? colw : wn * 32 + l32) * 2 + h) * 16
                              : B_OFF + (h * BN + colw) * 4;
  constexpr int BSTEP = TM ? 32 * 32 : (BN / CW) * 32;
  typedef uint32_t wvec __attribute__((ext_vector_type(CW)));
  typedef f16 svec __attribute__((ext_vector_type(CW)));
  auto read_w = [&](uint32_t off) {
    if constexpr (!TM) {
      return *(const wvec*)(smem + off);
    } else {
      wvec w;
#pragma unroll
      for (int j = 0; j < CW; ++j) w[j] = *(const uint32_t*)(smem + off + j * CSTEP * 4);
      return w;
    }
  };
  auto read_s = [&](uint32_t off) {
    if constexpr (!TM) {
      return *(const svec*)(smem + off);
    } else {
      svec s;
#pragma unroll
      for (int j = 0; j < CW; ++j) s[j] = *(const f16*)(smem + off + j * CSTEP * 2);
      return s;
    }
  };

  auto chunk = [&](int ch, auto stc) {
    constexpr int st = decltype(stc)::value;
    // Chunk ch's loads are complete once at most (STAGES-2) later chunks' loads
    // are outstanding; the barrier then publishes every thread's pieces and
    // guarantees the stage refilled below has been consumed by all waves.
    wait_vmcnt<(STAGES - 2) * Sh::LOADS_PER_CHUNK>();
    __builtin_amdgcn_s_barrier();
    issue(min(ch + STAGES - 1, nch - 1), (st + STAGES - 1) % STAGES);
    if constexpr (RBL == 0) return;   // no live rows: loads and barriers only
    const int k0 = ch * PF2_BK;
    const int gi0 = k0 / g;
    f16x8 af[2][RB];
    wvec wv[2];
    svec sv[2], zv[2];
    // G64: the chunk lies in one group, so its scale (zero) row is read and
    // sanitised once; otherwise each step reads the row of its own group.
    svec sc = {}, nzc = {};
    u32x4 bp[ROWP ? CW : 1];   // ROWP: the lane's piece of each column tile
    if constexpr (ROWP) {
#pragma unroll
      for (int j = 0; j < CW; ++j)
        bp[j] = *(const u32x4*)(smem + b_off + st * B_BYTES + j * BSTEP);
    }
    if constexpr (G64) {
      const svec s0 = read_s(S_OFF + st * S_BYTES + colw * 2);
#pragma unroll
      for (int j = 0; j < CW; ++j) sc[j] = sanitize_scale(s0[j]);
      if constexpr (INT4) {
        const svec z0 = read_s(Z_OFF + st * S_BYTES + colw * 2);
#pragma unroll
        for (int j = 0; j < CW; ++j) nzc[j] = -clamp_zero(z0[j]);
      }
    }
    auto frag = [&](int t, int slot) {
      if constexpr (ROWP) {
#pragma unroll
        for (int j = 0; j < CW; ++j) wv[slot][j] = bp[j][t];
      } else {
        wv[slot] = read_w(b_off + st * B_BYTES + t * 2 * BN * 4);
      }
      if constexpr (!G64) {
        const int sr = (k0 + 16 * t + 8 * h) / g - gi0;
        const uint32_t so = (sr * BN + colw) * 2;
        sv[slot] = read_s(S_OFF + st * S_BYTES + so);
        if constexpr (INT4) zv[slot] = read_s(Z_OFF + st * S_BYTES + so);
      }
#pragma unroll
      for (int rb = 0; rb < RBL; ++rb)
        af[slot][rb] = *(const f16x8*)(smem + a_off[t] + st * A_BYTES + rb * 32 * 128);
    };
    auto decode = [&](int slot, f16x8 (&b)[CW]) {
#pragma unroll
      for (int j = 0; j < CW; ++j) {
        f16 nz = 0, sj;
        if constexpr (G64) {
          sj = sc[j];
          if constexpr (INT4) nz = nzc[j];
        } else {
          sj = sanitize_scale(sv[slot][j]);
          if constexpr (INT4) nz = -clamp_zero(zv[slot][j]);
        }
        b[j] = WordDq<INT4>::run(wv[slot][j], sj, nz);
      }
    };
    // Software pipeline: step t+1's fragments are read and decoded while
    // step t's MFMAs occupy the matrix pipe.
    frag(0, 0);
    f16x8 bq[2][CW];
    decode(0, bq[0]);
#pragma unroll
    for (int t = 0; t < PF2_BK / 16; ++t) {
      const int cur = t & 1;
      if (t + 1 < PF2_BK / 16) frag(t + 1, cur ^ 1);
#pragma unroll
      for (int rb = 0; rb < RBL; ++rb)
#pragma unroll
        for (int j = 0; j < CW; ++j)
          acc[rb][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[cur][rb], bq[cur][j],
                                                              acc[rb][j], 0, 0, 0);
      if (t + 1 < PF2_BK / 16) decode(cur ^ 1, bq[cur ^ 1]);
      // Interleave each MFMA with a share of the next step's LDS reads and
      // decode VALU so the matrix pipe never drains while they issue.  Up to
      // 3 LDS reads and 9 VALU ops after each MFMA (front-loading the next
      // step's operands) measured 2-6% faster than 1 and 3 at M = 512..8192.
#pragma unroll
      for (int i = 0; i < RBL * CW; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
        __builtin_amdgcn_sched_group_barrier(0x100, MM_PF2_SCHED_DS, 0);   // DS read
        __builtin_amdgcn_sched_group_barrier(0x002, MM_PF2_SCHED_VALU, 0);   // VALU
      }
    }
  };
  // The ring position of chunk ch is (ch - c_beg) % STAGES: unroll by STAGES so
  // every LDS offset is a compile-time constant.
  for (int ch = c_beg; ch < nch; ch += STAGES) {
    static_for(
        [&](auto stc) {
          constexpr int st = decltype(stc)::value;
          if (st == 0 || ch + st < nch) chunk(ch + st, stc);
        },
        std::make_integer_sequence<int, STAGES>{});
  }
  wait_vmcnt<0>();
}

// Column map of the tile-major (TM) pair kernels: each wave's 64 LDS columns
// are 32 output columns twice, first from the gate matrix and then the same
// columns from the up matrix.  Output column of LDS column P (o0 = the
// block's first output column), clamped so a w-column piece stays in range.
MM_DEV int pair_out_col(int o0, int P, int w, int nout) {
  return min(o0 + 32 * (P >> 6) + (P & 31), nout - w);
}
MM_DEV bool pair_is_up(int P) { return (P & 32) != 0; }

}  // namespace mmpf
