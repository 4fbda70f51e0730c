// Shared device helpers for the gfx950 FP4 (E2M1) / INT4 dequant-GEMM library.
//
// Weight layout everywhere is the reference's "Marlin" layout
// (metal_marlin/kernels_core.py:1830-1937, src/marlin_gemm.metal:938-1006):
//   B      uint32 [K/8, N]   word (kp, n) holds rows k = 8kp+i in bits 4i..4i+3
//   scales fp16   [K/g, N]
//   zeros  fp16   [K/g, N]   (INT4 only)
// The kernels read that layout directly: one lane loads 16 bytes = the words of
// four adjacent columns for one word-row, and each of the four words feeds a
// different MFMA column tile (column c of tile j is matrix column 4c + j).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

typedef _Float16 f16;
typedef f16 f16x2 __attribute__((ext_vector_type(2)));
typedef f16 f16x4 __attribute__((ext_vector_type(4)));
typedef f16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

#define MM_DEV __device__ __forceinline__

// ---------------------------------------------------------------------------
// Scale / zero-point sanitising.  The reference replaces a non-finite
// f32 dequant product by 0 (src/marlin_gemm.metal:130-137); for a finite scale
// the product E2M1*s (or (q-z)*s) is always finite in f32, so the guard only
// fires for a non-finite scale, where every weight of the group becomes 0.
// Zero points are clamped to [-127, 127] (src/marlin_gemm.metal:118-120).
// ---------------------------------------------------------------------------
MM_DEV f16 sanitize_scale(f16 s) {
  return __builtin_isfinite((float)s) ? s : (f16)0.0f;
}
MM_DEV f16 clamp_zero(f16 z) {
  float zf = (float)z;
  zf = zf < -127.0f ? -127.0f : (zf > 127.0f ? 127.0f : zf);
  return (f16)zf;   // exact: the clamp bounds are fp16 values
}

// ---------------------------------------------------------------------------
// FP4 E2M1: one word (8 codes, k = 0..7 LSB first) -> 8 fp16 weights
// fp16_RNE(E2M1[code] * s), as 4 pairs (k0,k1) (k2,k3) (k4,k5) (k6,k7).
// gfx950's packed fp4->f16 convert gives the exact E2M1 value of the two
// nibbles of one byte (scale operand 1.0); the packed fp16 multiply then
// rounds the exact product once to nearest-even, which is the reference's
// fp16_RNE(E2M1 * f32(s)) (the f32 product of two such values is exact).
// ---------------------------------------------------------------------------
template <int B>
MM_DEV f16x2 e2m1_pair_c(uint32_t w) {
  return __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 1.0f, B);
}

MM_DEV f16x8 dq_fp4_word(uint32_t w, f16x2 s2) {
  f16x2 p0 = e2m1_pair_c<0>(w) * s2;
  f16x2 p1 = e2m1_pair_c<1>(w) * s2;
  f16x2 p2 = e2m1_pair_c<2>(w) * s2;
  f16x2 p3 = e2m1_pair_c<3>(w) * s2;
  return f16x8{p0.x, p0.y, p1.x, p1.y, p2.x, p2.y, p3.x, p3.y};
}

// ---------------------------------------------------------------------------
// INT4 asymmetric: w = fp16_RNE(fp16(q - z) * s)  (src/marlin_gemm.metal:
// 1984-2012 with safe_dequant_u4_value :153-156).  q is recovered exactly by
// the magic-bias trick (nibble OR 0x6400 is the fp16 value 1024 + q), q - z
// is one RNE fp16 subtraction, then one RNE fp16 multiply.
// ---------------------------------------------------------------------------
MM_DEV f16x2 u4_pair(uint32_t w, int shift) {
  const uint32_t t = (w >> shift) & 0xFFu;       // nibbles k, k+1 at bits 0..7
  const uint32_t u = ((t | (t << 12)) & 0x000F000Fu) | 0x64006400u;
  return __builtin_bit_cast(f16x2, u);
}

MM_DEV f16x8 dq_u4_word(uint32_t w, f16x2 negz2, f16x2 s2) {
  const f16x2 m1024 = {(f16)-1024.0f, (f16)-1024.0f};
  f16x2 p0 = ((u4_pair(w, 0) + m1024) + negz2) * s2;
  f16x2 p1 = ((u4_pair(w, 8) + m1024) + negz2) * s2;
  f16x2 p2 = ((u4_pair(w, 16) + m1024) + negz2) * s2;
  f16x2 p3 = ((u4_pair(w, 24) + m1024) + negz2) * s2;
  return f16x8{p0.x, p0.y, p1.x, p1.y, p2.x, p2.y, p3.x, p3.y};
}

// ---------------------------------------------------------------------------
// Error reporting shared by every C entry point.
// ---------------------------------------------------------------------------
void mm_set_error(const char* fmt, ...);

#define MM_CHECK_ARG(cond, ...)      \
  do {                               \
    if (!(cond)) {                   \
      mm_set_error(__VA_ARGS__);     \
      return 1;                      \
    }                                \
  } while (0)

#define MM_CHECK_LAUNCH(what)                                             \
  do {                                                                    \
    hipError_t e__ = hipGetLastError();                                   \
    if (e__ != hipSuccess) {                                              \
      mm_set_error("%s: launch failed: %s", what, hipGetErrorString(e__)); \
      return 2;                                                           \
    }                                                                     \
  } while (0)

__host__ __device__ static inline int mm_cdiv(int a, int b) { return (a + b - 1) / b; }

// ---------------------------------------------------------------------------
// 16-byte accesses coherent across the XCDs' L2s (the cache policy the
// compiler gives agent-scope atomic loads and stores on gfx950: sc1), for the
// split-K partial sums: a raw buffer resource over the partial-sum array, so a
// lane moves 4 floats per instruction instead of 4 scalar atomics.
// ---------------------------------------------------------------------------
MM_DEV __amdgpu_buffer_rsrc_t mm_rsrc(const void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, 0x7fffffff,
                                           0x00020000);
}
constexpr int MM_CPOL_SC1 = 16;
// A buffer offset past mm_rsrc's range (0x7fffffff bytes): loads return zero
// and fetch nothing (offsets added to it stay below 2^32).
constexpr uint32_t MM_DEAD_OFFSET = 0x80000000u;
MM_DEV f32x4 load_agent_x4(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
  return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0,
                                                                         MM_CPOL_SC1));
}
MM_DEV void store_agent_x4(__amdgpu_buffer_rsrc_t r, uint32_t byte_off, f32x4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, byte_off, 0,
                                         MM_CPOL_SC1);
}
