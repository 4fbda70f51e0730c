// Bulk dequantizers and weight quantizers (FP4 E2M1 and asymmetric INT4),
// plus the library's error-string plumbing.
//
// Compiled with -ffp-contract=off: the quantizers must reproduce the
// reference's numpy float32 arithmetic operation by operation.
#include <stdarg.h>
#include <stdio.h>

#include "mm_common.h"

static thread_local char g_err[512] = "";

void mm_set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

extern "C" const char* mm_last_error(void) { return g_err; }

// ---------------------------------------------------------------------------
// Bulk dequant [K/8, N] -> [K, N] fp16, one thread per packed word.
// kernels_core.py:747-791 (inline dequant_fp4: grid (N, K/8), 8 rows per
// thread); bit-exact with src/marlin_gemm.metal:130-185.
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256)
k_fp4_dequant(const uint32_t* __restrict__ B, const f16* __restrict__ S,
              f16* __restrict__ W, int K, int N, int g) {
  const int n = blockIdx.x * 256 + threadIdx.x;
  const int kp = blockIdx.y;
  if (n >= N) return;
  const uint32_t w = B[(size_t)kp * N + n];
  const f16 s = S[(size_t)((kp * 8) / g) * N + n];
  f16* out = W + (size_t)kp * 8 * N + n;
  if (!__builtin_isfinite((float)s)) {          // reference guard -> +0.0
#pragma unroll
    for (int i = 0; i < 8; ++i) out[(size_t)i * N] = (f16)0.0f;
    return;
  }
  const f16x8 v = dq_fp4_word(w, f16x2{s, s});
#pragma unroll
  for (int i = 0; i < 8; ++i) out[(size_t)i * N] = v[i];
}

__global__ void __launch_bounds__(256)
k_u4_dequant(const uint32_t* __restrict__ B, const f16* __restrict__ S,
             const f16* __restrict__ Z, f16* __restrict__ W, int K, int N, int g) {
  const int n = blockIdx.x * 256 + threadIdx.x;
  const int kp = blockIdx.y;
  if (n >= N) return;
  const uint32_t w = B[(size_t)kp * N + n];
  const size_t gi = (size_t)((kp * 8) / g) * N + n;
  const f16 s = S[gi];
  const f16 nz = -clamp_zero(Z[gi]);
  f16* out = W + (size_t)kp * 8 * N + n;
  if (!__builtin_isfinite((float)s)) {
#pragma unroll
    for (int i = 0; i < 8; ++i) out[(size_t)i * N] = (f16)0.0f;
    return;
  }
  const f16x8 v = dq_u4_word(w, f16x2{nz, nz}, f16x2{s, s});
#pragma unroll
  for (int i = 0; i < 8; ++i) out[(size_t)i * N] = v[i];
}

// ---------------------------------------------------------------------------
// FP4 quantizer, Marlin layout: metal_marlin/quantize_fp4.py:131-284 with
// quantize_to_fp4 :64-107.  One thread per (group, output column n); the input
// is W [N, K] (out_features, in_features), fp16 or fp32.
// ---------------------------------------------------------------------------
MM_DEV uint32_t e2m1_nearest(float v) {
  const float T[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};
  // NaN: np.clip keeps it and argmin over all-NaN distances picks index 0 of
  // the negative table (NaN >= 0 is false): code 8.
  if (v != v) return 8u;
  const bool neg = !(v >= 0.0f);
  // np.clip(v, lo, hi) == minimum(maximum(v, lo), hi)
  const float c = neg ? fminf(fmaxf(v, -6.0f), 0.0f) : fminf(fmaxf(v, 0.0f), 6.0f);
  uint32_t best = 0;
  float bd = fabsf(neg ? c + T[0] : c - T[0]);
#pragma unroll
  for (int i = 1; i < 8; ++i) {
    const float d = fabsf(neg ? c + T[i] : c - T[i]);
    if (d < bd) {   // strict: ties keep the lower index, like argmin
      bd = d;
      best = i;
    }
  }
  return best + (neg ? 8u : 0u);
}

template <typename T>
MM_DEV float ld_f32(const T* p) { return (float)*p; }

template <typename T>
__global__ void __launch_bounds__(256)
k_fp4_quantize(const T* __restrict__ Wt, int N, int K, int g,
               uint32_t* __restrict__ B, f16* __restrict__ S) {
  const int n = blockIdx.x * 256 + threadIdx.x;
  const int gi = blockIdx.y;
  if (n >= N) return;
  const T* row = Wt + (size_t)n * K + (size_t)gi * g;
  // np.max and np.maximum propagate NaN (fmaxf would drop it).
  float amax = 0.0f;
  bool nan = false;
  for (int k = 0; k < g; ++k) {
    const float a = fabsf(ld_f32(row + k));
    nan |= a != a;
    amax = fmaxf(amax, a);
  }
  amax = nan ? __builtin_nanf("") : fmaxf(amax, 1e-7f);
  S[(size_t)gi * N + n] = (f16)(amax / 6.0f);
  const int wpg = g / 8;
  for (int w8 = 0; w8 < wpg; ++w8) {
    uint32_t word = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float v = ld_f32(row + 8 * w8 + i) / amax * 6.0f;
      word |= e2m1_nearest(v) << (4 * i);
    }
    B[((size_t)gi * wpg + w8) * N + n] = word;
  }
}

// ---------------------------------------------------------------------------
// Calibration-aware FP4 quantizer: the activation_ranges branch of
// quantize_fp4.py:205-256, in numpy's own arithmetic (the host derives the
// constants the way numpy does):
//   group max   np.percentile(|w|, p) ('linear': order statistics kprev and
//               knext of the group's |w|, numpy's _lerp in float32 with
//               weight gamma) when use_pct, else the absmax; a NaN in the
//               group gives NaN (numpy sorts NaN last and flags the slice);
//               then max(., f32(1e-7))
//   mode 0      group max as is (no input range)
//   mode 1      act > 1: f32(c1 * gmax) + f32(c2 * gmax), c1 = f32(1 - sf),
//               c2 = f32(sf)
//   mode 2      act <= 1: the calibrated max gmax * sqrt(act) is a float64
//               product, so the blend f32(c1 * gmax) + sf * (gmax * att) and
//               the scale's division by 6 run in float64, and the scale is the
//               float64 quotient rounded once to fp16
//   codes       nearest E2M1 of w / f32(group max) * 6, as the weight-only path
// ---------------------------------------------------------------------------
struct FqCal {
  int use_pct, kprev, knext;
  float gamma;
  int mode;
  float c1, c2;
  double sf, att;
};

// k-th smallest (0-based) of |row[0..g)| by rank counting (offline, g^2).
template <typename T>
MM_DEV float kth_abs(const T* row, int g, int k) {
  for (int i = 0; i < g; ++i) {
    const float v = fabsf(ld_f32(row + i));
    int less = 0, eq = 0;
    for (int j = 0; j < g; ++j) {
      const float a = fabsf(ld_f32(row + j));
      less += a < v;
      eq += a == v;
    }
    if (less <= k && k < less + eq) return v;
  }
  return __builtin_nanf("");
}

// fp16 of a float64 value, rounded once: round to float with the sticky bit
// kept in the last place (round-to-odd), then float -> fp16 to nearest even.
// Round-to-odd to 24 bits followed by a rounding to 11 bits is the correctly
// rounded result (the intermediate has more than 2 extra bits).
MM_DEV f16 f16_from_f64(double d) {
  float f = (float)d;
  if ((double)f != d && f == f) {
    uint32_t b = __builtin_bit_cast(uint32_t, f);
    if (fabs((double)f) > fabs(d)) b -= 1;     // back toward zero (truncation)
    f = __builtin_bit_cast(float, b | 1u);
  }
  return (f16)f;
}

template <typename T>
__global__ void __launch_bounds__(256)
k_fp4_quantize_cal(const T* __restrict__ Wt, int N, int K, int g, FqCal cal,
                   uint32_t* __restrict__ B, f16* __restrict__ S) {
  const int n = blockIdx.x * 256 + threadIdx.x;
  const int gi = blockIdx.y;
  if (n >= N) return;
  const T* row = Wt + (size_t)n * K + (size_t)gi * g;
  float amax = 0.0f;
  bool nan = false;
  for (int k = 0; k < g; ++k) {
    const float a = fabsf(ld_f32(row + k));
    nan |= a != a;
    amax = fmaxf(amax, a);
  }
  float gmw = amax;
  if (nan) {
    gmw = __builtin_nanf("");
  } else if (cal.use_pct) {
    const float a = kth_abs(row, g, cal.kprev);
    const float b = cal.knext == cal.kprev ? a : kth_abs(row, g, cal.knext);
    const float diff = b - a;
    gmw = cal.gamma >= 0.5f ? b - diff * (1.0f - cal.gamma) : a + diff * cal.gamma;
  }
  gmw = gmw != gmw ? gmw : fmaxf(gmw, 1e-7f);    // np.maximum propagates NaN
  float gmf;
  f16 scale;
  if (cal.mode == 2) {
    const double gm = (double)(cal.c1 * gmw) + cal.sf * ((double)gmw * cal.att);
    scale = f16_from_f64(gm / 6.0);
    gmf = (float)gm;
  } else {
    gmf = cal.mode == 1 ? cal.c1 * gmw + cal.c2 * gmw : gmw;
    scale = (f16)(gmf / 6.0f);
  }
  S[(size_t)gi * N + n] = scale;
  const int wpg = g / 8;
  for (int w8 = 0; w8 < wpg; ++w8) {
    uint32_t word = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float v = ld_f32(row + 8 * w8 + i) / gmf * 6.0f;
      word |= e2m1_nearest(v) << (4 * i);
    }
    B[((size_t)gi * wpg + w8) * N + n] = word;
  }
}

// ---------------------------------------------------------------------------
// Asymmetric INT4 quantizer, Marlin layout: metal_marlin.py:184-280
// (pack_u4_weights).  Input W [N, K] fp16.
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256)
k_u4_quantize(const f16* __restrict__ Wt, int N, int K, int g,
              uint32_t* __restrict__ B, f16* __restrict__ S, f16* __restrict__ Z) {
  const int n = blockIdx.x * 256 + threadIdx.x;
  const int gi = blockIdx.y;
  if (n >= N) return;
  const f16* row = Wt + (size_t)n * K + (size_t)gi * g;
  float mn = (float)row[0], mx = (float)row[0];
  for (int k = 1; k < g; ++k) {
    const float v = (float)row[k];
    mn = fminf(mn, v);
    mx = fmaxf(mx, v);
  }
  const float s = fmaxf((mx - mn) / 15.0f, 1e-7f);
  const float z = rintf(-mn / s);
  S[(size_t)gi * N + n] = (f16)s;
  Z[(size_t)gi * N + n] = (f16)z;
  const int wpg = g / 8;
  for (int w8 = 0; w8 < wpg; ++w8) {
    uint32_t word = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      float q = rintf((float)row[8 * w8 + i] / s + z);
      q = fminf(fmaxf(q, 0.0f), 15.0f);
      word |= (uint32_t)q << (4 * i);
    }
    B[((size_t)gi * wpg + w8) * N + n] = word;
  }
}

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------
static int check_dims(const char* who, int K, int N, int g) {
  MM_CHECK_ARG(K > 0 && N > 0, "%s: K=%d and N=%d must be positive", who, K, N);
  MM_CHECK_ARG(K % 8 == 0, "%s: K=%d must be divisible by 8", who, K);
  MM_CHECK_ARG(g > 0 && g % 8 == 0, "%s: group_size=%d must be a positive multiple of 8", who, g);
  MM_CHECK_ARG(K % g == 0, "%s: K=%d must be divisible by group_size=%d", who, K, g);
  return 0;
}

extern "C" int mm_fp4_dequant(const uint32_t* B, const uint16_t* S, uint16_t* W, int K, int N,
                              int g, void* stream) {
  if (int rc = check_dims("mm_fp4_dequant", K, N, g)) return rc;
  dim3 grid(mm_cdiv(N, 256), K / 8);
  hipLaunchKernelGGL(k_fp4_dequant, grid, dim3(256), 0, (hipStream_t)stream, B,
                     (const f16*)S, (f16*)W, K, N, g);
  MM_CHECK_LAUNCH("mm_fp4_dequant");
  return 0;
}

extern "C" int mm_u4_dequant(const uint32_t* B, const uint16_t* S, const uint16_t* Z, uint16_t* W,
                             int K, int N, int g, void* stream) {
  if (int rc = check_dims("mm_u4_dequant", K, N, g)) return rc;
  dim3 grid(mm_cdiv(N, 256), K / 8);
  hipLaunchKernelGGL(k_u4_dequant, grid, dim3(256), 0, (hipStream_t)stream, B, (const f16*)S,
                     (const f16*)Z, (f16*)W, K, N, g);
  MM_CHECK_LAUNCH("mm_u4_dequant");
  return 0;
}

extern "C" int mm_fp4_quantize(const void* W, int w_is_f32, int N, int K, int g, uint32_t* B,
                               uint16_t* S, void* stream) {
  if (int rc = check_dims("mm_fp4_quantize", K, N, g)) return rc;
  dim3 grid(mm_cdiv(N, 256), K / g);
  if (w_is_f32)
    hipLaunchKernelGGL(k_fp4_quantize<float>, grid, dim3(256), 0, (hipStream_t)stream,
                       (const float*)W, N, K, g, B, (f16*)S);
  else
    hipLaunchKernelGGL(k_fp4_quantize<f16>, grid, dim3(256), 0, (hipStream_t)stream,
                       (const f16*)W, N, K, g, B, (f16*)S);
  MM_CHECK_LAUNCH("mm_fp4_quantize");
  return 0;
}

extern "C" int mm_fp4_quantize_calibrated(const void* W, int w_is_f32, int N, int K, int g,
                                          int use_pct, int kprev, int knext, float gamma,
                                          int mode, float c1, float c2, double sf, double att,
                                          uint32_t* B, uint16_t* S, void* stream) {
  if (int rc = check_dims("mm_fp4_quantize_calibrated", K, N, g)) return rc;
  MM_CHECK_ARG(!use_pct || (kprev >= 0 && kprev < g && knext >= kprev && knext < g),
               "mm_fp4_quantize_calibrated: order statistics %d, %d outside a group of %d",
               kprev, knext, g);
  MM_CHECK_ARG(mode >= 0 && mode <= 2, "mm_fp4_quantize_calibrated: mode must be 0, 1 or 2");
  const FqCal cal{use_pct != 0, kprev, knext, gamma, mode, c1, c2, sf, att};
  dim3 grid(mm_cdiv(N, 256), K / g);
  if (w_is_f32)
    hipLaunchKernelGGL(k_fp4_quantize_cal<float>, grid, dim3(256), 0, (hipStream_t)stream,
                       (const float*)W, N, K, g, cal, B, (f16*)S);
  else
    hipLaunchKernelGGL(k_fp4_quantize_cal<f16>, grid, dim3(256), 0, (hipStream_t)stream,
                       (const f16*)W, N, K, g, cal, B, (f16*)S);
  MM_CHECK_LAUNCH("mm_fp4_quantize_calibrated");
  return 0;
}

extern "C" int mm_u4_quantize(const uint16_t* W, int N, int K, int g, uint32_t* B, uint16_t* S,
                              uint16_t* Z, void* stream) {
  if (int rc = check_dims("mm_u4_quantize", K, N, g)) return rc;
  dim3 grid(mm_cdiv(N, 256), K / g);
  hipLaunchKernelGGL(k_u4_quantize, grid, dim3(256), 0, (hipStream_t)stream, (const f16*)W, N,
                     K, g, B, (f16*)S, (f16*)Z);
  MM_CHECK_LAUNCH("mm_u4_quantize");
  return 0;
}
