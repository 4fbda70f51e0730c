// Flat-group FP4 E2M1 quantize / dequantize / nibble-pair packing: the
// `FP4Metal` surface of metal_marlin/fp4_metal.py:71-314.
//
// Unlike the Marlin-layout quantizer (mm_quant.hip), groups run over the
// flattened tensor: group i is elements [i*g, (i+1)*g), the last group padded
// with zeros (fp4_metal.py:150-160).  Per group:
//   scale = max(max|x| / 6, 1e-8)                       (f32, :161-163)
//   v     = x / scale                                   (f32, :166)
//   code  = (v < 0 ? 8 : 0) | argmin_j |E2M1_POS[j] - |v||  (ties -> lower j,
//           :167-172)
// numpy propagates NaN through max, so a group holding a NaN has a NaN scale
// and every code 0 (argmin over all-NaN distances returns 0; NaN < 0 is
// false).  Dequantize is the f32 product E2M1[code] * scale[i / g]
// (fp4_metal.py:192-235, _compat.py:348-374).
//
// Compiled with -ffp-contract=off and correctly rounded f32 division: every
// f32 operation matches numpy's.
//
// Layout: one wave per group (64 lanes stride over the group, consecutive
// lanes on consecutive elements), 4 waves per block.  HBM-bound: 4 B (f32;
// 2 B for fp16/bf16) in and 1 B out per element plus 4 B per group.
#include "mm_common.h"

void mm_set_error(const char* fmt, ...);

#define FF_CHECK(cond, ...)          \
  do {                               \
    if (!(cond)) {                   \
      mm_set_error(__VA_ARGS__);     \
      return 1;                      \
    }                                \
  } while (0)

namespace {

constexpr int FF_WAVES = 4;

template <typename T>
MM_DEV float ff_load(const T* p, size_t i);
template <>
MM_DEV float ff_load<float>(const float* p, size_t i) { return p[i]; }
template <>
MM_DEV float ff_load<f16>(const f16* p, size_t i) { return (float)p[i]; }
template <>
MM_DEV float ff_load<uint16_t>(const uint16_t* p, size_t i) {   // bf16 bits
  return __uint_as_float((uint32_t)p[i] << 16);
}

MM_DEV uint8_t ff_code(float v) {
  const float P[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};
  const float a = fabsf(v);
  uint32_t best = 0;
  float bd = fabsf(P[0] - a);
#pragma unroll
  for (int j = 1; j < 8; ++j) {
    const float d = fabsf(P[j] - a);
    if (d < bd) {      // strict: ties keep the lower index; NaN never wins
      bd = d;
      best = j;
    }
  }
  return (uint8_t)((v < 0.0f ? 8u : 0u) | best);
}

template <typename T>
__global__ void __launch_bounds__(FF_WAVES * 64)
k_flat_quantize(const T* __restrict__ x, size_t n, int g, size_t ngroups,
                uint8_t* __restrict__ codes, float* __restrict__ scales) {
  const int lane = threadIdx.x & 63;
  const size_t grp = (size_t)blockIdx.x * FF_WAVES + (threadIdx.x >> 6);
  if (grp >= ngroups) return;
  const size_t base = grp * (size_t)g;
  const size_t end = base + (size_t)g < n ? base + (size_t)g : n;   // zero padding past n
  float m = 0.0f;
  bool nan = false;
  for (size_t i = base + lane; i < end; i += 64) {
    const float a = fabsf(ff_load(x, i));
    nan |= a != a;
    m = a > m ? a : m;
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
  nan = __any(nan);
  float s = m / 6.0f;
  s = s > 1e-8f ? s : 1e-8f;
  if (nan) s = __builtin_nanf("");
  if (lane == 0) scales[grp] = s;
  for (size_t i = base + lane; i < end; i += 64) codes[i] = ff_code(ff_load(x, i) / s);
}

__global__ void __launch_bounds__(256)
k_flat_dequantize(const uint8_t* __restrict__ codes, const float* __restrict__ scales, size_t n,
                  int g, float* __restrict__ out) {
  const float E[16] = {0.0f,  0.5f,  1.0f,  1.5f,  2.0f,  3.0f,  4.0f,  6.0f,
                       -0.0f, -0.5f, -1.0f, -1.5f, -2.0f, -3.0f, -4.0f, -6.0f};
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256)
    out[i] = E[codes[i] & 15u] * scales[i / (size_t)g];
}

__global__ void __launch_bounds__(256)
k_pack_pair(const uint8_t* __restrict__ lo, const uint8_t* __restrict__ hi, size_t n,
            uint8_t* __restrict__ out) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256)
    out[i] = (uint8_t)((lo[i] & 15u) | ((hi[i] & 15u) << 4));
}

unsigned grid_1d(size_t n) {
  const size_t b = (n + 255) / 256;
  return (unsigned)(b < 65536 ? (b ? b : 1) : 65536);
}

}  // namespace

// dtype: 0 f32, 1 fp16, 2 bf16 (bits).
extern "C" int mm_fp4_flat_quantize(const void* x, size_t n, int dtype, int group_size,
                                    uint8_t* codes, float* scales, void* stream) {
  FF_CHECK(group_size > 0, "mm_fp4_flat_quantize: group_size=%d must be > 0", group_size);
  FF_CHECK(dtype >= 0 && dtype <= 2, "mm_fp4_flat_quantize: dtype=%d must be 0 (f32), 1 (fp16) "
           "or 2 (bf16)", dtype);
  if (n == 0) return 0;
  const size_t ngroups = (n + group_size - 1) / group_size;
  FF_CHECK(ngroups / FF_WAVES < ((size_t)1 << 31), "mm_fp4_flat_quantize: too many groups");
  const dim3 grid((unsigned)((ngroups + FF_WAVES - 1) / FF_WAVES));
  hipStream_t st = (hipStream_t)stream;
  if (dtype == 0)
    hipLaunchKernelGGL(k_flat_quantize<float>, grid, dim3(FF_WAVES * 64), 0, st,
                       (const float*)x, n, group_size, ngroups, codes, scales);
  else if (dtype == 1)
    hipLaunchKernelGGL(k_flat_quantize<f16>, grid, dim3(FF_WAVES * 64), 0, st, (const f16*)x, n,
                       group_size, ngroups, codes, scales);
  else
    hipLaunchKernelGGL(k_flat_quantize<uint16_t>, grid, dim3(FF_WAVES * 64), 0, st,
                       (const uint16_t*)x, n, group_size, ngroups, codes, scales);
  const hipError_t e = hipGetLastError();
  FF_CHECK(e == hipSuccess, "mm_fp4_flat_quantize: launch failed: %s", hipGetErrorString(e));
  return 0;
}

extern "C" int mm_fp4_flat_dequantize(const uint8_t* codes, const float* scales, size_t n,
                                      size_t nscales, int group_size, float* out, void* stream) {
  FF_CHECK(group_size > 0, "mm_fp4_flat_dequantize: group_size=%d must be > 0", group_size);
  FF_CHECK(nscales * (size_t)group_size >= n,
           "mm_fp4_flat_dequantize: %zu scales x group_size %d cover fewer than the %zu codes",
           nscales, group_size, n);
  if (n == 0) return 0;
  hipLaunchKernelGGL(k_flat_dequantize, dim3(grid_1d(n)), dim3(256), 0, (hipStream_t)stream,
                     codes, scales, n, group_size, out);
  const hipError_t e = hipGetLastError();
  FF_CHECK(e == hipSuccess, "mm_fp4_flat_dequantize: launch failed: %s", hipGetErrorString(e));
  return 0;
}

extern "C" int mm_fp4_pack_pair(const uint8_t* lo, const uint8_t* hi, size_t n, uint8_t* out,
                                void* stream) {
  if (n == 0) return 0;
  hipLaunchKernelGGL(k_pack_pair, dim3(grid_1d(n)), dim3(256), 0, (hipStream_t)stream, lo, hi, n,
                     out);
  const hipError_t e = hipGetLastError();
  FF_CHECK(e == hipSuccess, "mm_fp4_pack_pair: launch failed: %s", hipGetErrorString(e));
  return 0;
}
