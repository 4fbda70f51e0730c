// Measurement aids (no counterpart in the reference).
//
// mm_stream_read: a read-only stream over a device buffer, used to measure the
// HBM read rate this GPU reaches for a given byte count in back-to-back
// launches -- the practical ceiling for a weight-streaming GEMM of the same
// size (launch, ramp-up and drain included).  Each block reads one contiguous
// slice with 16-byte non-temporal loads, four in flight per lane, and folds
// the words into one value that is stored only if it equals a sentinel (so the
// loads are kept but nothing is written).
//
// mm_mfma_ceiling: MFMA 32x32x16 f16 with nothing else in the loop, fed with
// caller-given operand values.  The matrix cores' sustained rate depends on
// the operand bits (the board's power limit lowers the clock as more bits
// toggle), so the ceiling of a GEMM is measured with its own operand values.
#include "mm_common.h"

namespace {

template <int U>
__global__ void __launch_bounds__(512)
k_stream_read(const u32x4* __restrict__ p, size_t n16, size_t per_block, uint32_t* sink) {
  const size_t beg = (size_t)blockIdx.x * per_block;
  const size_t end = beg + per_block < n16 ? beg + per_block : n16;
  uint32_t acc = 0;
  for (size_t i = beg + threadIdx.x; i < end; i += (size_t)blockDim.x * U) {
    u32x4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const size_t j = i + (size_t)u * blockDim.x;
      v[u] = j < end ? __builtin_nontemporal_load(p + j) : u32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int u = 0; u < U; ++u) acc ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
  }
  if (acc == 0x9e3779b9u) sink[blockIdx.x * blockDim.x + threadIdx.x] = acc;
}

// One block per CU, 8 waves, each wave the prefill kernel's 4 x 2 tile of
// 32x32 accumulators.  Each lane holds 4 A and 4 B operand vectors taken from
// the buffers and rotates them every step, so consecutive MFMAs see
// different data as a GEMM's do.  Per iteration: 32 MFMAs per wave.
__global__ void __launch_bounds__(512)
k_mfma_ceiling(const f16x8* __restrict__ a, const f16x8* __restrict__ b, size_t n8, int iters,
               float* sink) {
  f16x8 av[4], bv[4];
  const size_t base = ((size_t)blockIdx.x * 512 + threadIdx.x) * 4;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    av[i] = a[(base + i) % n8];
    bv[i] = b[(base + 2 + i) % n8];
  }
  f32x16 acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x16{};
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[(i + u) & 3], bv[(j + 2 * u) & 3],
                                                             acc[i][j], 0, 0, 0);
  }
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) s += acc[i][j][threadIdx.x & 15];
  sink[(size_t)blockIdx.x * 512 + threadIdx.x] = s;
}

}  // namespace

extern "C" int mm_mfma_ceiling(const uint16_t* a, const uint16_t* b, size_t n_halves, int iters,
                               float* sink, size_t sink_bytes, void* stream) {
  MM_CHECK_ARG(a != nullptr && b != nullptr && ((uintptr_t)a & 15) == 0 &&
                   ((uintptr_t)b & 15) == 0 && n_halves >= 8 && n_halves % 8 == 0,
               "mm_mfma_ceiling: operand buffers must be 16-byte aligned, n_halves a positive "
               "multiple of 8");
  MM_CHECK_ARG(iters >= 0, "mm_mfma_ceiling: iters must be >= 0");
  constexpr int blocks = 256;
  MM_CHECK_ARG(sink != nullptr && sink_bytes >= (size_t)blocks * 512 * sizeof(float),
               "mm_mfma_ceiling: sink must hold %d floats", blocks * 512);
  hipLaunchKernelGGL(k_mfma_ceiling, dim3(blocks), dim3(512), 0, (hipStream_t)stream,
                     (const f16x8*)a, (const f16x8*)b, n_halves / 8, iters, sink);
  MM_CHECK_LAUNCH("mm_mfma_ceiling");
  return 0;
}

extern "C" int mm_stream_read(const void* p, size_t bytes, uint32_t* sink, size_t sink_bytes,
                              void* stream) {
  MM_CHECK_ARG(p != nullptr && ((uintptr_t)p & 15) == 0 && bytes % 16 == 0,
               "mm_stream_read: buffer must be 16-byte aligned and a multiple of 16 bytes");
  if (bytes == 0) return 0;
  // Measured on MI355X: 512 blocks of 512 threads are best up to ~16 MiB,
  // many small blocks above that.
  const bool small = bytes <= (16u << 20);
  const int blocks = small ? 512 : 8192, threads = small ? 512 : 256;
  MM_CHECK_ARG(sink != nullptr && sink_bytes >= (size_t)blocks * threads * sizeof(uint32_t),
               "mm_stream_read: sink must hold %d words", blocks * threads);
  const size_t n16 = bytes / 16;
  const size_t per = (n16 + blocks - 1) / blocks;
  hipLaunchKernelGGL(k_stream_read<4>, dim3(blocks), dim3(threads), 0, (hipStream_t)stream,
                     (const u32x4*)p, n16, per, sink);
  MM_CHECK_LAUNCH("mm_stream_read");
  return 0;
}
