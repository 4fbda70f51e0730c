// Measurement aids for bench.py (no counterpart in the reference; built into
// libmmfp4_bench.so, not into the GEMM library).
//
// mm_stream_read: a read-only stream over a device buffer, used to measure the
// HBM read rate this GPU reaches for a given byte count in back-to-back
// launches -- the practical ceiling for a weight-streaming GEMM of the same
// size (launch, ramp-up and drain included).  The grid, the loads in flight
// per lane, the non-temporal hint and the order (one contiguous slice per
// block, or all blocks sweeping the buffer together) are parameters, so the
// ceiling can be swept rather than assumed.  The loaded words are folded into
// one value that is stored only if it equals a sentinel (so the loads are
// kept but nothing is written).
//
// mm_mfma_ceiling: MFMA 32x32x16 f16 with nothing else in the loop, fed with
// caller-given operand values.  The matrix cores' sustained rate depends on
// the operand bits (the board's power limit lowers the clock as more bits
// toggle), so the ceiling of a GEMM is measured with its own operand values.
#include <stdarg.h>
#include <stdio.h>

#include "mm_common.h"

namespace {

namespace err {
thread_local char g_err[512];
}

template <int U, bool NT, bool STRIDE>
__global__ void __launch_bounds__(1024)
k_stream_read(const u32x4* __restrict__ p, size_t n16, size_t per_block, uint32_t* sink) {
  // Contiguous: block b reads [b * per_block, (b + 1) * per_block), lanes
  // stepping by blockDim.  Grid-stride: element i of the sweep is read by
  // thread (i mod (grid threads)), so all blocks move through the buffer
  // together.
  const size_t nthr = STRIDE ? (size_t)gridDim.x * blockDim.x : blockDim.x;
  const size_t beg = STRIDE ? 0 : (size_t)blockIdx.x * per_block;
  const size_t end = STRIDE ? n16 : (beg + per_block < n16 ? beg + per_block : n16);
  const size_t t0 = STRIDE ? (size_t)blockIdx.x * blockDim.x + threadIdx.x : threadIdx.x;
  uint32_t acc = 0;
  for (size_t i = beg + t0; i < end; i += nthr * U) {
    u32x4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const size_t j = i + (size_t)u * nthr;
      if (j < end)
        v[u] = NT ? __builtin_nontemporal_load(p + j) : p[j];
      else
        v[u] = u32x4{0, 0, 0, 0};
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

void mm_set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(err::g_err, sizeof(err::g_err), fmt, ap);
  va_end(ap);
}

extern "C" const char* mm_bench_last_error(void) { return err::g_err; }

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

template <int U>
static void launch_read(bool nt, bool stride, int blocks, int threads, const u32x4* p, size_t n16,
                        size_t per, uint32_t* sink, hipStream_t st) {
  if (nt && stride)
    hipLaunchKernelGGL((k_stream_read<U, true, true>), dim3(blocks), dim3(threads), 0, st, p, n16,
                       per, sink);
  else if (nt)
    hipLaunchKernelGGL((k_stream_read<U, true, false>), dim3(blocks), dim3(threads), 0, st, p,
                       n16, per, sink);
  else if (stride)
    hipLaunchKernelGGL((k_stream_read<U, false, true>), dim3(blocks), dim3(threads), 0, st, p,
                       n16, per, sink);
  else
    hipLaunchKernelGGL((k_stream_read<U, false, false>), dim3(blocks), dim3(threads), 0, st, p,
                       n16, per, sink);
}

extern "C" int mm_stream_read(const void* p, size_t bytes, uint32_t* sink, size_t sink_bytes,
                              int blocks, int threads, int unroll, int mode, void* stream) {
  MM_CHECK_ARG(p != nullptr && ((uintptr_t)p & 15) == 0 && bytes % 16 == 0,
               "mm_stream_read: buffer must be 16-byte aligned and a multiple of 16 bytes");
  if (blocks == 0) {
    // Default plan, measured on MI355X: 512 blocks of 512 threads up to
    // ~16 MiB, many small blocks above that.
    const bool small = bytes <= (16u << 20);
    blocks = small ? 512 : 8192;
    threads = small ? 512 : 256;
  }
  MM_CHECK_ARG(blocks > 0 && threads >= 64 && threads <= 1024 && threads % 64 == 0,
               "mm_stream_read: blocks must be positive and threads a multiple of 64 up to 1024");
  MM_CHECK_ARG(unroll == 1 || unroll == 2 || unroll == 4 || unroll == 8 || unroll == 16,
               "mm_stream_read: unroll must be 1, 2, 4, 8 or 16");
  MM_CHECK_ARG(mode >= 0 && mode <= 3, "mm_stream_read: mode must be 0..3");
  MM_CHECK_ARG(sink != nullptr && sink_bytes >= (size_t)blocks * threads * sizeof(uint32_t),
               "mm_stream_read: sink must hold %d words", blocks * threads);
  if (bytes == 0) return 0;
  const size_t n16 = bytes / 16;
  const size_t per = (n16 + blocks - 1) / blocks;
  const bool nt = mode & 1, stride = mode & 2;
  const hipStream_t st = (hipStream_t)stream;
  const u32x4* q = (const u32x4*)p;
  switch (unroll) {
    case 1: launch_read<1>(nt, stride, blocks, threads, q, n16, per, sink, st); break;
    case 2: launch_read<2>(nt, stride, blocks, threads, q, n16, per, sink, st); break;
    case 4: launch_read<4>(nt, stride, blocks, threads, q, n16, per, sink, st); break;
    case 8: launch_read<8>(nt, stride, blocks, threads, q, n16, per, sink, st); break;
    default: launch_read<16>(nt, stride, blocks, threads, q, n16, per, sink, st); break;
  }
  MM_CHECK_LAUNCH("mm_stream_read");
  return 0;
}
