// Measurement aid (no counterpart in the reference): a read-only stream over
// a device buffer, used to measure the HBM read rate this GPU reaches for a
// given byte count in back-to-back launches -- the practical ceiling for a
// weight-streaming GEMM of the same size (launch, ramp-up and drain included).
//
// Each block reads one contiguous slice with 16-byte non-temporal loads, four
// in flight per lane, and folds the words into one value that is stored only
// if it equals a sentinel (so the loads are kept but nothing is written).
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

}  // namespace

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
