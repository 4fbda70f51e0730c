/* Measurement aids for bench.py: libmmfp4_bench.so, built beside libmmfp4.so
 * from bench_aids/mm_bench_aids.hip.  Not part of the drop-in ABI (they have
 * no counterpart in the reference); the GEMM library does not export them.
 * Status codes and mm_bench_last_error follow the library's convention:
 * 0 ok, 1 bad argument, 2 launch failure. */
#ifndef MMFP4_BENCH_AIDS_H
#define MMFP4_BENCH_AIDS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

const char* mm_bench_last_error(void);

/* Reads `bytes` (a multiple of 16, 16-byte aligned) of device memory once
 * and writes nothing (sink: a scratch buffer that a sentinel test keeps the
 * loads alive for; it must hold blocks x threads words).  The HBM read rate
 * reachable for that many bytes in back-to-back launches is the practical
 * ceiling of a weight-streaming GEMM of the same size.
 *   blocks, threads  grid (threads a multiple of 64, at most 1024); blocks 0
 *                    picks the default plan (512 x 512 up to 16 MiB, else
 *                    8192 x 256) and ignores threads
 *   unroll           16-byte loads in flight per lane: 1, 2, 4, 8 or 16
 *   mode             bit 0: non-temporal loads; bit 1: grid-stride order
 *                    (all blocks sweep the buffer together) instead of one
 *                    contiguous slice per block */
int mm_stream_read(const void* p, size_t bytes, uint32_t* sink, size_t sink_bytes, int blocks,
                   int threads, int unroll, int mode, void* stream);

/* Runs MFMA 32x32x16 f16 and nothing else on 256 blocks of 8 waves (one block
 * per CU), with operand values taken from a and b (n_halves fp16 each, a
 * multiple of 8, 16-byte aligned); sink receives 256 x 512 floats.  One launch
 * performs 256 * 8 * iters * 32 MFMAs of 32768 flops: the sustained
 * matrix-core rate with a GEMM's own operand values (the rate falls as more
 * operand bits toggle, because the board's power limit lowers the clock). */
int mm_mfma_ceiling(const uint16_t* a, const uint16_t* b, size_t n_halves, int iters, float* sink,
                    size_t sink_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MMFP4_BENCH_AIDS_H */
