"""Decode-path kernel selection with the reference's finer kernel names
(metal_marlin/inference/decode.py:505-537, select_decode_kernel).

The names are the reference's kernel families.  On MI355X every one of them
is served by the same entry point, mm_fp4_gemm, which picks its kernel from
the shape: "decode_gemv_fp4", "_wide", "_tiled" and "_batched" map to the
skinny decode kernels (k_skinny, k_skinny_dual, k_strip), "marlin_gemm_fp4"
to the skinny kernels up to M = 32 and the MFMA tile kernel above.
"""

from __future__ import annotations

__all__ = ["select_decode_kernel"]


def select_decode_kernel(M: int, N: int, K: int) -> str:
    """M > 8: "marlin_gemm_fp4"; 1 < M <= 8: "decode_gemv_fp4_batched";
    M == 1: "decode_gemv_fp4_wide" for N >= 512, else "decode_gemv_fp4_tiled"
    for K > 8192, else "decode_gemv_fp4"."""
    if M > 8:
        return "marlin_gemm_fp4"
    if M > 1:
        return "decode_gemv_fp4_batched"
    if N >= 512:
        return "decode_gemv_fp4_wide"
    if K > 8192:
        return "decode_gemv_fp4_tiled"
    return "decode_gemv_fp4"
