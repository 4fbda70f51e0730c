"""Kernel-selection rules of the reference's two selectors
(kernels_core.py:3833-3852 and inference/decode.py:505-537), checked at the
boundaries its own selection tests use (tests/test_decode_kernel_selection.py):
M = 1 / 2..8 / 9+, N = 512, K = 8192."""

from __future__ import annotations

import pytest


def test_inference_selector_boundaries():
    from mmfp4.decode import select_decode_kernel as sel
    assert sel(1, 256, 4096) == "decode_gemv_fp4"
    for n in (512, 1024, 8192):
        assert sel(1, n, 4096) == "decode_gemv_fp4_wide"
    for k in (8193, 16384, 32768):
        assert sel(1, 256, k) == "decode_gemv_fp4_tiled"
    assert sel(1, 8192, 8192) == "decode_gemv_fp4_wide"
    assert sel(1, 512, 16384) == "decode_gemv_fp4_wide"   # wide wins over tiled
    assert sel(1, 511, 8192) == "decode_gemv_fp4"
    for m in (2, 4, 8):
        assert sel(m, 256, 4096) == "decode_gemv_fp4_batched"
    for m in (9, 16, 128):
        assert sel(m, 256, 4096) == "marlin_gemm_fp4"


@pytest.mark.parametrize("m", [1, 2, 4, 8, 9, 16, 32, 64])
def test_kernels_core_selector(m):
    from mmfp4 import select_decode_kernel as sel
    assert sel(m, 4096, 4096) == ("marlin_gemm_fp4" if m > 8 else "decode_gemv_fp4")
