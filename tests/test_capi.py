"""The C-ABI library loads, exports exactly what include/mmfp4.h declares, and
rejects bad arguments before touching the GPU (runs without a GPU)."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest
import torch

from mmfp4 import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "mmfp4.h"


def declared() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(mm_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_all_bound_symbols():
    assert declared() == sorted(_lib.SIGNATURES)


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in declared():
        assert hasattr(lib, name), name


@pytest.mark.parametrize("M,N,K,g,msg", [
    (1, 64, 7, 8, "divisible by 8"),
    (1, 66, 64, 32, "divisible by 4"),
    (1, 64, 64, 12, "group_size"),
    (1, 64, 96, 64, "group_size"),
])
def test_gemm_rejects_bad_shapes(M, N, K, g, msg):
    with pytest.raises(ValueError, match=msg):
        _lib.call("mm_fp4_gemm", None, None, None, None, M, N, K, g, None, 0, None)
    with pytest.raises(ValueError, match=msg):
        _lib.call("mm_u4_gemm", None, None, None, None, None, M, N, K, g, None, 0, None)


def test_misaligned_operands_rejected():
    with pytest.raises(ValueError, match="aligned"):
        _lib.call("mm_fp4_gemm", ctypes.c_void_p(2), ctypes.c_void_p(16), ctypes.c_void_p(16),
                  ctypes.c_void_p(16), 1, 64, 64, 32, None, 0, None)


def test_other_entry_points_validate():
    with pytest.raises(ValueError, match="num_experts"):
        _lib.call("mm_moe_sort", None, 4, 2, 2000, None, None, None, None)
    with pytest.raises(ValueError, match="act"):
        _lib.call("mm_moe_grouped_gemm", None, None, None, 1, 2, 4, None, None, 4, 64, 64, 32, 7,
                  None, None)
    with pytest.raises(ValueError, match="H="):
        _lib.call("mm_moe_combine", None, None, None, 4, 2, 12, None, None)
    with pytest.raises(ValueError, match="group_size"):
        _lib.call("mm_fp4_dequant", None, None, None, 64, 16, 24, None)
    with pytest.raises(ValueError, match="divisible by 8"):
        _lib.call("mm_u4_quantize", None, 16, 12, 4, None, None, None, None)


def test_workspace_size_is_sane():
    lib = _lib.load()
    assert lib.mm_gemm_workspace_bytes(1, 4096, 14336) >= 4 * 4096
    assert lib.mm_gemm_workspace_bytes(2048, 14336, 4096) == 65536


def test_host_tensors_are_refused():
    import mmfp4
    a = torch.zeros(1, 64, dtype=torch.float16)
    b = torch.zeros(8, 64, dtype=torch.int32)
    s = torch.zeros(2, 64, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="GPU only"):
        mmfp4.marlin_gemm_fp4(a, b, s, 32)
    with pytest.raises(RuntimeError, match="GPU only"):
        mmfp4.dequant_fp4(b, s, 64, 64, 32)


def test_new_entry_points_validate():
    with pytest.raises(ValueError, match="group_size"):
        _lib.call("mm_fp4_flat_quantize", None, 16, 0, 0, None, None, None)
    with pytest.raises(ValueError, match="dtype"):
        _lib.call("mm_fp4_flat_quantize", None, 16, 5, 8, None, None, None)
    with pytest.raises(ValueError, match="cover fewer"):
        _lib.call("mm_fp4_flat_dequantize", None, None, 300, 2, 128, None, None)
    with pytest.raises(ValueError, match="scales_layout"):
        _lib.call("mm_fp4_gemm_rowpacked", None, None, None, None, 1, 64, 256, 64, 2, None, 0,
                  None)
    with pytest.raises(ValueError, match="scales_layout 0"):      # M > 32, [N, K/g] scales
        _lib.call("mm_fp4_gemm_rowpacked", None, None, None, None, 33, 64, 256, 64, 1, None, 0,
                  None)
    with pytest.raises(ValueError, match="divisible by 8"):       # M > 32, N % 8 != 0
        _lib.call("mm_fp4_gemm_rowpacked", None, None, None, None, 33, 60, 256, 64, 0, None, 0,
                  None)
    with pytest.raises(ValueError, match="built-in scratch"):
        _lib.call("mm_fp4_gemm_noalloc", None, None, None, None, 256, 4096, 4096, 128, None)
    with pytest.raises(ValueError, match="shared expert"):
        _lib.call("mm_moe_mlp_shared_fp4", None, None, 0, None, 4, 2, 8, 256, 128, None, None,
                  None, None, None, None, None, None, ctypes.c_float(1.0), None, 128, None, None,
                  None, None, None)


def test_measurement_aids_live_outside_the_gemm_abi():
    """bench.py's read-ceiling and MFMA-ceiling probes are exported by the
    bench-only library, not by libmmfp4.so; their argument checks run without
    a GPU."""
    import bench_aids
    lib = _lib.load()
    for name in ("mm_stream_read", "mm_mfma_ceiling"):
        assert not hasattr(lib, name), name
        assert hasattr(bench_aids.load(), name), name
    with pytest.raises(ValueError, match="unroll"):
        bench_aids.call("mm_stream_read", ctypes.c_void_p(256), 4096, ctypes.c_void_p(256),
                        1 << 20, 64, 64, 3, 1, None)
    with pytest.raises(ValueError, match="n_halves"):
        bench_aids.call("mm_mfma_ceiling", ctypes.c_void_p(256), ctypes.c_void_p(256), 12, 1,
                        ctypes.c_void_p(256), 1 << 20, None)


def test_calibrated_quantizer_and_interleaved_int4_validate():
    with pytest.raises(ValueError, match="order statistics"):
        _lib.call("mm_fp4_quantize_calibrated", None, 1, 4, 256, 128, 1, 130, 131,
                  ctypes.c_float(0.5), 0, ctypes.c_float(0.0), ctypes.c_float(1.0),
                  ctypes.c_double(1.0), ctypes.c_double(1.0), None, None, None)
    with pytest.raises(ValueError, match="mode"):
        _lib.call("mm_fp4_quantize_calibrated", None, 1, 4, 256, 128, 0, 0, 0,
                  ctypes.c_float(0.0), 3, ctypes.c_float(0.0), ctypes.c_float(1.0),
                  ctypes.c_double(1.0), ctypes.c_double(1.0), None, None, None)
    with pytest.raises(ValueError, match="SZ"):
        _lib.call("mm_u4_gemm_sz", None, None, None, None, None, None, 1, 64, 64, 32, None, 0,
                  None)
