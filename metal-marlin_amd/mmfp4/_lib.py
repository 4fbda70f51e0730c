"""ctypes binding of libmmfp4.so (the gfx950 HIP kernels behind a C ABI).

There is no CPU or PyTorch fallback: if the library is missing, or a tensor is
not on a ROCm device, the call raises.  All launches are asynchronous on the
current torch stream of the tensors' device.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "libmmfp4.so"

_c_int, _c_size, _vp = ctypes.c_int, ctypes.c_size_t, ctypes.c_void_p

# name -> (restype, argtypes); must match include/mmfp4.h
SIGNATURES: dict[str, tuple] = {
    "mm_last_error": (ctypes.c_char_p, []),
    "mm_fp4_dequant": (_c_int, [_vp, _vp, _vp, _c_int, _c_int, _c_int, _vp]),
    "mm_u4_dequant": (_c_int, [_vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _vp]),
    "mm_fp4_quantize": (_c_int, [_vp, _c_int, _c_int, _c_int, _c_int, _vp, _vp, _vp]),
    "mm_u4_quantize": (_c_int, [_vp, _c_int, _c_int, _c_int, _vp, _vp, _vp, _vp]),
    "mm_gemm_workspace_bytes": (_c_size, [_c_int, _c_int, _c_int]),
    "mm_fp4_gemm": (_c_int, [_vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _c_int, _vp, _c_size,
                             _vp]),
    "mm_fp4_gemm_noalloc": (_c_int, [_vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _c_int, _vp]),
    "mm_fp4_gemm_rowpacked": (_c_int, [_vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _c_int,
                                       _c_int, _vp, _c_size, _vp]),
    "mm_fp4_gemm_mmfp4": (_c_int, [_vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _c_int, _vp,
                                   _c_size, _vp]),
    "mm_fp4_gate_up_rowpacked": (_c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _c_int, _c_int, _c_int,
                                          _c_int, _c_int, _vp, _c_size, _vp]),
    "mm_u4_gemm": (_c_int, [_vp, _vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _c_int, _vp,
                            _c_size, _vp]),
    "mm_fp4_gate_up": (_c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _c_int,
                                _c_int, _vp, _c_size, _vp]),
    "mm_fp4_gemm_multi": (_c_int, [_vp, _c_int, _vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _vp,
                                   _c_size, _vp]),
    "mm_moe_sort": (_c_int, [_vp, _c_int, _c_int, _c_int, _vp, _vp, _vp, _vp]),
    "mm_moe_sort_i64": (_c_int, [_vp, _c_int, _c_int, _c_int, _vp, _vp, _vp, _vp]),
    "mm_moe_router_workspace_bytes": (_c_size, [_c_int, _c_int, _c_int]),
    "mm_moe_router": (_c_int, [_vp, _vp, _vp, _c_int, _c_int, _c_int, _c_int, _c_int, _vp, _vp,
                               _vp, _c_size, _vp]),
    "mm_softmax_topk": (_c_int, [_vp, _c_int, _c_int, _c_int, _c_int, _c_int, _vp, _vp, _vp]),
    "mm_moe_grouped_gemm": (_c_int, [_vp, _vp, _vp, _c_int, _c_int, _c_int, _vp, _vp, _c_int,
                                     _c_int, _c_int, _c_int, _c_int, _vp, _vp]),
    "mm_moe_combine": (_c_int, [_vp, _vp, _vp, _c_int, _c_int, _c_int, _vp, _vp]),
    "mm_moe_mlp_fp4": (_c_int, [_vp, _vp, _c_int, _vp, _c_int, _c_int, _c_int, _c_int, _c_int,
                                _vp, _vp, _vp, _vp, _c_int, _vp, _vp, _vp, _vp, _vp]),
    "mm_moe_mlp_shared_fp4": (_c_int, [_vp, _vp, _c_int, _vp, _c_int, _c_int, _c_int, _c_int,
                                       _c_int, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                       ctypes.c_float, _vp, _c_int, _vp, _vp, _vp, _vp, _vp]),
    "mm_fp4_flat_quantize": (_c_int, [_vp, _c_size, _c_int, _c_int, _vp, _vp, _vp]),
    "mm_fp4_flat_dequantize": (_c_int, [_vp, _vp, _c_size, _c_size, _c_int, _vp, _vp]),
    "mm_fp4_pack_pair": (_c_int, [_vp, _vp, _c_size, _vp, _vp]),
    "mm_stream_read": (_c_int, [_vp, _c_size, _vp, _c_size, _vp]),
    "mm_mfma_ceiling": (_c_int, [_vp, _vp, _c_size, _c_int, _vp, _c_size, _vp]),
}

_lib = None
_lock = threading.Lock()


class MMError(RuntimeError):
    """A libmmfp4 entry point returned a non-zero status."""


def load() -> ctypes.CDLL:
    """Load libmmfp4.so once; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise ImportError(
                    f"{LIB_PATH} is missing: build it with `python metal-marlin_amd/build.py` "
                    "(or __graft_entry__.build()); there is no CPU fallback")
            lib = ctypes.CDLL(str(LIB_PATH))
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
    return _lib


def call(name: str, *args) -> None:
    """Invoke entry point `name`; raise MMError (ValueError for bad arguments)."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != 0:
        msg = lib.mm_last_error().decode(errors="replace")
        if rc == 1:
            raise ValueError(msg)
        raise MMError(msg)


def ptr(t: torch.Tensor | None) -> ctypes.c_void_p:
    return ctypes.c_void_p(0 if t is None else t.data_ptr())


def stream_of(t: torch.Tensor) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def require_device(*tensors: torch.Tensor) -> torch.device:
    """All tensors on one ROCm device; no host tensors (no CPU path exists)."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not isinstance(t, torch.Tensor):
            raise TypeError(f"expected torch.Tensor, got {type(t).__name__}")
        if t.device.type != "cuda":
            raise RuntimeError(
                f"tensor on {t.device}: the FP4/INT4 kernels run on the GPU only "
                "(move inputs to a ROCm device)")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"tensors on different devices: {dev} vs {t.device}")
    return dev


# ---------------------------------------------------------------------------
# Per-(device, stream) workspace.  Its head holds split-K arrival counters that
# the kernels leave at zero, so it is allocated zeroed once and reused.
# ---------------------------------------------------------------------------
_ws: dict[tuple[int, int], torch.Tensor] = {}


def workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    key = (device.index if device.index is not None else torch.cuda.current_device(),
           torch.cuda.current_stream(device).cuda_stream)
    buf = _ws.get(key)
    if buf is None or buf.numel() < nbytes:
        size = max(nbytes, 1 << 20)
        if buf is not None:
            size = max(size, 2 * buf.numel())
        buf = torch.zeros(size, dtype=torch.uint8, device=device)
        _ws[key] = buf
    return buf
