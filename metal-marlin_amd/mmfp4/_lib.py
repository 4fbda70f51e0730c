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
    "mm_fp4_quantize_calibrated": (_c_int, [_vp, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int,
                                            _c_int, ctypes.c_float, _c_int, ctypes.c_float,
                                            ctypes.c_float, ctypes.c_double, ctypes.c_double,
                                            _vp, _vp, _vp]),
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
    "mm_u4_gemm_sz": (_c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _c_int,
                               _vp, _c_size, _vp]),
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
    "mm_moe_gemm_shared_fp4": (_c_int, [_vp, _vp, _c_int, _vp, _c_int, _c_int, _c_int, _c_int,
                                        _c_int, _vp, _vp, _vp, _vp, _c_int, _vp, _vp, _vp, _vp]),
    "mm_fp4_flat_quantize": (_c_int, [_vp, _c_size, _c_int, _c_int, _vp, _vp, _vp]),
    "mm_fp4_flat_dequantize": (_c_int, [_vp, _vp, _c_size, _c_size, _c_int, _vp, _vp]),
    "mm_fp4_pack_pair": (_c_int, [_vp, _vp, _c_size, _vp, _vp]),
}

_lib = None
_lock = threading.Lock()


class _Bound:
    """The entry points as attributes, bound once at load (no per-call
    getattr on the CDLL)."""


F = _Bound()


class MMError(RuntimeError):
    """A libmmfp4 entry point returned a non-zero status."""


_binding = None


def binding():
    """The per-call torch binding (_mmfp4_torch.so, built next to the library)
    or None when it was not built; both call the same C ABI."""
    global _binding
    if _binding is None:
        load()
        try:
            from . import _mmfp4_torch as b        # links libmmfp4.so from this directory
        except ImportError:
            b = False
        _binding = b
    return _binding or None


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
                setattr(F, name, fn)
            _lib = lib
    return _lib


def check(rc: int) -> None:
    """Raise for a non-zero status: ValueError for a bad argument (1),
    MMError for a launch failure."""
    if rc != 0:
        msg = _lib.mm_last_error().decode(errors="replace")
        if rc == 1:
            raise ValueError(msg)
        raise MMError(msg)


def call(name: str, *args) -> None:
    """Invoke entry point `name`; raise MMError (ValueError for bad arguments)."""
    if _lib is None:
        load()
    check(getattr(F, name)(*args))


def _stamp(t: torch.Tensor) -> tuple:
    return (t._version, t.data_ptr(), tuple(t.shape), t.dtype)


def derived(src: torch.Tensor, key: str, build, also: torch.Tensor | None = None):
    """build(src), cached on the tensor object `src` under `key` and rebuilt
    when src (or `also`, a second input of build) is written in place (its
    version counter) or points at other storage.  The copy lives exactly as
    long as the source tensor object; a caller that passes a fresh view each
    time gets no caching."""
    cache = getattr(src, "_mmfp4_derived", None)
    stamp = _stamp(src) + (_stamp(also) if also is not None else ())
    hit = cache.get(key) if cache is not None else None
    if hit is not None and hit[0] == stamp:
        return hit[1]
    out = build(src)
    if cache is None:
        cache = {}
        try:
            src._mmfp4_derived = cache
        except (AttributeError, RuntimeError):
            return out
    cache[key] = (stamp, out)
    return out


def ptr(t: torch.Tensor | None) -> ctypes.c_void_p:
    return ctypes.c_void_p(0 if t is None else t.data_ptr())


try:                                   # current stream without a Stream object
    _raw_stream = torch._C._cuda_getCurrentRawStream
except AttributeError:                 # pragma: no cover - older torch
    def _raw_stream(index: int) -> int:
        return torch.cuda.current_stream(index).cuda_stream


def raw_stream(device_index: int) -> int:
    """Handle of the current torch stream on a device, as an integer."""
    return _raw_stream(device_index)


def stream_of(t: torch.Tensor) -> ctypes.c_void_p:
    return ctypes.c_void_p(_raw_stream(t.get_device()))


def require_device(*tensors: torch.Tensor) -> torch.device:
    """All tensors on one ROCm device; no host tensors (no CPU path exists)."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not isinstance(t, torch.Tensor):
            raise TypeError(f"expected torch.Tensor, got {type(t).__name__}")
        if not t.is_cuda:
            raise RuntimeError(
                f"tensor on {t.device}: the FP4/INT4 kernels run on the GPU only "
                "(move inputs to a ROCm device)")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"tensors on different devices: {dev} vs {t.device}")
    return dev


def same_device_index(*tensors: torch.Tensor) -> int:
    """Device index shared by every (non-None) tensor, which must all be on a
    ROCm device: the cheap check of the per-call hot path."""
    idx = -1
    for t in tensors:
        if t is None:
            continue
        i = t.get_device()
        if i < 0:
            raise RuntimeError(
                f"tensor on {t.device}: the FP4/INT4 kernels run on the GPU only "
                "(move inputs to a ROCm device)")
        if idx < 0:
            idx = i
        elif i != idx:
            raise RuntimeError(f"tensors on different devices: cuda:{idx} vs cuda:{i}")
    return idx


# ---------------------------------------------------------------------------
# Per-(device, stream) workspace.  Its head holds split-K arrival counters that
# the kernels leave at zero, so it is allocated zeroed once and reused.
# ---------------------------------------------------------------------------
_ws: dict[tuple[int, int], torch.Tensor] = {}


def workspace_on(index: int, stream: int, nbytes: int) -> torch.Tensor:
    """Workspace of at least `nbytes` for (device index, raw stream): one
    zero-initialised buffer per pair (at least 1 MiB, grown by doubling),
    held by the per-call binding when it is built (so both call paths share
    it), else here.  Buffers are kept until release_workspaces()."""
    b = binding()
    if b:
        return b.workspace(index, stream, nbytes)
    key = (index, stream)
    buf = _ws.get(key)
    if buf is None or buf.numel() < nbytes:
        size = max(nbytes, 1 << 20)
        if buf is not None:
            size = max(size, 2 * buf.numel())
        buf = torch.zeros(size, dtype=torch.uint8, device=torch.device("cuda", index))
        _ws[key] = buf
    return buf


def release_workspaces() -> None:
    """Drop every cached workspace (for callers that create and destroy many
    streams: one buffer per stream is otherwise kept for the process).  Call
    it once the work queued on those streams has finished; a captured HIP
    graph that used a released workspace must not be replayed afterwards."""
    b = binding()
    if b:
        b.release_workspaces()
    _ws.clear()


def workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    index = device.index if device.index is not None else torch.cuda.current_device()
    return workspace_on(index, _raw_stream(index), nbytes)
