"""Flat-group FP4 E2M1 quantization: the `FP4Metal` surface of
metal_marlin/fp4_metal.py:71-314, on gfx950 kernels (mm_fp4flat.hip).

    fp4 = FP4Metal()
    indices, scales = fp4.quantize(tensor, group_size=128)
    reconstructed = fp4.dequantize(indices, scales, group_size=128)

Groups run over the flattened tensor (the last one padded with zeros);
scales are float32 `max(max|x| / 6, 1e-8)` per group; indices are unpacked
uint8 codes `sign_bit | nearest positive E2M1 index` in the input's shape.
The reference runs these on the host in numpy (its Metal pipelines are
compiled but never dispatched); here every call runs on the GPU.  numpy
inputs are copied to the current ROCm device and the results copied back as
numpy arrays, so callers see the reference's types.  There is no CPU path:
without a ROCm device and the built library, `available` is False and the
calls raise.
"""

from __future__ import annotations

import numpy as np
import torch

from . import _lib

__all__ = ["FP4Metal", "quantize_fp4_metal", "dequantize_fp4_metal", "E2M1_VALUES",
           "E2M1_POSITIVE"]

# metal_marlin/_compat.py:283-310
E2M1_VALUES = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0,
                        -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0], dtype=np.float32)
E2M1_POSITIVE = E2M1_VALUES[:8].copy()

_DTYPE_CODE = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}


def _gpu_available() -> bool:
    try:
        _lib.load()
    except (ImportError, OSError):
        return False
    return torch.cuda.is_available()


def _to_device(x, dtype=None) -> tuple[torch.Tensor, bool]:
    """(device tensor, came_from_numpy)."""
    if isinstance(x, torch.Tensor):
        t = x
        from_np = False
    else:
        t = torch.from_numpy(np.ascontiguousarray(np.asarray(x)))
        from_np = True
    if t.device.type != "cuda":
        if not from_np:
            raise RuntimeError(f"tensor on {t.device}: FP4Metal runs on the GPU only "
                               "(move the tensor to a ROCm device)")
        if not torch.cuda.is_available():
            raise RuntimeError("FP4Metal needs a ROCm device (there is no CPU path)")
        t = t.to(torch.device("cuda", torch.cuda.current_device()))
    if dtype is not None and t.dtype != dtype:
        t = t.to(dtype)
    return t.contiguous(), from_np


class FP4Metal:
    """Flat-group FP4 E2M1 quantize / dequantize / pack (fp4_metal.py:71-314)."""

    def __init__(self, device=None):
        # `device` is accepted for signature compatibility (the reference takes a
        # Metal device); the current ROCm device is used.
        del device
        self._e2m1_table = E2M1_VALUES
        self._e2m1_positive = E2M1_POSITIVE
        self._available = _gpu_available()

    @property
    def available(self) -> bool:
        """True when the gfx950 library is built and a ROCm device is visible."""
        return self._available

    def quantize(self, values, group_size: int = 128):
        """-> (indices uint8 in the shape of `values`, scales float32 [n_groups]),
        torch tensors on the input's device for a tensor input, numpy arrays for
        array input (fp4_metal.py:130-190).  fp16 / bf16 / f32 tensors are read
        as they are; other dtypes are converted to float32 first, as the
        reference's `astype(np.float32)` does."""
        if group_size <= 0:
            raise ValueError(f"group_size must be > 0, got {group_size}")
        t, from_np = _to_device(values)
        if t.dtype not in _DTYPE_CODE:
            t = t.to(torch.float32)
        n = t.numel()
        n_groups = -(-n // group_size)
        codes = torch.empty(t.shape, dtype=torch.uint8, device=t.device)
        scales = torch.empty((n_groups,), dtype=torch.float32, device=t.device)
        _lib.call("mm_fp4_flat_quantize", _lib.ptr(t), n, _DTYPE_CODE[t.dtype], group_size,
                  _lib.ptr(codes), _lib.ptr(scales), _lib.stream_of(t))
        if from_np:
            return codes.cpu().numpy(), scales.cpu().numpy()
        return codes, scales

    def dequantize(self, indices, scales, group_size: int = 128):
        """E2M1[indices] * scales[group] as float32 in the shape of `indices`
        (fp4_metal.py:192-276).  Indices are read through their low 4 bits
        (the reference's table lookup raises for values above 15)."""
        if group_size <= 0:
            raise ValueError(f"group_size must be > 0, got {group_size}")
        idx, from_np = _to_device(indices)
        if idx.dtype != torch.uint8:
            idx = (idx.to(torch.int64) & 0xF).to(torch.uint8)
        sc, _ = _to_device(scales)
        if sc.device != idx.device:
            sc = sc.to(idx.device)
        sc = sc.reshape(-1).to(torch.float32).contiguous()
        n = idx.numel()
        if sc.numel() * group_size < n:
            raise ValueError(f"{sc.numel()} scales x group_size {group_size} cover fewer than "
                             f"the {n} indices")
        out = torch.empty(idx.shape, dtype=torch.float32, device=idx.device)
        _lib.call("mm_fp4_flat_dequantize", _lib.ptr(idx), _lib.ptr(sc), n, sc.numel(),
                  group_size, _lib.ptr(out), _lib.stream_of(idx))
        return out.cpu().numpy() if from_np else out

    def pack_pair(self, lo, hi):
        """lo | (hi << 4) per byte, each operand masked to 4 bits
        (fp4_metal.py:278-300).  Operands broadcast against each other."""
        a, from_np = _to_device(lo)
        b, _ = _to_device(hi)
        if b.device != a.device:
            b = b.to(a.device)
        a, b = torch.broadcast_tensors(a.to(torch.uint8), b.to(torch.uint8))
        a, b = a.contiguous(), b.contiguous()
        out = torch.empty(a.shape, dtype=torch.uint8, device=a.device)
        _lib.call("mm_fp4_pack_pair", _lib.ptr(a), _lib.ptr(b), a.numel(), _lib.ptr(out),
                  _lib.stream_of(a))
        return out.cpu().numpy() if from_np else out


def quantize_fp4_metal(values, group_size: int = 128):
    """FP4Metal().quantize (fp4_metal.py:303-307)."""
    return FP4Metal().quantize(values, group_size)


def dequantize_fp4_metal(indices, scales, group_size: int = 128):
    """FP4Metal().dequantize (fp4_metal.py:310-314)."""
    return FP4Metal().dequantize(indices, scales, group_size)
