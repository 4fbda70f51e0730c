"""FP4 E2M1 / asymmetric INT4 weight quantizers (the reference's
`metal_marlin.quantize_fp4` and `metal_marlin.pack_u4_weights` surface), run
on the GPU by libmmfp4.so.

The arithmetic reproduces the reference's numpy float32 steps operation by
operation, so packed words, scales and zero points are bit-identical to what
the reference produces for the same weights.  numpy inputs are accepted and
numpy outputs returned (as the reference does); torch inputs stay torch.
"""

from __future__ import annotations

import numpy as np
import torch

from . import _lib

E2M1_VALUES = np.array(
    [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0,
     -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0], dtype=np.float32)


def _to_device(x, dtype: torch.dtype | None = None, device=None) -> tuple[torch.Tensor, bool]:
    """(tensor on a ROCm device, came_from_numpy)."""
    if isinstance(x, np.ndarray):
        t = torch.from_numpy(np.ascontiguousarray(x))
        dev = device if device is not None else torch.device("cuda", torch.cuda.current_device())
        t = t.to(dev)
        from_np = True
    else:
        t, from_np = x, False
        if device is not None:
            t = t.to(device)
    _lib.require_device(t)
    if dtype is not None and t.dtype != dtype:
        t = t.to(dtype)
    return t.contiguous(), from_np


def _out(t: torch.Tensor, to_numpy: bool, np_dtype=None):
    if not to_numpy:
        return t
    a = t.cpu().numpy()
    return a.view(np_dtype) if np_dtype is not None else a


def quantize_fp4(weight, group_size: int = 128, activation_ranges=None,
                 marlin_layout: bool = True):
    """Quantize W [out_features, in_features] to FP4 E2M1, Marlin layout:
    (packed [K/8, N] uint32, scales [K/group_size, N] fp16).
    quantize_fp4.py:131-284; with activation_ranges ({"percentile",
    "smooth_factor", "input_range"}) the calibration-aware group maxima of
    :205-256 (percentile clip, sqrt(act) attenuation for act <= 1, blend),
    bit-identical to the reference's numpy arithmetic."""
    if not marlin_layout:
        raise ValueError("Legacy layout is not supported. Use marlin_layout=True.")
    w, from_np = _to_device(weight)
    if w.dtype not in (torch.float16, torch.float32):
        w = w.to(torch.float32)
    N, K = w.shape
    if K % 8 != 0:
        raise ValueError(f"Pack axis ({K}) must be divisible by 8")
    if K % group_size != 0:
        raise ValueError(f"Pack axis ({K}) must be divisible by group_size ({group_size})")
    packed = torch.empty((K // 8, N), dtype=torch.int32, device=w.device)
    scales = torch.empty((K // group_size, N), dtype=torch.float16, device=w.device)
    if activation_ranges is None:
        _lib.call("mm_fp4_quantize", _lib.ptr(w), int(w.dtype == torch.float32), N, K,
                  group_size, _lib.ptr(packed), _lib.ptr(scales), _lib.stream_of(w))
    else:
        c = _calibration_constants(activation_ranges, group_size)
        _lib.call("mm_fp4_quantize_calibrated", _lib.ptr(w), int(w.dtype == torch.float32), N, K,
                  group_size, *c, _lib.ptr(packed), _lib.ptr(scales), _lib.stream_of(w))
    return _out(packed, from_np, np.uint32), _out(scales, from_np)


def _calibration_constants(activation_ranges, group_size: int) -> tuple:
    """The constants numpy derives from the calibration dict in the
    reference's activation_ranges branch (quantize_fp4.py:205-256), for
    mm_fp4_quantize_calibrated: (use_pct, kprev, knext, gamma, mode, c1, c2,
    sf, att).

    * np.percentile(|w|, p, axis=group) ('linear'): q = f32(p) / f32(100),
      index vi = (g - 1) * q in float32, neighbours floor(vi) and floor(vi) + 1
      (both the last when vi >= g - 1, where numpy's gamma is vi + 1);
    * (1.0 - sf) and sf meet a float32 array as Python floats (float32 ops);
      np.sqrt(act) is a float64 scalar, which makes the act <= 1 blend float64.
    "percentile", "smooth_factor" and the range ends are read as Python
    numbers."""
    pct = float(activation_ranges.get("percentile", 100.0))
    sf = float(activation_ranges.get("smooth_factor", 1.0))
    if not 0.0 <= pct <= 100.0:
        raise ValueError("Percentiles must be in the range [0, 100]")
    use_pct, kprev, knext, gamma = 0, 0, 0, 0.0
    if pct < 100.0:
        use_pct = 1
        q = np.true_divide(pct, np.float32(100))
        vi = np.float32((group_size - 1) * q)
        prev = np.floor(vi)
        if vi >= group_size - 1:
            kprev = knext = group_size - 1
            gamma = float(vi - np.float32(-1))
        else:
            kprev, knext = int(prev), int(prev) + 1
            gamma = float(vi - prev)
    input_range = activation_ranges.get("input_range")
    mode, att = 0, 1.0
    if input_range is not None:
        a_min, a_max = input_range
        act = max(abs(float(a_min)), abs(float(a_max)))
        if act > 1.0:
            mode = 1
        else:
            mode, att = 2, float(np.sqrt(act))
    c1, c2 = float(np.float32(1.0 - sf)), float(np.float32(sf))
    return use_pct, kprev, knext, gamma, mode, c1, c2, sf, att


def unpack_fp4(packed, scales, group_size: int = 128, marlin_layout: bool | None = None):
    """Dequantize Marlin-layout FP4 to fp16 [K, N] (quantize_fp4.py:287-343)."""
    if marlin_layout is False:
        raise ValueError("Legacy layout is not supported. Use marlin_layout=True.")
    p, from_np = _to_device(packed.view(np.int32) if isinstance(packed, np.ndarray) else packed)
    s, _ = _to_device(scales, torch.float16, p.device)
    K, N = p.shape[0] * 8, p.shape[1]
    from .kernels import dequant_fp4
    return _out(dequant_fp4(p, s, K, N, group_size), from_np)


def compute_quantization_error(original, packed, scales, group_size: int = 128,
                               marlin_layout: bool | None = None) -> dict[str, float]:
    """mse / rmse / max_error / mean_relative_error of the round trip
    (quantize_fp4.py:346-396), computed on the GPU."""
    recon = unpack_fp4(packed, scales, group_size, marlin_layout)
    recon = torch.as_tensor(recon).to(torch.float32)
    orig = torch.as_tensor(original).to(recon.device, torch.float32)
    diff = orig - recon.t()
    mse = torch.mean(diff * diff)
    rel = torch.abs(diff) / (torch.abs(orig) + 1e-7)
    return {"mse": float(mse), "rmse": float(torch.sqrt(mse)),
            "max_error": float(torch.max(torch.abs(diff))),
            "mean_relative_error": float(torch.mean(rel))}


def pack_u4_weights(weight, group_size: int = 128):
    """Asymmetric INT4 quantizer (metal_marlin.py:184-280): W [out, in] ->
    (packed [K/8, N] uint32 bits, scales fp16 [K/g, N], zeros fp16 [K/g, N])."""
    w, from_np = _to_device(weight, torch.float16)
    N, K = w.shape
    if K % 8 != 0:
        raise ValueError(f"K ({K}) must be divisible by 8")
    if K % group_size != 0:
        raise ValueError(f"K ({K}) must be divisible by group_size ({group_size})")
    packed = torch.empty((K // 8, N), dtype=torch.int32, device=w.device)
    scales = torch.empty((K // group_size, N), dtype=torch.float16, device=w.device)
    zeros = torch.empty_like(scales)
    _lib.call("mm_u4_quantize", _lib.ptr(w), N, K, group_size, _lib.ptr(packed),
              _lib.ptr(scales), _lib.ptr(zeros), _lib.stream_of(w))
    return _out(packed, from_np, np.uint32), _out(scales, from_np), _out(zeros, from_np)


def unpack_u4_weights(packed, scales, zeros, orig_shape: tuple[int, int] | None = None):
    """INT4 dequant back to [out, in] fp16 (metal_marlin.py:283-348)."""
    p, from_np = _to_device(packed.view(np.int32) if isinstance(packed, np.ndarray) else packed)
    s, _ = _to_device(scales, torch.float16, p.device)
    z, _ = _to_device(zeros, torch.float16, p.device)
    K, N = p.shape[0] * 8, p.shape[1]
    if s.shape[1] != N:
        raise ValueError(f"scales shape {tuple(s.shape)} N-dimension mismatch with packed "
                         f"shape ({p.shape[0]}, {N})")
    if z.shape != s.shape:
        raise ValueError(f"zeros shape {tuple(z.shape)} must match scales shape {tuple(s.shape)}")
    if K % s.shape[0] != 0:
        raise ValueError(f"K={K} must be evenly divisible by num_groups={s.shape[0]}")
    from .kernels import dequant_int4
    w = dequant_int4(p, s, z, K, N, K // s.shape[0]).t()
    if orig_shape is not None:
        w = w[: orig_shape[0], : orig_shape[1]]
    return _out(w.contiguous(), from_np)
