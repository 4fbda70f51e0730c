"""numpy restatement of the reference's FP4/INT4 quantizers, dequantizers and
fp32 dequant+matmul (test infrastructure; see oracle/__init__.py)."""

from __future__ import annotations

import numpy as np

# E2M1 code -> value, bit layout [sign | exp(2) | mantissa].
# metal_marlin/_compat.py:283-302, metal_marlin/quantize_fp4.py:37-57
E2M1_VALUES = np.array(
    [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0,
     -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0],
    dtype=np.float32,
)
_E2M1_POS = E2M1_VALUES[:8]
_E2M1_NEG = -_E2M1_POS


def unpack_nibbles(packed: np.ndarray) -> np.ndarray:
    """[K/8, N] uint32 -> [K, N] uint8 codes; word (kp, n) holds row 8kp+i in
    bits 4i..4i+3 (quantize_fp4.py:280-282, metal_marlin.py:268-272)."""
    packed = np.ascontiguousarray(packed).view(np.uint32)
    kp, n = packed.shape
    codes = np.empty((kp * 8, n), dtype=np.uint8)
    for i in range(8):
        codes[i::8] = ((packed >> np.uint32(4 * i)) & np.uint32(0xF)).astype(np.uint8)
    return codes


def pack_nibbles(codes: np.ndarray) -> np.ndarray:
    """[K, N] codes -> [K/8, N] uint32 (inverse of unpack_nibbles)."""
    k, n = codes.shape
    packed = np.zeros((k // 8, n), dtype=np.uint32)
    for i in range(8):
        packed |= codes[i::8].astype(np.uint32) << np.uint32(4 * i)
    return packed


def e2m1_decode(codes: np.ndarray) -> np.ndarray:
    """Unscaled E2M1 value (float32), code 8 -> -0.0.
    src/marlin_gemm.metal:170-185 (dequant_fp4_bitwise)."""
    return E2M1_VALUES[codes.astype(np.int64)]


def _expand_groups(t: np.ndarray, group_size: int) -> np.ndarray:
    return np.repeat(t, group_size, axis=0)


def dequant_fp4(packed: np.ndarray, scales: np.ndarray, group_size: int) -> np.ndarray:
    """Bit-exact reference dequant: w = fp16_RNE(E2M1[code] * f32(scale)),
    with a non-finite f32 product replaced by +0.0.

    src/marlin_gemm.metal:130-137 (safe_dequant) applied to :170-185; the same
    value as tests/test_dequant.py:253-262 (ref_dequant_fp4_bulk) for finite
    scales.  Returns [K, N] float16.
    """
    codes = unpack_nibbles(packed)
    s = _expand_groups(np.asarray(scales, dtype=np.float16).astype(np.float32), group_size)
    with np.errstate(over="ignore", invalid="ignore"):
        prod = e2m1_decode(codes) * s            # exact in fp32
        prod = np.where(np.isfinite(prod), prod, np.float32(0.0))
        return prod.astype(np.float16)            # one RNE rounding


def dequant_u4(packed: np.ndarray, scales: np.ndarray, zeros: np.ndarray,
               group_size: int) -> np.ndarray:
    """Bit-exact reference INT4 dequant: w = fp16_RNE(fp16(q - clamp(z,+-127)) * s),
    non-finite f32 product -> +0.0.

    src/marlin_gemm.metal:118-120 (clamp_zero_point), :148-156
    (safe_dequant_u4_value), :1984-2012 (fused_dequant_u4x8: the magic-bias
    nibble is exactly q); tests/test_dequant.py:206-221 (ref_dequant_u4_bulk).
    Returns [K, N] float16.
    """
    q = unpack_nibbles(packed).astype(np.float32)
    z = np.asarray(zeros, dtype=np.float16).astype(np.float32)
    z = np.clip(z, -127.0, 127.0)
    s = _expand_groups(np.asarray(scales, dtype=np.float16).astype(np.float32), group_size)
    z = _expand_groups(z, group_size)
    with np.errstate(over="ignore", invalid="ignore"):
        diff = (q - z).astype(np.float16).astype(np.float32)
        prod = diff * s
        prod = np.where(np.isfinite(prod), prod, np.float32(0.0))
        return prod.astype(np.float16)


def quantize_to_fp4(values: np.ndarray) -> np.ndarray:
    """Nearest E2M1 code; >= 0 (incl. -0.0) -> codes 0-7, < 0 -> 8-15; ties
    resolve to the lower table index (argmin).  quantize_fp4.py:64-107."""
    flat = np.asarray(values, dtype=np.float32).reshape(-1)
    out = np.zeros(flat.shape[0], dtype=np.uint8)
    pos = flat >= 0
    neg = ~pos
    if pos.any():
        v = np.clip(flat[pos], 0, 6.0)
        out[pos] = np.argmin(np.abs(v[:, None] - _E2M1_POS[None, :]), axis=1).astype(np.uint8)
    if neg.any():
        v = np.clip(flat[neg], -6.0, 0)
        out[neg] = (np.argmin(np.abs(v[:, None] - _E2M1_NEG[None, :]), axis=1) + 8).astype(np.uint8)
    return out.reshape(np.shape(values))


def quantize_fp4(weight: np.ndarray, group_size: int = 128):
    """Weight-only FP4 quantizer, Marlin layout.  quantize_fp4.py:131-284:
    w = W.T (f32) -> [K, N]; absmax per group of `group_size` rows, floored at
    1e-7; scales = fp16(absmax/6); codes = nearest E2M1 of w/absmax*6 (f32,
    using the f32 absmax, not the fp16 scale); pack 8 rows per uint32.

    weight: [N, K] (out_features, in_features).  Returns (packed [K/8, N]
    uint32, scales [K/group_size, N] float16).
    """
    w = np.asarray(weight).astype(np.float32).T
    k, n = w.shape
    if k % 8 != 0:
        raise ValueError(f"Pack axis ({k}) must be divisible by 8")
    if k % group_size != 0:
        raise ValueError(f"Pack axis ({k}) must be divisible by group_size ({group_size})")
    g = w.reshape(k // group_size, group_size, n)
    gmax = np.max(np.abs(g), axis=1, keepdims=True)
    gmax = np.maximum(gmax, np.float32(1e-7))
    scales = (gmax / np.float32(6.0)).astype(np.float16).squeeze(1)
    w_scaled = (g / gmax.astype(np.float32) * np.float32(6.0)).reshape(k, n)
    return pack_nibbles(quantize_to_fp4(w_scaled)), scales


def quantize_fp4_calibrated(weight: np.ndarray, group_size: int,
                            activation_ranges: dict):
    """Calibration-aware FP4 quantizer, Marlin layout: the activation_ranges
    branch of quantize_fp4.py:205-256, with numpy's own dtype flow (NEP 50):

    * group max: np.percentile(|w|, p) over the group when p < 100 (numpy's
      'linear' method on float32), else the absmax; floored at 1e-7 (f32);
    * with "input_range" (a_min, a_max), act = max(|a_min|, |a_max|):
      act > 1  -> calibrated = group max, blended in float32:
                  (1 - sf) * gmax + sf * calibrated;
      act <= 1 -> calibrated = gmax * np.sqrt(act), a float64 scalar, so the
                  blend (and the scale's division by 6) runs in float64;
    * scales = fp16(group_max / 6); codes = nearest E2M1 of w / f32(group_max) * 6.

    "percentile", "smooth_factor" and the range ends are taken as Python
    numbers (the reference's defaults 100.0 and 1.0).
    """
    pct = float(activation_ranges.get("percentile", 100.0))
    sf = float(activation_ranges.get("smooth_factor", 1.0))
    input_range = activation_ranges.get("input_range")
    w = np.asarray(weight).astype(np.float32).T
    k, n = w.shape
    if k % 8 != 0:
        raise ValueError(f"Pack axis ({k}) must be divisible by 8")
    if k % group_size != 0:
        raise ValueError(f"Pack axis ({k}) must be divisible by group_size ({group_size})")
    g = w.reshape(k // group_size, group_size, n)
    if pct < 100.0:
        gmw = np.percentile(np.abs(g), pct, axis=1, keepdims=True)
    else:
        gmw = np.max(np.abs(g), axis=1, keepdims=True)
    gmw = np.maximum(gmw, 1e-7)
    if input_range is not None:
        a_min, a_max = input_range
        act = max(abs(float(a_min)), abs(float(a_max)))
        cal = gmw if act > 1.0 else gmw * np.sqrt(act)
        gmax = (1.0 - sf) * gmw + sf * cal
    else:
        gmax = gmw
    scales = (gmax / 6.0).astype(np.float16).squeeze(1)
    w_scaled = (g / gmax.astype(np.float32) * 6.0).reshape(k, n)
    return pack_nibbles(quantize_to_fp4(w_scaled)), scales


def pack_u4_weights(weight: np.ndarray, group_size: int = 128):
    """Asymmetric INT4 quantizer, Marlin layout.  metal_marlin.py:184-280:
    w = fp16(W).T as f32; per group s = max((max-min)/15, 1e-7) (f32),
    z = round_half_even(-min/s) (not clipped), q = clip(round(w/s + z), 0, 15)
    with the f32 s and z; scales and zeros returned as fp16.

    Returns (packed [K/8, N] uint32, scales fp16 [K/g, N], zeros fp16 [K/g, N]).
    """
    w = np.asarray(weight).astype(np.float16).T.astype(np.float32)
    k, n = w.shape
    if k % 8 != 0:
        raise ValueError(f"K ({k}) must be divisible by 8")
    if k % group_size != 0:
        raise ValueError(f"K ({k}) must be divisible by group_size ({group_size})")
    g = w.reshape(k // group_size, group_size, n)
    gmin = g.min(axis=1)
    gmax = g.max(axis=1)
    s = np.maximum((gmax - gmin) / np.float32(15.0), np.float32(1e-7))
    z = np.round(-gmin / s).astype(np.float32)
    se = _expand_groups(s, group_size)
    ze = _expand_groups(z, group_size)
    q = np.round(w / se + ze).clip(0, 15).astype(np.uint32)
    return pack_nibbles(q), s.astype(np.float16), z.astype(np.float16)


def dequant_fp4_f32(packed: np.ndarray, scales: np.ndarray, group_size: int) -> np.ndarray:
    """fp32 dequant used by the reference's CPU GEMM path (no fp16 rounding):
    B[k, n] = E2M1[code] * f32(scale).  kernels_core.py:1872-1901."""
    codes = unpack_nibbles(packed)
    s = _expand_groups(np.asarray(scales, dtype=np.float16).astype(np.float32), group_size)
    return e2m1_decode(codes) * s


def dequant_u4_f32(packed: np.ndarray, scales: np.ndarray, zeros: np.ndarray,
                   group_size: int) -> np.ndarray:
    """fp32 INT4 dequant of the reference's CPU GEMM path: (q - z) * s in fp32.
    kernels_core.py:1996-2013."""
    q = unpack_nibbles(packed).astype(np.float32)
    s = _expand_groups(np.asarray(scales, dtype=np.float16).astype(np.float32), group_size)
    z = _expand_groups(np.asarray(zeros, dtype=np.float16).astype(np.float32), group_size)
    return (q - z) * s


def gemm_fp4_ref(a: np.ndarray, packed: np.ndarray, scales: np.ndarray,
                 group_size: int) -> np.ndarray:
    """C = fp16(A_f32 @ B_f32), the reference's own fp32 dequant+matmul
    (kernels_core.py:1860-1905; tests/test_gemm.py:260-263).  a: [M, K]."""
    b = dequant_fp4_f32(packed, scales, group_size)
    return (np.asarray(a, dtype=np.float32) @ b).astype(np.float16)


def gemm_u4_ref(a: np.ndarray, packed: np.ndarray, scales: np.ndarray, zeros: np.ndarray,
                group_size: int) -> np.ndarray:
    """INT4 counterpart, kernels_core.py:1989-2017."""
    b = dequant_u4_f32(packed, scales, zeros, group_size)
    return (np.asarray(a, dtype=np.float32) @ b).astype(np.float16)


def max_abs_rel(out: np.ndarray, ref: np.ndarray) -> float:
    """max |out - ref| / max |ref| (the north-star parity measure)."""
    out = np.asarray(out, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    denom = max(float(np.max(np.abs(ref))), 1e-30)
    return float(np.max(np.abs(out - ref))) / denom


# ---------------------------------------------------------------------------
# Flat-group FP4 (FP4Metal, metal_marlin/fp4_metal.py:130-300)
# ---------------------------------------------------------------------------
def flat_quantize(values: np.ndarray, group_size: int = 128):
    """FP4Metal.quantize (fp4_metal.py:130-190): flatten to float32, pad the
    last group with zeros (:150-160), scales = max(max|x| / 6, 1e-8) in f32
    (:161-163), v = x / scale (:166), code = (8 if v < 0 else 0) | argmin_j
    |E2M1_POS[j] - |v|| (:167-172, ties to the lower j).  Returns (codes
    uint8 in the input's shape, scales float32 [n_groups])."""
    v = np.asarray(values)
    flat = v.reshape(-1).astype(np.float32)
    n = flat.shape[0]
    n_groups = (n + group_size - 1) // group_size
    padded = np.zeros(n_groups * group_size, np.float32)
    padded[:n] = flat
    g = padded.reshape(n_groups, group_size)
    with np.errstate(invalid="ignore", divide="ignore"):
        scales = np.maximum(np.max(np.abs(g), axis=1) / np.float32(6.0), np.float32(1e-8))
        normalized = (g / scales[:, None]).reshape(-1)
        dist = np.abs(_E2M1_POS[None, :] - np.abs(normalized)[:, None])
    pos_idx = np.argmin(dist, axis=1).astype(np.uint8)        # all-NaN rows -> 0
    sign = np.where(normalized < 0, np.uint8(8), np.uint8(0))
    codes = (sign | pos_idx)[:n].reshape(v.shape)
    return codes, scales.astype(np.float32)


def flat_dequantize(codes: np.ndarray, scales: np.ndarray, group_size: int = 128) -> np.ndarray:
    """FP4Metal.dequantize (fp4_metal.py:192-276): E2M1[code] * scale in
    float32, groups over the flattened codes; shape of `codes`."""
    c = np.asarray(codes)
    s = np.asarray(scales, dtype=np.float32).reshape(-1)
    flat = E2M1_VALUES[c.reshape(-1).astype(np.int64)]
    n = flat.shape[0]
    padded = np.zeros(s.shape[0] * group_size, np.float32)
    padded[:n] = flat
    with np.errstate(invalid="ignore"):
        deq = padded.reshape(-1, group_size) * s[:, None]
    return deq.reshape(-1)[:n].reshape(c.shape)


def pack_pair(lo: np.ndarray, hi: np.ndarray) -> np.ndarray:
    """FP4Metal.pack_pair (fp4_metal.py:278-300): (lo & 15) | ((hi & 15) << 4)."""
    lo = np.asarray(lo, dtype=np.uint8)
    hi = np.asarray(hi, dtype=np.uint8)
    return (lo & np.uint8(0x0F)) | ((hi & np.uint8(0x0F)) << np.uint8(4))
