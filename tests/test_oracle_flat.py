"""Pins the oracle's flat-group FP4 functions (FP4Metal,
metal_marlin/fp4_metal.py:130-300) with checks the mathematics fixes: a
float64 nearest-value brute force with ties to the lower index, the scale
closed form and its floor, sign from v < 0, zero padding, NaN/inf groups and
hand-computed known answers."""

from __future__ import annotations

import numpy as np
import pytest

from oracle import fp4 as ofp4

POS64 = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0])


def _nearest_lower(a: float) -> int:
    best, bd = 0, abs(POS64[0] - a)
    for j in range(1, 8):
        d = abs(POS64[j] - a)
        if d < bd:
            best, bd = j, d
    return best


def test_flat_known_answers():
    # max 6 -> scale 1: codes are the values' own nearest entries; the ties
    # 0.25 (0 | 0.5), 0.75 (0.5 | 1), 1.25 (1 | 1.5), 5 (4 | 6) take the lower
    # index; -0.0 has no sign bit (-0.0 < 0 is false).
    x = np.array([6, -3, 0.25, 0.75, -0.0, 0, 1.25, 5], np.float32)
    codes, scales = ofp4.flat_quantize(x, 8)
    assert codes.tolist() == [7, 13, 0, 1, 0, 0, 2, 6]
    assert scales.dtype == np.float32 and scales.tolist() == [1.0]
    deq = ofp4.flat_dequantize(codes, scales, 8)
    assert deq.tolist() == [6, -3, 0, 0.5, 0, 0, 1.0, 4]
    # scale = max|x| / 6: doubling the input doubles the scale, not the codes
    c2, s2 = ofp4.flat_quantize(2 * x, 8)
    assert np.array_equal(c2, codes) and s2.tolist() == [2.0]


def test_flat_bruteforce_nearest(rng):
    x = rng.normal(0, 1, (37, 53)).astype(np.float32)      # 1961 values, ragged last group
    g = 64
    codes, scales = ofp4.flat_quantize(x, g)
    flat = x.reshape(-1)
    n_groups = -(-flat.size // g)
    assert codes.shape == x.shape and scales.shape == (n_groups,)
    for gi in range(n_groups):
        seg = flat[gi * g:(gi + 1) * g].astype(np.float64)
        # f32(max / 6) is the correctly rounded quotient (double rounding
        # through float64 is innocuous for division)
        s = np.float32(np.max(np.abs(seg)) / 6.0)
        assert scales[gi] == max(s, np.float32(1e-8))
    v = (flat / np.repeat(scales, g)[:flat.size]).astype(np.float32)
    for j, (vj, cj) in enumerate(zip(v.tolist(), codes.reshape(-1).tolist())):
        assert cj == ((8 if vj < 0 else 0) | _nearest_lower(abs(vj))), j


def test_flat_floor_padding_and_specials():
    # all-zero group -> scale floor 1e-8 (f32), codes 0; a tiny group divides by
    # the floor; the second group of a ragged input is zero-padded
    x = np.array([0, 0, 0, 0, 3e-8, -6e-8, 1e-8, 0, 1.5, -0.75], np.float32)
    codes, scales = ofp4.flat_quantize(x, 4)
    assert scales[0] == np.float32(1e-8) and scales[1] == np.float32(1e-8)
    assert scales[2] == np.float32(1.5) / np.float32(6.0)
    assert codes[:4].tolist() == [0, 0, 0, 0]
    v = x[4:8] / np.float32(1e-8)
    assert codes[4:8].tolist() == [(8 if t < 0 else 0) | _nearest_lower(abs(t)) for t in v]
    assert codes[8:].tolist() == [7, 8 | 5]              # -0.75 / 0.25 = -3
    # a NaN makes its group's scale NaN and every code 0; inf gives scale inf
    # and codes 0 (x / inf = +-0, inf / inf = NaN); other groups unaffected
    y = np.array([1, np.nan, -2, 3, 1, np.inf, -2, 3, 6, 3, -1.5, 0.5], np.float32)
    codes, scales = ofp4.flat_quantize(y, 4)
    assert np.isnan(scales[0]) and np.isinf(scales[1]) and scales[2] == 1.0
    assert codes[:8].tolist() == [0] * 8
    assert codes[8:].tolist() == [7, 5, 8 | 3, 1]


def test_flat_dequant_round_trip_bound(rng):
    x = rng.normal(0, 0.02, (4096,)).astype(np.float32)
    codes, scales = ofp4.flat_quantize(x, 128)
    deq = ofp4.flat_dequantize(codes, scales, 128)
    s = np.repeat(scales, 128).astype(np.float64)
    # the widest gap between E2M1 magnitudes is 2 (4 -> 6): error <= 1 * scale
    assert np.all(np.abs(deq.astype(np.float64) - x) <= s * (1.0 + 1e-6))
    # dequant is exactly E2M1[code] * scale in f32
    assert np.array_equal(deq, ofp4.E2M1_VALUES[codes] * np.repeat(scales, 128))


def test_pack_pair_known_answers():
    lo = np.array([0, 1, 15, 0x1F, 7], np.uint8)
    hi = np.array([0, 2, 15, 0x21, 8], np.uint8)
    assert ofp4.pack_pair(lo, hi).tolist() == [0x00, 0x21, 0xFF, 0x1F, 0x87]
