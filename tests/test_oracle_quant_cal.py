"""Pins the oracle's calibration-aware FP4 quantizer (quantize_fp4.py:205-256,
`oracle.fp4.quantize_fp4_calibrated`).

* golden vectors written by the reference's own quantize_fp4 with
  activation_ranges (tests/golden/make_quantize_fp4_vectors.py);
* the percentile group maximum against an exact-rational order statistic with
  linear interpolation at index (n - 1) * p / 100 (a wrong index rule, a
  missing interpolation or an off-by-one order statistic fails it);
* reductions the formulas fix: smooth_factor = 0 with act > 1, and
  percentile = 100 without an input range, are the weight-only quantizer;
  act = 1/4 (1/16) halves (quarters) the group maximum, and the float64 scale
  is the correctly rounded fp16 of max/12 (max/24);
* the codes are the nearest E2M1 values of w / f32(group max) * 6.
"""

from __future__ import annotations

from fractions import Fraction
from pathlib import Path

import numpy as np
import pytest

from oracle import fp4 as ofp4

GOLD = Path(__file__).resolve().parent / "golden" / "quantize_fp4_vectors.npz"
CAL_CASES = ["cal_p999_f32", "cal_p90_small_f16", "cal_large_sf03_f32", "cal_small_sf1_g32_f32",
             "cal_p50_g8_f32", "cal_p99_crafted_f32", "cal_p37_quarter_f16", "cal_f64_blend_f32"]


def cal_case(d, name):
    pct, sf, a_min, a_max = d[f"{name}__cal"]
    ar = {"percentile": float(pct), "smooth_factor": float(sf)}
    if not np.isnan(a_min):
        ar["input_range"] = (float(a_min), float(a_max))
    return d[f"{name}__w"], int(d[f"{name}__g"]), ar


@pytest.mark.parametrize("name", CAL_CASES)
def test_calibrated_matches_reference_vectors(name):
    d = np.load(GOLD)
    w, g, ar = cal_case(d, name)
    packed, scales = ofp4.quantize_fp4_calibrated(w, g, ar)
    assert np.array_equal(packed, d[f"{name}__packed"])
    assert np.array_equal(scales.view(np.uint16), d[f"{name}__scales"].view(np.uint16))


def _exact_percentile(vals, pct) -> Fraction:
    """Linear-method percentile in exact rationals: sorted values x, index
    h = (n - 1) * p / 100, x[floor h] + (h - floor h) * (x[floor h + 1] - x[floor h])."""
    x = sorted(Fraction(float(v)) for v in vals)
    h = (len(x) - 1) * Fraction(pct) / 100
    lo = int(h)
    if lo >= len(x) - 1:
        return x[-1]
    return x[lo] + (h - lo) * (x[lo + 1] - x[lo])


@pytest.mark.parametrize("g,pct", [(8, 50.0), (8, 62.5), (32, 90.0), (128, 99.9), (128, 37.0),
                                   (64, 0.0), (16, 100.0 - 1e-9)])
def test_percentile_group_max_brute_force(rng, g, pct):
    n = 6
    w = rng.normal(0, 1.0, (n, 2 * g)).astype(np.float32)
    w[0, :g] = np.round(w[0, :g] * 4) / 4           # ties among the group values
    _, scales = ofp4.quantize_fp4_calibrated(w, g, {"percentile": pct})
    wk = w.T.reshape(2, g, n)
    for gi in range(2):
        for col in range(n):
            exact = max(_exact_percentile(np.abs(wk[gi, :, col]), pct), Fraction(1e-7))
            want = np.float16(float(exact / 6))
            got = scales[gi, col]
            # numpy rounds q, the index and the lerp in float32: the group max
            # may be off by float32 ulps, which moves the fp16 scale by at most one ulp
            assert abs(int(got.view(np.uint16)) - int(want.view(np.uint16))) <= 1, (gi, col)
    # an integral index (g - 1) * p / 100 picks an order statistic exactly
    if float((g - 1) * pct / 100).is_integer():
        for gi in range(2):
            for col in range(n):
                exact = _exact_percentile(np.abs(wk[gi, :, col]), pct)
                assert scales[gi, col] == np.float16(np.float32(exact) / np.float32(6.0))


def test_smooth_zero_and_full_percentile_reduce_to_weight_only(rng):
    w = rng.normal(0, 0.05, (24, 256)).astype(np.float32)
    ref = ofp4.quantize_fp4(w, 128)
    for ar in ({"percentile": 100.0},
               {"percentile": 100.0, "input_range": (-3.0, 2.0), "smooth_factor": 0.0},
               {"input_range": (-1.5, 7.0), "smooth_factor": 1.0}):
        got = ofp4.quantize_fp4_calibrated(w, 128, ar)
        assert np.array_equal(got[0], ref[0]), ar
        assert np.array_equal(got[1].view(np.uint16), ref[1].view(np.uint16)), ar


@pytest.mark.parametrize("act,factor", [(0.25, Fraction(1, 2)), (0.0625, Fraction(1, 4))])
def test_attenuation_by_sqrt_act(rng, act, factor):
    """act <= 1, smooth_factor 1: group max = absmax * sqrt(act) (exact for
    these act), scale = fp16 of the float64 quotient by 6: the correctly
    rounded fp16 of absmax * factor / 6 unless that quotient's float64
    rounding lands on an fp16 tie (checked not to happen here)."""
    w = rng.normal(0, 0.05, (16, 256)).astype(np.float32)
    _, scales = ofp4.quantize_fp4_calibrated(w, 128, {"input_range": (-act, act / 2)})
    amax = np.abs(w.T.reshape(2, 128, 16)).max(axis=1)
    for gi in range(2):
        for col in range(16):
            exact = Fraction(float(amax[gi, col])) * factor / 6
            want = np.float16(float(exact))           # float(Fraction) rounds correctly
            assert scales[gi, col].view(np.uint16) == want.view(np.uint16)
    # and it differs from the weight-only scale: the attenuation is applied
    _, s0 = ofp4.quantize_fp4(w, 128)
    assert np.all(scales.astype(np.float32) < s0.astype(np.float32))


def test_blend_act_above_one_is_weight_max(rng):
    """act > 1: calibrated = the weight maximum, so any smooth_factor blends
    two equal values; the float32 blend is within one float32 ulp of it."""
    w = rng.normal(0, 0.05, (16, 256)).astype(np.float32)
    _, s0 = ofp4.quantize_fp4(w, 128)
    for sf in (0.1, 0.3, 0.77):
        _, s = ofp4.quantize_fp4_calibrated(w, 128, {"input_range": (-5.0, 2.0),
                                                     "smooth_factor": sf})
        d = np.abs(s.view(np.uint16).astype(np.int32) - s0.view(np.uint16).astype(np.int32))
        assert d.max() <= 1


def test_calibrated_codes_are_nearest_value(rng):
    w = rng.normal(0, 0.02, (32, 256)).astype(np.float32)
    ar = {"percentile": 95.0, "input_range": (-0.5, 0.2), "smooth_factor": 0.5}
    packed, scales = ofp4.quantize_fp4_calibrated(w, 128, ar)
    codes = ofp4.unpack_nibbles(packed)
    wk = w.T.reshape(2, 128, 32).astype(np.float64)
    gmw = np.maximum(np.percentile(np.abs(wk), 95.0, axis=1, keepdims=True), 1e-7)
    gmax = 0.5 * gmw + 0.5 * gmw * np.sqrt(0.5)
    v = np.clip(wk / gmax * 6.0, -6, 6).reshape(256, 32)
    vals = ofp4.E2M1_VALUES.astype(np.float64)
    chosen = np.abs(v - vals[codes])
    best = np.min(np.abs(v[..., None] - vals[None, None, :]), axis=-1)
    assert np.all(chosen <= best + 1e-5)
    # percentile < 100 clips: some group values exceed the group max
    assert np.any(np.abs(wk) > gmax)
