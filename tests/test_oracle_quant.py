"""Pins the oracle's quantizers: golden vectors written by the reference's
own quantize_fp4 (tests/golden/make_quantize_fp4_vectors.py) and invariants."""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

from oracle import fp4 as ofp4

GOLD = Path(__file__).resolve().parent / "golden" / "quantize_fp4_vectors.npz"
CASES = ["w_normal_f16", "w_crafted_f32", "w_crafted_f16", "w_normal_f32_g32"]


@pytest.mark.parametrize("name", CASES)
def test_quantize_fp4_matches_reference_vectors(name):
    d = np.load(GOLD)
    w, g = d[f"{name}__w"], int(d[f"{name}__g"])
    packed, scales = ofp4.quantize_fp4(w, g)
    assert np.array_equal(packed, d[f"{name}__packed"])
    assert np.array_equal(scales.view(np.uint16), d[f"{name}__scales"].view(np.uint16))


def test_quantize_fp4_is_nearest_value(rng):
    w = rng.normal(0, 0.02, (32, 256)).astype(np.float32)
    packed, scales = ofp4.quantize_fp4(w, 128)
    codes = ofp4.unpack_nibbles(packed)                       # [K, N]
    wk = w.T.reshape(2, 128, 32)
    amax = np.maximum(np.abs(wk).max(axis=1, keepdims=True), np.float32(1e-7))
    v = (wk / amax * np.float32(6.0)).reshape(256, 32).astype(np.float64)
    vals = ofp4.E2M1_VALUES.astype(np.float64)
    chosen = np.abs(v - vals[codes])
    best = np.min(np.abs(v[..., None] - vals[None, None, :]), axis=-1)
    assert np.all(chosen <= best + 1e-12)
    # the group absmax maps to +-6 exactly
    assert np.all(np.isin(codes.max(axis=0), [7, 15]))


def test_pack_u4_round_trip_and_extremes(rng):
    w = rng.normal(0, 0.02, (64, 256)).astype(np.float16)
    packed, s, z = ofp4.pack_u4_weights(w, 128)
    q = ofp4.unpack_nibbles(packed).astype(np.float64)
    wt = w.T.astype(np.float64).reshape(2, 128, 64)
    sf = s.astype(np.float64)[:, None, :]
    zf = z.astype(np.float64)[:, None, :]
    rec = ((q.reshape(2, 128, 64) - zf) * sf)
    # within half a step (+ fp16 rounding of s and z) wherever no clipping occurs
    assert np.max(np.abs(rec - wt) / sf) <= 0.5 + 0.02
    # per-group minimum maps to q = 0 when the zero point is in range
    assert np.all(q.reshape(2, 128, 64).min(axis=1) == 0)


def test_pack_u4_matches_reference_test_quantizer_when_no_clip(rng):
    # tests/test_gemm.py:146-187 quantize_int4 uses the same formula but clips z
    # to [0, 15] and divides by the fp16 scale; for inputs whose group minimum is
    # an exact multiple of the scale both agree on q.
    w = rng.integers(-7, 8, (16, 128)).astype(np.float16) * np.float16(0.125)
    packed, s, z = ofp4.pack_u4_weights(w, 128)
    wf = w.T.astype(np.float32)
    mn, mx = wf.min(axis=0), wf.max(axis=0)
    s_ref = np.maximum((mx - mn) / 15.0, np.float32(1e-7))
    z_ref = np.clip(np.round(-mn / s_ref), 0, 15)
    q_ref = np.clip(np.round(wf / s_ref + z_ref), 0, 15).astype(np.uint32)
    assert np.array_equal(ofp4.unpack_nibbles(packed), q_ref)
