"""Write tests/golden/quantize_fp4_vectors.npz: input/output vectors of the
reference's FP4 quantizer (metal_marlin/quantize_fp4.py:131-284, numpy path),
weight-only and with activation_ranges (the calibration-aware branch,
:205-256: percentile group maxima, the smooth_factor blend and the
sqrt(act_scale) attenuation, whose float64 promotion decides scale bits).

The codes the quantizer picks for inputs at or next to E2M1 midpoints depend
on float32 rounding of w / absmax * 6 and on argmin's tie order; no closed form
pins that, so the vectors come from the reference function itself.  This
script is run once, in a container where /root/reference exists; it imports
that one file by path (its Metal branch is an optional import that fails
cleanly without a package) and stores plain arrays only.
"""

from __future__ import annotations

import importlib.util
import sys
from pathlib import Path

import numpy as np

REF = Path("/root/reference/metal_marlin/quantize_fp4.py")
OUT = Path(__file__).resolve().parent / "quantize_fp4_vectors.npz"


def crafted(rows: int, k: int, seed: int) -> np.ndarray:
    """Each 128-long group holds its absmax (6 * a) plus every E2M1 midpoint
    times a, and neighbours one float32 ulp either side."""
    rng = np.random.default_rng(seed)
    mids = np.array([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0], dtype=np.float32)
    w = np.zeros((rows, k), dtype=np.float32)
    for r in range(rows):
        for g0 in range(0, k, 128):
            a = np.float32(rng.uniform(0.001, 0.05))
            vals = [np.float32(6.0) * a]
            for m in mids:
                v = m * a
                vals += [v, np.nextafter(v, np.float32(np.inf)), np.nextafter(v, np.float32(0))]
            vals = np.array(vals, dtype=np.float32)
            vals = np.concatenate([vals, -vals[1:]])
            grp = rng.normal(0.0, 0.5 * a, 128).astype(np.float32)
            grp[: len(vals)] = vals
            w[r, g0:g0 + 128] = grp
    return w


def f64_sensitive(rows: int, k: int, act: float, sf: float, seed: int) -> np.ndarray:
    """Groups whose fp16 scale differs between the reference's float64 blend
    (gmax * np.sqrt(act) is a float64 scalar product) and the same blend done
    in float32: found by search over random group maxima, each placed at
    the group's first element over small N(0, 0.1 * max) values."""
    rng = np.random.default_rng(seed)
    att = np.sqrt(act)
    out = np.empty((rows, k), dtype=np.float32)
    for r in range(rows):
        for g0 in range(0, k, 128):
            while True:
                m = np.float32(rng.uniform(0.01, 0.1))
                f64 = np.float16(((1.0 - sf) * np.float32(m) + sf * (np.float64(m) * att)) / 6.0)
                c = np.float32(np.float32(1.0 - sf) * m) + np.float32(sf) * (m * np.float32(att))
                if f64 != np.float16(np.float32(c) / np.float32(6.0)):
                    break
            grp = rng.normal(0.0, 0.1 * float(m), 128).astype(np.float32)
            grp[0] = m
            out[r, g0:g0 + 128] = grp
    return out


def main() -> None:
    spec = importlib.util.spec_from_file_location("ref_quantize_fp4", REF)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    assert not mod._USE_METAL
    rng = np.random.default_rng(0)
    cases = {
        "w_normal_f16": (rng.normal(0, 0.02, (64, 256)).astype(np.float16), 128),
        "w_crafted_f32": (crafted(16, 256, 1), 128),
        "w_crafted_f16": (crafted(16, 256, 2).astype(np.float16), 128),
        "w_normal_f32_g32": (rng.normal(0, 1.0, (24, 256)).astype(np.float32), 32),
    }
    arrays = {}
    for name, (w, g) in cases.items():
        packed, scales = mod.quantize_fp4(w, group_size=g)
        arrays[f"{name}__w"] = w
        arrays[f"{name}__g"] = np.array(g, dtype=np.int32)
        arrays[f"{name}__packed"] = packed.astype(np.uint32)
        arrays[f"{name}__scales"] = scales.astype(np.float16)
    # Calibration-aware cases: (weights, group, percentile, smooth_factor,
    # input_range or None).  Outlier columns exercise the percentile clip.
    wo = rng.normal(0, 0.02, (48, 512)).astype(np.float32)
    wo[:, ::61] *= 40.0
    cal = {
        "cal_p999_f32": (wo, 128, 99.9, 1.0, None),
        "cal_p90_small_f16": (rng.normal(0, 0.02, (40, 256)).astype(np.float16), 128, 90.0, 0.6,
                              (-0.4, 0.3)),
        "cal_large_sf03_f32": (wo[:, :256].copy(), 64, 100.0, 0.3, (-4.0, 3.0)),
        "cal_small_sf1_g32_f32": (rng.normal(0, 1.0, (24, 256)).astype(np.float32), 32, 100.0,
                                  1.0, (-0.5, 0.5)),
        "cal_p50_g8_f32": (rng.normal(0, 1.0, (16, 64)).astype(np.float32), 8, 50.0, 0.5,
                           (-0.09, 0.01)),
        "cal_p99_crafted_f32": (crafted(16, 256, 3), 128, 99.0, 0.25, (-0.7, 0.2)),
        "cal_p37_quarter_f16": (crafted(8, 256, 4).astype(np.float16), 128, 37.5, 1.0,
                                (-0.25, 0.125)),
        "cal_f64_blend_f32": (f64_sensitive(12, 256, 0.3, 0.6, 5), 128, 100.0, 0.6, (-0.3, 0.1)),
    }
    for name, (w, g, pct, sf, rng_in) in cal.items():
        ar = {"percentile": pct, "smooth_factor": sf}
        if rng_in is not None:
            ar["input_range"] = rng_in
        packed, scales = mod.quantize_fp4(w, group_size=g, activation_ranges=ar)
        arrays[f"{name}__w"] = w
        arrays[f"{name}__g"] = np.array(g, dtype=np.int32)
        arrays[f"{name}__cal"] = np.array([pct, sf, *(rng_in if rng_in else (np.nan, np.nan))],
                                          dtype=np.float64)
        arrays[f"{name}__packed"] = packed.astype(np.uint32)
        arrays[f"{name}__scales"] = scales.astype(np.float16)
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)", file=sys.stderr)


if __name__ == "__main__":
    main()
