"""GPU parity: bulk dequantizers bit-exact with the oracle (which is pinned to
the reference's known answers), quantizers bit-exact with the reference's own
quantizer output (golden vectors) and with the oracle."""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from gpu_helpers import announce, to_dev, to_np
from oracle import fp4 as ofp4

pytestmark = pytest.mark.gpu

GOLD = Path(__file__).resolve().parent / "golden" / "quantize_fp4_vectors.npz"


def _word(codes):
    w = 0
    for i, c in enumerate(codes):
        w |= (c & 0xF) << (4 * i)
    return w


def test_fp4_dequant_all_codes_all_fp16_scales():
    import mmfp4
    bits = np.arange(0x10000, dtype=np.uint32).astype(np.uint16)
    scales = bits.view(np.float16)          # includes inf / nan / subnormals
    n = scales.shape[0]
    packed = np.tile(np.array([[_word(range(8))], [_word(range(8, 16))]], np.uint32), (1, n))
    announce("fp4 dequant exhaustive 16 codes x 65536 scales")
    out = to_np(mmfp4.dequant_fp4(to_dev(packed), to_dev(scales.reshape(1, n)), 16, n, 16))
    ref = ofp4.dequant_fp4(packed, scales.reshape(1, n), 16)
    assert np.array_equal(out.view(np.uint16), ref.view(np.uint16))


@pytest.mark.parametrize("K,N,g", [(128, 64, 32), (1024, 520, 128), (4096, 4096, 128)])
def test_fp4_dequant_random(rng, K, N, g):
    import mmfp4
    packed = rng.integers(0, 2**32, (K // 8, N), dtype=np.uint64).astype(np.uint32)
    scales = rng.normal(0, 0.01, (K // g, N)).astype(np.float16)
    scales.reshape(-1)[:7] = [0.0, -0.0, 6e-8, 1e-5, 60000.0, np.inf, np.nan]
    announce(f"fp4 dequant random K={K} N={N} g={g}")
    out = to_np(mmfp4.dequant_fp4(to_dev(packed), to_dev(scales), K, N, g))
    ref = ofp4.dequant_fp4(packed, scales, g)
    assert np.array_equal(out.view(np.uint16), ref.view(np.uint16))


def test_u4_dequant_exhaustive_and_random(rng):
    import mmfp4
    # every q (column of 16 rows) x zero points x scales
    zs = np.concatenate([np.arange(-3, 19), rng.uniform(-3, 18, 42), [200.0, -300.0]])
    ss = np.concatenate([rng.uniform(1e-4, 4, 30), [0.0, 65504.0, np.inf, np.nan]])
    zz, sc = np.meshgrid(zs.astype(np.float16), ss.astype(np.float16))
    n = zz.size
    packed = np.tile(np.array([[_word(range(8))], [_word(range(8, 16))]], np.uint32), (1, n))
    announce(f"u4 dequant exhaustive n={n}")
    out = to_np(mmfp4.dequant_int4(to_dev(packed), to_dev(sc.reshape(1, n)),
                                   to_dev(zz.reshape(1, n)), 16, n, 16))
    ref = ofp4.dequant_u4(packed, sc.reshape(1, n), zz.reshape(1, n), 16)
    assert np.array_equal(out.view(np.uint16), ref.view(np.uint16))


@pytest.mark.parametrize("name", ["w_normal_f16", "w_crafted_f32", "w_crafted_f16",
                                  "w_normal_f32_g32"])
def test_quantize_fp4_matches_reference_vectors(name):
    import mmfp4
    d = np.load(GOLD)
    w, g = d[f"{name}__w"], int(d[f"{name}__g"])
    announce(f"quantize_fp4 golden {name}")
    packed, scales = mmfp4.quantize_fp4(to_dev(w), group_size=g)
    assert np.array_equal(to_np(packed).view(np.uint32), d[f"{name}__packed"])
    assert np.array_equal(to_np(scales).view(np.uint16), d[f"{name}__scales"].view(np.uint16))


@pytest.mark.parametrize("dtype", [np.float16, np.float32])
def test_quantize_fp4_random_vs_oracle(rng, dtype):
    import mmfp4
    w = rng.normal(0, 0.02, (384, 1024)).astype(dtype)
    announce(f"quantize_fp4 random {dtype.__name__}")
    packed, scales = mmfp4.quantize_fp4(w, group_size=128)     # numpy in -> numpy out
    rp, rs = ofp4.quantize_fp4(w, 128)
    assert np.array_equal(packed, rp)
    assert np.array_equal(scales.view(np.uint16), rs.view(np.uint16))


def test_pack_u4_vs_oracle(rng):
    import mmfp4
    w = rng.normal(0, 0.02, (256, 1024)).astype(np.float16)
    w[0, :128] = 0.0                                   # constant group -> floor scale
    announce("pack_u4_weights random")
    packed, s, z = mmfp4.pack_u4_weights(to_dev(w), group_size=128)
    rp, rs, rz = ofp4.pack_u4_weights(w, 128)
    assert np.array_equal(to_np(packed).view(np.uint32), rp)
    assert np.array_equal(to_np(s).view(np.uint16), rs.view(np.uint16))
    assert np.array_equal(to_np(z).view(np.uint16), rz.view(np.uint16))
    back = to_np(mmfp4.unpack_u4_weights(packed, s, z))
    assert back.shape == (256, 1024)
    assert np.array_equal(back.T.view(np.uint16), ofp4.dequant_u4(rp, rs, rz, 128).view(np.uint16))


CAL_CASES = ["cal_p999_f32", "cal_p90_small_f16", "cal_large_sf03_f32", "cal_small_sf1_g32_f32",
             "cal_p50_g8_f32", "cal_p99_crafted_f32", "cal_p37_quarter_f16", "cal_f64_blend_f32"]


@pytest.mark.parametrize("name", CAL_CASES)
def test_quantize_fp4_calibrated_matches_reference_vectors(name):
    """quantize_fp4(activation_ranges=...) on the GPU: codes and scales
    bit-identical to the reference's calibration-aware branch
    (quantize_fp4.py:205-256) and to the oracle."""
    import mmfp4
    d = np.load(GOLD)
    pct, sf, a_min, a_max = d[f"{name}__cal"]
    ar = {"percentile": float(pct), "smooth_factor": float(sf)}
    if not np.isnan(a_min):
        ar["input_range"] = (float(a_min), float(a_max))
    w, g = d[f"{name}__w"], int(d[f"{name}__g"])
    announce(f"quantize_fp4 calibrated golden {name}")
    packed, scales = mmfp4.quantize_fp4(w, group_size=g, activation_ranges=ar)
    assert np.array_equal(packed, d[f"{name}__packed"])
    assert np.array_equal(scales.view(np.uint16), d[f"{name}__scales"].view(np.uint16))


@pytest.mark.parametrize("dtype", [np.float16, np.float32])
@pytest.mark.parametrize("ar", [{"percentile": 99.5},
                                {"percentile": 12.5, "input_range": (-9.0, 3.0),
                                 "smooth_factor": 0.45},
                                {"percentile": 80.0, "input_range": (-0.37, 0.2),
                                 "smooth_factor": 0.8},
                                {"input_range": (0.0, 0.6)},
                                {"percentile": 100.0, "input_range": (-2.0, 0.5),
                                 "smooth_factor": 0.0}])
def test_quantize_fp4_calibrated_random_vs_oracle(rng, dtype, ar):
    import mmfp4
    w = rng.normal(0, 0.03, (96, 512)).astype(dtype)
    w[:, ::37] *= 30
    w[5, 128:256] = 0                                # an all-zero group: 1e-7 floor
    announce(f"quantize_fp4 calibrated random {dtype.__name__} {ar}")
    packed, scales = mmfp4.quantize_fp4(to_dev(w), group_size=128, activation_ranges=ar)
    rp, rs = ofp4.quantize_fp4_calibrated(w, 128, ar)
    assert np.array_equal(to_np(packed).view(np.uint32), rp)
    assert np.array_equal(to_np(scales).view(np.uint16), rs.view(np.uint16))


def test_quantize_fp4_calibrated_nan_group_and_bad_percentile(rng):
    import mmfp4
    w = rng.normal(0, 0.03, (8, 256)).astype(np.float32)
    w[3, 7] = np.nan
    ar = {"percentile": 90.0, "input_range": (-0.5, 0.5), "smooth_factor": 0.5}
    announce("quantize_fp4 calibrated NaN group")
    with np.errstate(invalid="ignore"):
        rp, rs = ofp4.quantize_fp4_calibrated(w, 128, ar)
    packed, scales = mmfp4.quantize_fp4(w, group_size=128, activation_ranges=ar)
    assert np.isnan(scales[0, 3]) and np.isnan(rs[0, 3])
    assert np.array_equal(np.isnan(scales), np.isnan(rs))
    ok = ~np.isnan(rs)
    assert np.array_equal(scales[ok].view(np.uint16), rs[ok].view(np.uint16))
    assert np.array_equal(packed, rp)
    with pytest.raises(ValueError):
        mmfp4.quantize_fp4(w, group_size=128, activation_ranges={"percentile": 101.0})
    # the weight-only path on the same NaN group: NaN scale, codes 8 (numpy's
    # clip keeps NaN and argmin over all-NaN distances returns index 0)
    with np.errstate(invalid="ignore"):
        rp, rs = ofp4.quantize_fp4(w, 128)
    packed, scales = mmfp4.quantize_fp4(w, group_size=128)
    assert np.array_equal(packed, rp)
    assert np.array_equal(np.isnan(scales), np.isnan(rs))
    assert np.all(ofp4.unpack_nibbles(rp)[:128, 3] == 8)
