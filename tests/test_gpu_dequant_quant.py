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
