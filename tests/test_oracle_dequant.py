"""Pins the oracle's dequantizers against the reference's known-answer tables
(tests/test_dequant.py) and closed forms, independently of the oracle code."""

from __future__ import annotations

import struct

import numpy as np
import pytest

from oracle import fp4 as ofp4

# tests/test_dequant.py:70-87 (FP4_E2M1_BITS): code -> fp16 bit pattern
FP4_E2M1_BITS = {0x0: 0x0000, 0x1: 0x3800, 0x2: 0x3C00, 0x3: 0x3E00, 0x4: 0x4000, 0x5: 0x4200,
                 0x6: 0x4400, 0x7: 0x4600, 0x8: 0x8000, 0x9: 0xB800, 0xA: 0xBC00, 0xB: 0xBE00,
                 0xC: 0xC000, 0xD: 0xC200, 0xE: 0xC400, 0xF: 0xC600}


def _word(codes):
    w = 0
    for i, c in enumerate(codes):
        w |= (c & 0xF) << (4 * i)
    return w


def _deq_words(words, scales, g):
    """Dequantize a 1-column problem: words [K/8], scales [K/g]."""
    p = np.array(words, dtype=np.uint32).reshape(-1, 1)
    s = np.array(scales, dtype=np.float16).reshape(-1, 1)
    return ofp4.dequant_fp4(p, s, g)[:, 0]


def test_e2m1_bit_table():
    out = _deq_words([_word(range(8)), _word(range(8, 16))], [1.0], 16)
    bits = out.view(np.uint16)
    for code in range(16):
        assert bits[code] == FP4_E2M1_BITS[code], code


def test_bitwise_decoder_closed_form():
    # fp16 bits = sign<<15 | (E+14)<<10 | M<<9 for E>0; 0x3800 for the subnormal
    # (tests/test_dequant.py:108-138), built here from the field definitions.
    for code in range(16):
        s, e, m = code >> 3, (code >> 1) & 3, code & 1
        if e == 0:
            bits = (s << 15) | ((14 << 10) if m else 0)
        else:
            bits = (s << 15) | ((e + 14) << 10) | (m << 9)
        assert FP4_E2M1_BITS[code] == bits


@pytest.mark.parametrize("scale", [0.125, 0.25, 0.5, 1.0, 2.0, 4.0, 10.0])
def test_unit_value_scaled(scale):
    # tests/test_dequant.py:839-847
    out = _deq_words([_word([2] * 8)], [scale], 8)
    assert np.all(out == np.float16(1.0 * np.float16(scale)))


def test_zero_scale_gives_zero():
    out = _deq_words([0xFFFFFFFF], [0.0], 8)
    assert np.all(out.astype(np.float32) == 0.0)


def test_large_scale_near_fp16_max():
    # tests/test_dequant.py:857-865: 6 * 5000 = 30000 is representable
    out = _deq_words([_word([7] * 8)], [5000.0], 8)
    assert np.all(out == np.float16(30000.0))


def test_overflow_and_nonfinite_scale():
    # finite f32 product above fp16 max rounds to inf (guard is on the f32
    # value, src/marlin_gemm.metal:130-137); a non-finite scale gives +0.
    out = _deq_words([_word([7] * 8)], [60000.0], 8)
    assert np.all(np.isinf(out))
    for bad in (np.inf, -np.inf, np.nan):
        out = _deq_words([_word(range(8, 16))], [bad], 8)
        assert np.all(out.view(np.uint16) == 0)


def test_group_transition():
    # tests/test_dequant.py:1459-1477
    out = _deq_words([_word([2] * 8)] * 2, [1.0, 10.0], 8)
    assert out[7] == np.float16(1.0) and out[8] == np.float16(10.0)


def test_exhaustive_codes_times_all_fp16_scales():
    """All 16 codes x every finite fp16 scale against one float64 rounding."""
    all_bits = np.arange(0x10000, dtype=np.uint32).astype(np.uint16)
    scales = all_bits.view(np.float16)
    scales = scales[np.isfinite(scales)]
    n = scales.shape[0]
    packed = np.tile(np.array([[_word(range(8))], [_word(range(8, 16))]], dtype=np.uint32), (1, n))
    out = ofp4.dequant_fp4(packed, scales.reshape(1, n), 16)
    e2m1 = np.array([0, .5, 1, 1.5, 2, 3, 4, 6, -0.0, -.5, -1, -1.5, -2, -3, -4, -6])
    exp = (e2m1[:, None] * scales.astype(np.float64)[None, :]).astype(np.float16)
    assert np.array_equal(out.view(np.uint16), exp.view(np.uint16))


# ---------------------------------------------------------------- INT4
def _fp16_bits(b):
    return np.frombuffer(struct.pack("<H", b), dtype=np.float16)[0]


def test_magic_bias_identity():
    # tests/test_dequant.py:162-169, 1117: (0x6400 | q) - 1024.0 == q
    bias = _fp16_bits(0x6400)
    assert float(bias) == 1024.0
    for q in range(16):
        assert float(np.float16(_fp16_bits(0x6400 | q) - bias)) == q


def test_u4_bulk_known_answer():
    # ref_dequant_u4_bulk, tests/test_dequant.py:206-221, for one packed word
    rng = np.random.default_rng(7)
    for _ in range(20):
        q = rng.integers(0, 16, 8)
        s = np.float16(rng.uniform(0.01, 2.0))
        z = np.float16(rng.integers(0, 16))
        p = np.array([[_word(q)]], dtype=np.uint32)
        out = ofp4.dequant_u4(p, np.array([[s]]), np.array([[z]]), 8)[:, 0]
        exp = np.array([np.float16((np.float16(v) - z) * s) for v in q], dtype=np.float16)
        assert np.array_equal(out.view(np.uint16), exp.view(np.uint16))


def test_u4_exhaustive_integral_zero_points():
    rng = np.random.default_rng(3)
    scales = rng.uniform(1e-4, 4.0, 64).astype(np.float16)
    zs = np.arange(-3, 19, dtype=np.float16)
    for s in scales:
        for z in zs:
            p = np.array([[_word(range(8))], [_word(range(8, 16))]], dtype=np.uint32)
            out = ofp4.dequant_u4(p, np.array([[s]]), np.array([[z]]), 16)[:, 0]
            exp = ((np.arange(16, dtype=np.float64) - float(z)) * float(s)).astype(np.float16)
            assert np.array_equal(out.view(np.uint16), exp.view(np.uint16))


def test_u4_zero_clamp():
    p = np.array([[_word([0] * 8)]], dtype=np.uint32)
    out = ofp4.dequant_u4(p, np.array([[1.0]]), np.array([[300.0]]), 8)
    assert np.all(out == np.float16(-127.0))
