"""Pins `oracle.fp4.pack_u4_weights` and `oracle.moe.router_topk` with checks
that the mathematics fixes, independent of the oracle's own formulas:

* pack_u4_weights (metal_marlin/metal_marlin.py:243-262): a float64
  nearest-integer brute force of q away from ties; crafted groups where the
  float32 scale and its fp16 rounding give different q; exact .5 ties of
  w/s + z and of -min/s (np.round is half-to-even); all-positive and
  all-negative groups, whose zero point falls outside [0, 15] and is kept.
* router_topk (metal_marlin/moe_dispatch.py:99-151): a float64 per-row
  softmax with an explicit descending sort, ties to the lower expert id,
  compared exactly on the ids.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import fp4 as ofp4
from oracle import moe as omoe


def _half_even(x: np.ndarray) -> np.ndarray:
    """Round half to even by hand in float64 (no np.round)."""
    f = np.floor(x)
    d = x - f
    up = (d > 0.5) | ((d == 0.5) & (np.mod(f, 2) == 1))
    return f + up


def _group(values, n_rows: int = 8) -> np.ndarray:
    """One quantization group of `n_rows` values in column 0 -> [N=1, K] weights."""
    v = np.asarray(values, dtype=np.float64)
    assert v.size == n_rows
    return v.astype(np.float16).reshape(1, n_rows)


def test_pack_u4_bruteforce_nearest_integer(rng):
    K, N, g = 1024, 96, 128
    w = rng.normal(0, 0.02, (N, K)).astype(np.float16)
    packed, s16, z16 = ofp4.pack_u4_weights(w, g)
    q = ofp4.unpack_nibbles(packed).astype(np.int64)            # [K, N]
    wk = w.T.astype(np.float64).reshape(K // g, g, N)
    mn, mx = wk.min(axis=1), wk.max(axis=1)
    # s = f32((max - min) / 15): (max - min) of two fp16 values is exact in f64
    s32 = np.maximum(((mx - mn) / 15.0).astype(np.float32), np.float32(1e-7)).astype(np.float64)
    assert np.array_equal(s16.view(np.uint16), s32.astype(np.float16).view(np.uint16))
    z = _half_even((-mn / s32))
    assert np.array_equal(z16.astype(np.float64), z)
    t = wk / s32[:, None, :] + z[:, None, :]
    frac = np.abs(t - np.floor(t) - 0.5)
    far = frac > 1e-3                                           # away from ties
    expect = np.clip(np.floor(t + 0.5), 0, 15)
    got = q.reshape(K // g, g, N)
    assert far.mean() > 0.99
    assert np.array_equal(got[far], expect[far])


def test_pack_u4_uses_f32_scale_not_fp16():
    # range 1.5 + 2^-10 -> s32 = 0.100065..., fp16(s32) = 0.10004...: values
    # such as w = 0.4502 put w/s32 and w/fp16(s) either side of a .5 boundary
    lo = 0.0
    hi = 1.5 + 2.0 ** -10
    s32 = np.float32(np.float32(hi - lo) / np.float32(15.0))
    s16 = np.float32(np.float16(s32))
    assert s32 != s16
    # search fp16 values w in (lo, hi) whose q differs under the two scales
    cand = np.arange(np.float16(0.01).view(np.uint16), np.float16(1.5).view(np.uint16),
                     dtype=np.uint16).view(np.float16).astype(np.float32)
    q32 = np.round(cand / s32)
    q16 = np.round(cand / s16)
    diff = cand[q32 != q16]
    assert diff.size > 0
    vals = ([lo, hi] + list(diff[:6].astype(np.float64)) + [0.75, 1.0] * 3)[:8]
    w16 = _group(vals)
    packed, s, z = ofp4.pack_u4_weights(w16, 8)
    q = ofp4.unpack_nibbles(packed)[:, 0].astype(np.float64)
    w64 = w16.astype(np.float64)[0]
    assert z[0, 0] == 0
    expect = np.clip(_half_even(w64 / np.float64(s32)), 0, 15)
    assert np.array_equal(q, expect)
    wrong = np.clip(_half_even(w64 / np.float64(s16)), 0, 15)
    assert not np.array_equal(q, wrong)


def test_pack_u4_half_even_ties():
    # s = 2^-7 exactly: min = -3s (z = 3), max = 12s.  w = 0.5s -> 3.5 -> 4;
    # w = 1.5s -> 4.5 -> 4; w = -0.5s -> 2.5 -> 2; w = 2.5s -> 5.5 -> 6.
    s = 2.0 ** -7
    vals = [-3 * s, 12 * s, 0.5 * s, 1.5 * s, -0.5 * s, 2.5 * s, 0.0, 4.0 * s]
    packed, sc, z = ofp4.pack_u4_weights(_group(vals), 8)
    assert float(sc[0, 0]) == s and float(z[0, 0]) == 3.0
    q = ofp4.unpack_nibbles(packed)[:, 0].tolist()
    assert q == [0, 15, 4, 4, 2, 6, 3, 7]
    # zero-point tie: -min/s = 2.5 -> z = 2 (half-even), not 3
    vals = [-2.5 * s, 12.5 * s, 0.0, s, 2 * s, -s, 3 * s, 5 * s]
    packed, sc, z = ofp4.pack_u4_weights(_group(vals), 8)
    assert float(sc[0, 0]) == s and float(z[0, 0]) == 2.0
    q = ofp4.unpack_nibbles(packed)[:, 0].tolist()
    # w/s + z = -0.5 -> -0 -> 0 (clip), 14.5 -> 14, 2, 3, 4, 1, 5, 7
    assert q == [0, 14, 2, 3, 4, 1, 5, 7]


@pytest.mark.parametrize("sign", [1.0, -1.0])
def test_pack_u4_one_signed_group_keeps_out_of_range_zero(sign):
    # every value of one sign: z = round(-min/s) lies outside [0, 15] and is
    # stored unclipped; q is clipped to [0, 15]
    s = 2.0 ** -8
    base = [4 * s, 4 * s + 15 * s] + [4 * s + k * s for k in (1, 3, 5, 7, 11, 14)]
    vals = [sign * v for v in base]
    w16 = _group(vals)
    packed, sc, z = ofp4.pack_u4_weights(w16, 8)
    assert float(sc[0, 0]) == s
    w = w16.astype(np.float64)[0]
    mn = w.min()
    z_exp = _half_even(np.array([-mn / s]))[0]
    assert float(z[0, 0]) == z_exp
    assert z_exp < 0 if sign > 0 else z_exp > 15
    q = ofp4.unpack_nibbles(packed)[:, 0].astype(np.float64)
    assert np.array_equal(q, np.clip(_half_even(w / s + z_exp), 0, 15))
    # reconstruction with the unclipped zero is exact for these grid values
    assert np.array_equal((q - z_exp) * s, w)


def _router_bruteforce(logits: np.ndarray, k: int, renorm: bool):
    x = np.asarray(logits, dtype=np.float64)
    ids = np.empty((x.shape[0], k), np.int64)
    probs = np.empty((x.shape[0], k), np.float64)
    for r in range(x.shape[0]):
        row = x[r]
        e = np.exp(row - row.max())
        p = e / e.sum()
        # explicit selection: largest value, lowest id among equals
        chosen = []
        for _ in range(k):
            best = -1
            for j in range(row.size):
                if j in chosen:
                    continue
                if best < 0 or p[j] > p[best]:
                    best = j
            chosen.append(best)
        ids[r] = chosen
        probs[r] = p[chosen] / (p[chosen].sum() if renorm else 1.0)
    return ids, probs


@pytest.mark.parametrize("renorm", [True, False])
def test_router_topk_bruteforce_random(rng, renorm):
    T, E, k = 64, 128, 8
    logits = rng.normal(0, 1, (T, E)).astype(np.float16).astype(np.float32)
    ids, p = omoe.router_topk(logits, k, renormalize=renorm)
    bids, bp = _router_bruteforce(logits, k, renorm)
    assert np.array_equal(ids.astype(np.int64), bids)
    assert np.allclose(p, bp, rtol=1e-6, atol=1e-7)
    # descending order within each row
    assert np.all(np.diff(p, axis=1) <= 0)


def test_router_topk_ties_lower_id_first():
    logits = np.array([[1.0, 3.0, 3.0, 2.0, 3.0, 0.0],
                       [0.0, 0.0, 0.0, 0.0, 0.0, 0.0],
                       [5.0, -1.0, 5.0, 5.0, -1.0, 4.0]], np.float32)
    ids, p = omoe.router_topk(logits, 3, renormalize=True)
    bids, bp = _router_bruteforce(logits, 3, True)
    assert ids.tolist() == [[1, 2, 4], [0, 1, 2], [0, 2, 3]]
    assert np.array_equal(ids, bids)
    assert np.allclose(p, bp, rtol=1e-6)
    assert np.allclose(p[1], 1.0 / 3.0)
