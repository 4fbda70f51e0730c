"""Pins the oracle's fp32 GEMM and MoE composition against closed forms,
brute force and the known-answer cases of the reference's tests."""

from __future__ import annotations

import numpy as np
import pytest

from oracle import fp4 as ofp4
from oracle import moe as omoe


def _rand_quant(rng, k, n, g):
    w = rng.normal(0, 0.02, (n, k)).astype(np.float16)
    return ofp4.quantize_fp4(w, g)


def test_gemm_brute_force_tiny(rng):
    a = rng.normal(0, 1, (3, 64)).astype(np.float16)
    packed, scales = _rand_quant(rng, 64, 16, 32)
    out = ofp4.gemm_fp4_ref(a, packed, scales, 32)
    e2m1 = [0, .5, 1, 1.5, 2, 3, 4, 6, -0.0, -.5, -1, -1.5, -2, -3, -4, -6]
    exp = np.zeros((3, 16))
    for m in range(3):
        for n in range(16):
            acc = 0.0
            for k in range(64):
                code = (int(packed[k // 8, n]) >> (4 * (k % 8))) & 0xF
                acc += float(a[m, k]) * e2m1[code] * float(scales[k // 32, n])
            exp[m, n] = acc
    assert np.max(np.abs(out.astype(np.float64) - exp)) <= 1e-3 * np.max(np.abs(exp))


def test_gemm_zero_input_and_linearity(rng):
    packed, scales = _rand_quant(rng, 256, 64, 128)
    assert np.all(ofp4.gemm_fp4_ref(np.zeros((2, 256), np.float16), packed, scales, 128) == 0)
    a = rng.normal(0, 1, (2, 256)).astype(np.float16)
    b = rng.normal(0, 1, (2, 256)).astype(np.float16)
    f = lambda x: ofp4.dequant_fp4_f32(packed, scales, 128).T @ x.T  # noqa: E731
    lhs = f((a.astype(np.float32) + b.astype(np.float32)))
    assert np.allclose(lhs, f(a.astype(np.float32)) + f(b.astype(np.float32)), rtol=1e-5,
                       atol=1e-5)


def test_gemm_large_k_all_ones():
    # tests/test_gemm.py:531-556: K = 32768, all-ones A and weights -> K * s
    K, N = 32768, 8
    packed = np.full((K // 8, N), 0x22222222, dtype=np.uint32)     # code 2 = 1.0
    scales = np.full((K // 128, N), 0.5, dtype=np.float16)
    out = ofp4.gemm_fp4_ref(np.ones((1, K), np.float16), packed, scales, 128)
    assert np.all(out == np.float16(K * 0.5))


def test_group_tokens_known_answers():
    # tests/test_moe.py:78-140
    ids = np.array([[0, 2], [1, 2], [0, 1]])
    s, off, inv = omoe.group_tokens_by_expert(ids, 3)
    assert list(np.diff(off)) == [2, 2, 2]
    flat = ids.reshape(-1)
    assert np.all(np.diff(flat[s]) >= 0)
    assert np.array_equal(s[inv], np.arange(6))
    assert list(s) == [0, 4, 2, 5, 1, 3]          # stable: ascending flat index
    _, off, _ = omoe.group_tokens_by_expert(np.array([[0], [2]]), 4)
    assert list(np.diff(off)) == [1, 0, 1, 0]
    _, off, _ = omoe.group_tokens_by_expert(np.array([[0, 1], [0, 2], [0, 1], [0, 2]]), 3)
    assert list(np.diff(off)) == [4, 2, 2]


def test_group_tokens_matches_stable_argsort(rng):
    ids = rng.integers(0, 16, (50, 4))
    s, off, inv = omoe.group_tokens_by_expert(ids, 16)
    assert np.array_equal(s, np.argsort(ids.reshape(-1), kind="stable"))


def test_combine_of_ones(rng):
    ids = rng.integers(0, 8, (10, 3))
    s, off, inv = omoe.group_tokens_by_expert(ids, 8)
    p = rng.random((10, 3)).astype(np.float32)
    out = omoe.combine(np.ones((30, 4), np.float16), p, s, 10, 3)
    assert np.allclose(out, p.sum(axis=1, keepdims=True))


def test_moe_forward_against_composed_pipeline(rng):
    E, T, k, H, I, g = 4, 6, 2, 128, 64, 32
    gu = [_rand_quant(rng, H, 2 * I, g) for _ in range(E)]
    dn = [_rand_quant(rng, I, H, g) for _ in range(E)]
    gup = np.stack([p for p, _ in gu]); gus = np.stack([s for _, s in gu])
    dnp = np.stack([p for p, _ in dn]); dns = np.stack([s for _, s in dn])
    x = rng.normal(0, 1, (T, H)).astype(np.float16)
    ids, probs = omoe.router_topk(rng.normal(0, 1, (T, E)), k)
    ref = omoe.moe_forward_ref(x, gup, gus, dnp, dns, ids, probs, g)
    # composed: sort -> gather -> per-expert MLP -> combine
    s, off, inv = omoe.group_tokens_by_expert(ids, E)
    xs = omoe.gather_for_experts(x, s, k)
    y = np.zeros((T * k, H), np.float32)
    for e in range(E):
        if off[e + 1] > off[e]:
            y[off[e]:off[e + 1]] = omoe.expert_mlp_ref(xs[off[e]:off[e + 1]], gup[e], gus[e],
                                                       dnp[e], dns[e], g)
    out = omoe.combine(y, probs, s, T, k)
    assert np.allclose(out, ref, rtol=1e-4, atol=1e-5)


def test_router_topk_renormalised(rng):
    ids, p = omoe.router_topk(rng.normal(0, 1, (5, 16)), 4)
    assert np.allclose(p.sum(axis=1), 1.0)
    _, p2 = omoe.router_topk(rng.normal(0, 1, (5, 16)), 4, renormalize=False)
    assert np.all(p2.sum(axis=1) < 1.0)
