"""Seeded random shapes, bit-exact against the oracle, across the GEMM entry
points: Marlin-layout FP4 (every kernel family by M, K, N and group size),
INT4, row-packed words with either scale layout, Marlin words with [N, K/g]
scales, and the gate/up pair (act=0) on Marlin and row-packed words.

Inputs are exact-arithmetic (small integer activations, E2M1 codes or INT4
nibbles with integral zero points, power-of-two group scales; INT4 group
sizes up to 128 keep the decode kernels' a * (1024 + q) sums below 2^19), so
every sum is exact in fp32 whatever the order and the single fp16 rounding
gives the oracle's bits.  Shapes the entry points refuse by contract (N % 8
for M > 32, row-packed group sizes) are skipped."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from gpu_helpers import announce, to_dev, to_np
from oracle import fp4 as ofp4

pytestmark = pytest.mark.gpu

MS = [1, 2, 3, 5, 8, 9, 13, 16, 17, 23, 32, 33, 47, 64, 100, 129, 200, 300]


def _same(out, ref) -> bool:
    return np.array_equal(to_np(out).view(np.uint16), np.asarray(ref, np.float16).view(np.uint16))


def _fp4(rng, K, N, g):
    return (ofp4.pack_nibbles(rng.integers(0, 16, (K, N)).astype(np.uint8)),
            (2.0 ** rng.integers(-4, 0, (K // g, N))).astype(np.float16))


def _case(rng, kind):
    M = int(rng.choice(MS))
    g = int(rng.choice({"fp4": [8, 32, 64, 128, 256], "u4": [32, 64, 128],
                        "rowp": [32, 64, 128, 256], "pair": [32, 64, 128, 256]}[kind]))
    K = g * int(rng.integers(1, max(2, 4096 // g) + 1))
    N = 8 * int(rng.integers(1, 600))
    if kind in ("fp4", "rowp") and rng.random() < 0.3:
        N -= 4                                   # N % 8 == 4 (decode sizes take it)
    return M, K, N, g


@pytest.mark.parametrize("seed", range(6))
def test_exact_fuzz(seed):
    import mmfp4
    from mmfp4 import _lib
    rng = np.random.default_rng(1000 + seed)
    ran = 0
    for case in range(40):
        kind = ["fp4", "u4", "rowp", "pair"][case % 4]
        M, K, N, g = _case(rng, kind)
        a = rng.integers(-3, 4, (M, K)).astype(np.float16)
        announce(f"exact fuzz seed={seed} case={case} {kind} M={M} K={K} N={N} g={g}")
        if kind == "fp4":
            p, s = _fp4(rng, K, N, g)
            ref = ofp4.gemm_fp4_ref(a, p, s, g)
            dp, ds = to_dev(p), to_dev(s)
            assert _same(mmfp4.marlin_gemm_fp4(to_dev(a), dp, ds, g), ref), (M, K, N, g)
        elif kind == "u4":
            p = ofp4.pack_nibbles(rng.integers(0, 16, (K, N)).astype(np.uint8))
            s = (2.0 ** rng.integers(-4, 0, (K // g, N))).astype(np.float16)
            z = rng.integers(0, 16, (K // g, N)).astype(np.float16)
            ref = ofp4.gemm_u4_ref(a, p, s, z, g)
            dp, ds, dz = to_dev(p), to_dev(s), to_dev(z)
            assert _same(mmfp4.marlin_gemm_int4(to_dev(a), dp, ds, dz, g), ref), (M, K, N, g)
        elif kind == "rowp":
            if not mmfp4.rowpacked_gemm_supported(M, N, K, g):
                continue
            p, s = _fp4(rng, K, N, g)
            ref = ofp4.gemm_fp4_ref(a, p, s, g)
            da, rows, dp = to_dev(a), to_dev(np.ascontiguousarray(p.T)), to_dev(p)
            ds, dst = to_dev(s), to_dev(np.ascontiguousarray(s.T))
            assert _same(mmfp4.mmfp4_gemm_rowpacked(da, rows, ds, g), ref), (M, K, N, g)
            if N != K // g:                      # [N, K/g] unambiguous
                assert _same(mmfp4.mmfp4_gemm_rowpacked(da, rows, dst, g), ref), (M, K, N, g)
                assert _same(mmfp4.mmfp4_gemm(da, dp, dst, g), ref), (M, K, N, g)
        else:
            gp, gs = _fp4(rng, K, N, g)
            up, us = _fp4(rng, K, N, g)
            ref = np.concatenate([ofp4.gemm_fp4_ref(a, gp, gs, g),
                                  ofp4.gemm_fp4_ref(a, up, us, g)], 1)
            da = to_dev(a)
            dgp, dgs, dup, dus = to_dev(gp), to_dev(gs), to_dev(up), to_dev(us)
            assert _same(mmfp4.fused_gate_up_gemm(da, dgp, dgs, dup, dus, g), ref), (M, K, N, g)
            if mmfp4.rowpacked_gemm_supported(M, N, K, g) and N % 8 == 0:
                rg, ru = to_dev(np.ascontiguousarray(gp.T)), to_dev(np.ascontiguousarray(up.T))
                out = torch.empty((M, 2 * N), dtype=torch.float16, device="cuda")
                ws = _lib.workspace(out.device,
                                    int(_lib.load().mm_gemm_workspace_bytes(M, 2 * N, K)))
                _lib.call("mm_fp4_gate_up_rowpacked", _lib.ptr(da), _lib.ptr(rg), _lib.ptr(dgs),
                          _lib.ptr(ru), _lib.ptr(dus), _lib.ptr(out), M, N, K, g, 0,
                          _lib.ptr(ws), ws.numel(), _lib.stream_of(da))
                assert _same(out, ref), (M, K, N, g, "rowpacked")
        ran += 1
    assert ran >= 30
