"""Bit-exact GEMM parity on exact-arithmetic inputs, for every kernel family.

Activations are small integers, weights are E2M1 codes (INT4: nibbles with
integral zero points) times power-of-two group scales in [2^-4, 2^-1].
Every product and every partial sum is then a multiple of 2^-5 (INT4: 2^-4)
below 2^19, exactly representable in fp32 (as is the decode kernels' INT4
form, integer sums of a * (1024 + q) below 2^19 per group), so the kernel's fp32 sums and the oracle's numpy
fp32 matmul (tests/test_gemm.py:260-263's dequant + matmul) are the same
exact value whatever the summation order, and one fp16 rounding gives the
same bits.  A single dropped, duplicated or mis-indexed k row, column, group
scale or split-K partial changes the output, which the max-abs-rel 1e-2 bar
of the other parity tests cannot see.

Each case is chosen to land on one kernel family (the selection rules of
gemm_dispatch / pair_dispatch / mm_moe_grouped_gemm):
  k_skinny_dual  M <= 8 narrow layers;  k_strip  8 < M <= 16, K*N <= 4096^2;
  k_skinny       M <= 16 wide (no split) and split-K (14336 -> 4096), MT=2 for
                 17..32 rows;  k_prefill2 M > 32 with K % 64 == 0 (and its
                 split-K reduce when the grid is small);  k_prefill  N % 8 != 0
                 or K % 64 != 0;  row-packed and [N, K/g]-scale variants;
                 multi (QKV); gate/up pair (act=0, no SwiGLU rounding);
                 k_moe_grouped and k_moe_prefill.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from gpu_helpers import announce, to_dev, to_np
from oracle import fp4 as ofp4

pytestmark = pytest.mark.gpu


def _exact_fp4(rng, K, N, g):
    """Random E2M1 codes and power-of-two scales in [2^-4, 2^-1] -> (packed [K/8, N], scales)."""
    codes = rng.integers(0, 16, (K, N)).astype(np.uint8)
    scales = (2.0 ** rng.integers(-4, 0, (K // g, N))).astype(np.float16)
    return ofp4.pack_nibbles(codes), scales


def _exact_u4(rng, K, N, g):
    q = rng.integers(0, 16, (K, N)).astype(np.uint8)
    scales = (2.0 ** rng.integers(-4, 0, (K // g, N))).astype(np.float16)
    zeros = rng.integers(0, 16, (K // g, N)).astype(np.float16)
    return ofp4.pack_nibbles(q), scales, zeros


def _acts(rng, M, K):
    return rng.integers(-3, 4, (M, K)).astype(np.float16)


def _bits(x) -> np.ndarray:
    return np.asarray(x, np.float16).view(np.uint16)


def _same(out: torch.Tensor, ref: np.ndarray):
    o = to_np(out)
    assert o.shape == ref.shape
    bad = np.nonzero(_bits(o) != _bits(ref))
    assert bad[0].size == 0, (f"{bad[0].size} outputs differ, first at {bad[0][0]},{bad[1][0]}: "
                              f"{o[bad[0][0], bad[1][0]]} vs {ref[bad[0][0], bad[1][0]]}")


DENSE = [
    # (M, K, N, g, family)
    (1, 4096, 6144, 128, "k_skinny_dual (qkv)"),
    (8, 4096, 4096, 128, "k_skinny_dual (small layer)"),
    (5, 4160, 3076, 64, "k_skinny_dual ragged"),
    (12, 4096, 4096, 128, "k_strip"),
    (16, 2048, 2048, 32, "k_strip g=32"),
    (1, 4096, 28672, 128, "k_skinny unsplit"),
    (1, 14336, 4096, 128, "k_skinny split-K"),
    (13, 14336, 4096, 64, "k_skinny split-K M=13"),
    (24, 4096, 28672, 128, "k_skinny MT=2, 128-column blocks"),
    (12, 4096, 28672, 64, "k_skinny MT=1, 128-column blocks"),
    (32, 4096, 6144, 128, "k_skinny MT=2 split-K, 64-column blocks"),
    (32, 14336, 4096, 128, "k_skinny MT=2 split-K"),
    (64, 4096, 1024, 128, "k_prefill2 64-row tile"),
    (128, 14336, 4096, 128, "k_prefill2 split-K + reduce"),
    (512, 4096, 14336, 128, "k_prefill2 (cfg4 M=512)"),
    (300, 2048, 1000, 64, "k_prefill2 ragged"),
    (100, 520, 260, 8, "k_prefill (N % 8, K % 64)"),
    (40, 200, 96, 8, "k_prefill (K % 64)"),
    # every tile shape bench.py times, at its full size: config 2 (M = 8, 32)
    # on the four Llama-3-8B layers, config 4 (M = 512, 2048) on both GEMMs
    (8, 4096, 6144, 128, "config 2 qkv M=8"),
    (8, 4096, 28672, 128, "config 2 gate_up M=8"),
    (8, 14336, 4096, 128, "config 2 down M=8"),
    (32, 4096, 4096, 128, "config 2 o M=32"),
    (32, 4096, 28672, 128, "config 2 gate_up M=32"),
    (512, 14336, 4096, 128, "config 4 down M=512"),
    (2048, 4096, 14336, 128, "config 4 up M=2048 (256x256 tiles, two rounds)"),
    (2048, 14336, 4096, 128, "config 4 down M=2048 (128x256 tiles over K=14336)"),
]


@pytest.mark.parametrize("M,K,N,g,family", DENSE)
def test_fp4_gemm_bit_exact(rng, M, K, N, g, family):
    import mmfp4
    packed, scales = _exact_fp4(rng, K, N, g)
    a = _acts(rng, M, K)
    ref = ofp4.gemm_fp4_ref(a, packed, scales, g)
    announce(f"exact fp4 {family} M={M} K={K} N={N} g={g}")
    _same(mmfp4.marlin_gemm_fp4(to_dev(a), to_dev(packed), to_dev(scales), g), ref)


@pytest.mark.parametrize("M,K,N,g,family", [d for d in DENSE if d[0] in (1, 12, 13, 24, 32, 64,
                                                                          128, 100)]
                         + [(16, 4096, 6144, 128, "config 3 qkv M=16"),
                            (16, 4096, 4096, 128, "config 3 o M=16"),
                            (16, 4096, 28672, 128, "config 3 gate_up M=16"),
                            (16, 14336, 4096, 128, "config 3 down M=16"),
                            (2048, 14336, 4096, 128, "INT4 prefill M=2048")])
def test_u4_gemm_bit_exact(rng, M, K, N, g, family):
    import mmfp4
    packed, s, z = _exact_u4(rng, K, N, g)
    a = _acts(rng, M, K)
    ref = ofp4.gemm_u4_ref(a, packed, s, z, g)
    announce(f"exact u4 {family} M={M} K={K} N={N} g={g}")
    _same(mmfp4.marlin_gemm_int4(to_dev(a), to_dev(packed), to_dev(s), to_dev(z), g), ref)


@pytest.mark.parametrize("K,N", [(4096, 14336), (14336, 4096)])
def test_fp4_gemm_bit_exact_m8192_rows(rng, K, N):
    """Config 4 at M = 8192 (256x256 tiles for both GEMMs): the whole output
    is computed on the GPU, and one seeded row of every 32-row block (so every
    row tile and every MFMA row block of it) is checked bit-exactly against the
    oracle.  Output rows depend only on their own activation row."""
    import mmfp4
    M, g = 8192, 128
    packed, scales = _exact_fp4(rng, K, N, g)
    a = _acts(rng, M, K)
    rows = np.arange(0, M, 32) + rng.integers(0, 32, M // 32)
    ref = ofp4.gemm_fp4_ref(a[rows], packed, scales, g)
    announce(f"exact fp4 config 4 M=8192 K={K} N={N} (row subset)")
    out = mmfp4.marlin_gemm_fp4(to_dev(a), to_dev(packed), to_dev(scales), g)
    _same(out[torch.from_numpy(rows).to(out.device)], ref)


@pytest.mark.parametrize("M,K,N,g", [(1, 4096, 6144, 128), (1, 14336, 4096, 128),
                                     (12, 4096, 4096, 64), (4, 4096, 28672, 128),
                                     (17, 4096, 4096, 128), (32, 14336, 4096, 128),
                                     (24, 4096, 28672, 64), (33, 4096, 1024, 128),
                                     (64, 4096, 1024, 128),
                                     (128, 14336, 4096, 128), (300, 2048, 1000, 64),
                                     (512, 4096, 14336, 128), (48, 2880, 1024, 64),
                                     (100, 1408, 528, 64), (1, 2880, 1024, 64),
                                     (5, 896, 4864, 128), (13, 1408, 2048, 64),
                                     (24, 2880, 516, 64), (32, 1408, 8192, 128),
                                     (1, 4096, 4096, 32), (9, 1440, 1024, 32),
                                     (17, 2048, 520, 32), (32, 14336, 4096, 32)])
def test_rowpacked_and_mmfp4_bit_exact(rng, M, K, N, g):
    """Row-packed words (both scale layouts) and Marlin words with [N, K/g]
    scales: the two-slab and skinny in-place variants (M <= 32, one and two
    row blocks, split-K) and the pipelined prefill kernel on row-packed words
    (M > 32: 64-, 128- and 256-row tiles, split-K, ragged N), and K % 256 != 0
    (rounds overhanging K) on both."""
    import mmfp4
    packed, scales = _exact_fp4(rng, K, N, g)
    a = _acts(rng, M, K)
    ref = ofp4.gemm_fp4_ref(a, packed, scales, g)
    da = to_dev(a)
    rows = to_dev(np.ascontiguousarray(packed.T))
    announce(f"exact row-packed / mmfp4 M={M} K={K} N={N} g={g}")
    _same(mmfp4.mmfp4_gemm_rowpacked(da, rows, to_dev(scales), g), ref)
    _same(mmfp4.mmfp4_gemm_rowpacked(da, rows, to_dev(np.ascontiguousarray(scales.T)), g), ref)
    _same(mmfp4.mmfp4_gemm(da, to_dev(packed), to_dev(np.ascontiguousarray(scales.T)), g), ref)


@pytest.mark.parametrize("M", [1, 12, 48])
def test_multi_qkv_bit_exact(rng, M):
    import mmfp4
    K, g = 4096, 128
    mats = [_exact_fp4(rng, K, n, g) for n in (4096, 1024, 1024)]
    a = _acts(rng, M, K)
    announce(f"exact qkv M={M}")
    outs = mmfp4.mmfp4_fused_qkv(to_dev(a), *[to_dev(t) for m in mats for t in m], g)
    for o, (p, s) in zip(outs, mats):
        _same(o, ofp4.gemm_fp4_ref(a, p, s, g))


@pytest.mark.parametrize("M", [1, 24, 256, 2048])
def test_gate_up_pair_bit_exact(rng, M):
    """Pair mode without the SwiGLU (act=0): [x @ Wg | x @ Wu], on Marlin
    and on row-packed words."""
    import mmfp4
    K, N, g = 4096, 3072, 128
    gp, gs = _exact_fp4(rng, K, N, g)
    up, us = _exact_fp4(rng, K, N, g)
    a = _acts(rng, M, K)
    ref = np.concatenate([ofp4.gemm_fp4_ref(a, gp, gs, g), ofp4.gemm_fp4_ref(a, up, us, g)], 1)
    announce(f"exact gate/up pair M={M}")
    _same(mmfp4.fused_gate_up_gemm(to_dev(a), to_dev(gp), to_dev(gs), to_dev(up), to_dev(us), g),
          ref)
    # the same pair on row-packed words, read in place (act=0 through the C ABI)
    from mmfp4 import _lib
    da = to_dev(a)
    rg, ru = to_dev(np.ascontiguousarray(gp.T)), to_dev(np.ascontiguousarray(up.T))
    dgs, dus = to_dev(gs), to_dev(us)
    out = torch.empty((M, 2 * N), dtype=torch.float16, device="cuda")
    ws = _lib.workspace(out.device, int(_lib.load().mm_gemm_workspace_bytes(M, 2 * N, K)))
    _lib.call("mm_fp4_gate_up_rowpacked", _lib.ptr(da), _lib.ptr(rg), _lib.ptr(dgs),
              _lib.ptr(ru), _lib.ptr(dus), _lib.ptr(out), M, N, K, g, 0, _lib.ptr(ws),
              ws.numel(), _lib.stream_of(da))
    _same(out, ref)


@pytest.mark.parametrize("g", [32, 128])
@pytest.mark.parametrize("K,N,what", [
    (4096, 512, "64-column blocks split along K (MT=1 to 16 rows, MT=2 above)"),
    (2048, 3072, "two-slab to 8 rows, column strips to 16, split MT=2 above"),
    (256, 25600, "64-column blocks unsplit to 8 rows, 128-column blocks above"),
])
def test_decode_every_row_count(rng, K, N, what, g):
    """Every M from 1 to 32 on the decode kernels, FP4 and INT4: the block
    reduction parks only the rows < M of each lane and hands row item
    (block row 16*mt + 4*q + rr) to wave (4*mt + rr) mod NW, so each row count
    exercises a different set of owning waves and masked lanes; g = 32 flushes
    the group scale every 32-k step, g = 128 every fourth."""
    import mmfp4
    packed, scales = _exact_fp4(rng, K, N, g)
    up, us, uz = _exact_u4(rng, K, N, g)
    dp, ds = to_dev(packed), to_dev(scales)
    dup, dus, duz = to_dev(up), to_dev(us), to_dev(uz)
    a_all = _acts(rng, 32, K)
    w = ofp4.dequant_fp4_f32(packed, scales, g)          # gemm_fp4_ref's operand, once
    wu = ofp4.dequant_u4_f32(up, us, uz, g)
    for M in range(1, 33):
        a = a_all[:M]
        announce(f"exact decode rows M={M} K={K} N={N} g={g} ({what})")
        _same(mmfp4.marlin_gemm_fp4(to_dev(a), dp, ds, g),
              (a.astype(np.float32) @ w).astype(np.float16))
        _same(mmfp4.marlin_gemm_int4(to_dev(a), dup, dus, duz, g),
              (a.astype(np.float32) @ wu).astype(np.float16))


@pytest.mark.parametrize("T,k,E,K,N", [(32, 8, 128, 2048, 1536), (32, 8, 128, 768, 2048),
                                       (1024, 8, 128, 2048, 1536), (1024, 8, 128, 768, 2048),
                                       (7, 3, 5, 256, 96)])
def test_grouped_gemm_bit_exact(rng, T, k, E, K, N):
    """Grouped expert GEMM rows (gathered, no activation) at the config-5
    shapes: decode-sized groups (k_moe_grouped) at T=32, prefill-sized
    (k_moe_prefill) at T=1024.  Row r of expert e is fp16(x[token(r)] @ W_e)."""
    import mmfp4
    from mmfp4 import moe_dispatch as md
    g = 128
    parts = [_exact_fp4(rng, K, N, g) for _ in range(E)]
    P = np.stack([p for p, _ in parts])
    S = np.stack([s for _, s in parts])
    x = _acts(rng, T, K)
    ids = np.stack([rng.permutation(E)[:k] for _ in range(T)]).astype(np.int32)
    sidx, offs, _ = md._sort(to_dev(ids), E)
    announce(f"exact grouped T={T} k={k} E={E} K={K} N={N}")
    y = md._grouped(to_dev(x), sidx, offs, True, k, T, to_dev(P), to_dev(S), g, 0)
    s_np = to_np(sidx).astype(np.int64)
    o_np = to_np(offs)
    ref = np.empty((T * k, N), np.float16)
    for e in range(E):
        r0, r1 = o_np[e], o_np[e + 1]
        if r1 > r0:
            ref[r0:r1] = ofp4.gemm_fp4_ref(x[s_np[r0:r1] // k], P[e], S[e], g)
    _same(y, ref)


@pytest.mark.parametrize("M,N", [(1, 1002), (9, 2001), (40, 1001), (300, 523)])
def test_odd_width_bit_exact(rng, M, N):
    """marlin_gemm_fp4 / marlin_gemm_int4 with N % 4 != 0 (the kernels store
    4 adjacent columns per lane): the operator pads a copy and returns the
    first N columns, bit-exact against the oracle."""
    import mmfp4
    K, g = 512, 64
    packed, scales = _exact_fp4(rng, K, N, g)
    a = _acts(rng, M, K)
    announce(f"exact odd width M={M} N={N}")
    out = mmfp4.marlin_gemm_fp4(to_dev(a), to_dev(packed), to_dev(scales), g)
    assert tuple(out.shape) == (M, N) and out.is_contiguous()
    _same(out, ofp4.gemm_fp4_ref(a, packed, scales, g))
    words_u32 = to_dev(packed).view(torch.uint32)         # uint32 words take the same path
    _same(mmfp4.marlin_gemm_fp4(to_dev(a), words_u32, to_dev(scales), g),
          ofp4.gemm_fp4_ref(a, packed, scales, g))
    q, s, z = _exact_u4(rng, K, N, g)
    _same(mmfp4.marlin_gemm_int4(to_dev(a), to_dev(q), to_dev(s), to_dev(z), g),
          ofp4.gemm_u4_ref(a, q, s, z, g))
