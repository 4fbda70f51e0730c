"""GPU parity of the row-packed MMFP4 layer (layers/mmfp4_linear.py:549-960)
against the oracle: both scale layouts, bias, int64 words, 3-D inputs, and
the functional mmfp4_gemm."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from gpu_helpers import TOL, announce, max_abs_rel, to_dev, to_np
from oracle import fp4 as ofp4

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("scales_layout", ["groups_first", "out_first"])
@pytest.mark.parametrize("M", [1, 5, 40])
def test_mmfp4_linear_vs_oracle(rng, scales_layout, M):
    import mmfp4
    out_f, in_f, g = 192, 512, 128
    w = rng.normal(0, 0.02, (out_f, in_f)).astype(np.float16)
    marlin, scales = ofp4.quantize_fp4(w, g)                # [in/8, out], [in/g, out]
    rowpacked = np.ascontiguousarray(marlin.T)               # [out, in/8]
    s = scales if scales_layout == "groups_first" else np.ascontiguousarray(scales.T)
    bias = rng.normal(0, 1, (out_f,)).astype(np.float16)
    x = rng.normal(0, 1, (2, M, in_f)).astype(np.float16)
    ref = np.stack([ofp4.gemm_fp4_ref(x[b], marlin, scales, g) for b in range(2)])
    ref = ref + bias.astype(np.float32)
    announce(f"MMFP4Linear M={M} scales={scales_layout}")
    layer = mmfp4.MMFP4Linear(to_dev(rowpacked.view(np.int32)), to_dev(s), to_dev(bias), g)
    y = layer(to_dev(x))
    assert tuple(y.shape) == (2, M, out_f) and y.dtype == torch.float16
    assert max_abs_rel(to_np(y), ref) <= TOL
    # int64 words (the reference's example builds them that way) give the same result
    layer64 = mmfp4.MMFP4Linear(to_dev(rowpacked.astype(np.int64)), to_dev(s), to_dev(bias), g)
    assert torch.equal(layer64(to_dev(x)), y)
    fn = mmfp4.layers.mmfp4_gemm(to_dev(x[0]), to_dev(rowpacked.view(np.int32)), to_dev(s), g)
    assert max_abs_rel(to_np(fn), ref[0] - bias.astype(np.float32)) <= TOL


def test_mmfp4_linear_errors():
    import mmfp4
    p = torch.zeros((16, 8), dtype=torch.int32, device="cuda")
    with pytest.raises(ValueError, match="n_groups"):
        mmfp4.MMFP4Linear(p, torch.zeros((3, 16), dtype=torch.float16, device="cuda"), None, 32)
    with pytest.raises(ValueError, match="bias must be shape"):
        mmfp4.MMFP4Linear(p, torch.zeros((2, 16), dtype=torch.float16, device="cuda"),
                          torch.zeros(15, device="cuda"), 32)
    layer = mmfp4.MMFP4Linear(p, torch.zeros((2, 16), dtype=torch.float16, device="cuda"),
                              None, 32)
    with pytest.raises(ValueError, match="Expected input last dim"):
        layer(torch.zeros((1, 32), dtype=torch.float16, device="cuda"))


def test_dispatch_gemm_fp4_and_gemmfp4(rng):
    """metal_dispatch.dispatch_gemm_fp4 / ops.GemmFp4 signatures over the same
    kernels, against the oracle; `out=` is filled in place."""
    import mmfp4
    M, K, N, g = 7, 256, 96, 32
    w = rng.normal(0, 0.02, (N, K)).astype(np.float16)
    p, s = ofp4.quantize_fp4(w, g)
    x = rng.normal(0, 1, (M, K)).astype(np.float16)
    ref = ofp4.gemm_fp4_ref(x, p, s, g)
    announce("dispatch_gemm_fp4 / GemmFp4")
    out = torch.empty((M, N), dtype=torch.float16, device="cuda")
    r = mmfp4.dispatch_gemm_fp4(None, to_dev(x), to_dev(p), to_dev(s), M, N, K, g, out=out)
    assert r is out and max_abs_rel(to_np(out), ref) <= TOL
    y = mmfp4.GemmFp4()(to_dev(x[None]), to_dev(p), to_dev(s), g)
    assert tuple(y.shape) == (1, M, N) and max_abs_rel(to_np(y[0]), ref) <= TOL


@pytest.mark.parametrize("M,K,N,g", [(1, 4096, 4096, 128), (4, 14336, 4096, 128),
                                     (16, 4096, 6144, 64), (1, 256, 4, 256), (7, 1024, 100, 128),
                                     (1, 4096, 28672, 128), (3, 2048, 1028, 64),
                                     (2, 4096, 6144, 128), (8, 1024, 3072, 64), (5, 4608, 4100, 128),
                                     (17, 14336, 4096, 128), (40, 4096, 4096, 128),
                                     (300, 2048, 1000, 64), (1024, 4096, 2048, 128)])
def test_rowpacked_gemm_in_place(M, K, N, g):
    """mm_fp4_gemm_rowpacked reads [N, K/8] words and the scales in place, in
    either layout the layer accepts ([K/g, N] canonical, [N, K/g] transposed)
    (layers/mmfp4_linear.py:549-598 without its per-call transpose): parity
    with the fp32 reference of the same weights, including the split-K shape
    14336 -> 4096, and above 16 rows the pipelined prefill kernel on the same
    words.  Both scale layouts give bit-identical results."""
    import mmfp4
    gen = torch.Generator(device="cuda").manual_seed(M * 3 + K + N)
    w = (torch.randn((N, K), generator=gen, device="cuda") * 0.02).half()
    a = torch.randn((M, K), generator=gen, device="cuda").half()
    marlin, scales = mmfp4.quantize_fp4(w, group_size=g)            # [K/8, N], [K/g, N]
    ref = a.float() @ mmfp4.dequant_fp4(marlin, scales, K, N, g).float()
    rows, srows = marlin.t().contiguous(), scales.t().contiguous()   # [N, K/8], [N, K/g]
    announce(f"row-packed gemm M={M} K={K} N={N} g={g}")
    out = mmfp4.mmfp4_gemm_rowpacked(a, rows, srows, g)
    assert max_abs_rel(to_np(out), to_np(ref)) <= TOL
    out_g = mmfp4.mmfp4_gemm_rowpacked(a, rows, scales, g)
    assert torch.equal(out_g.view(torch.int16), out.view(torch.int16))
    # the layer-level functional entry takes this path and agrees
    for sc in (srows, scales):
        fn = mmfp4.layers.mmfp4_gemm(a, rows, sc, g)
        assert torch.equal(fn.view(torch.int16), out.view(torch.int16))


def test_rowpacked_gemm_refuses_unsupported_shapes():
    import mmfp4
    a = torch.zeros((33, 512), dtype=torch.float16, device="cuda")
    rows = torch.zeros((64, 64), dtype=torch.int32, device="cuda")
    s = torch.ones((64, 4), dtype=torch.float16, device="cuda")
    with pytest.raises(ValueError):                          # M > 32 needs N % 8 == 0
        mmfp4.mmfp4_gemm_rowpacked(a, rows[:60], s[:60], 128)
    with pytest.raises(ValueError):                          # M > 32 needs g % 64 == 0
        mmfp4.mmfp4_gemm_rowpacked(a, rows, torch.ones((16, 64), dtype=torch.float16,
                                                       device="cuda"), 32)
    with pytest.raises(ValueError):                          # g % 32 != 0
        mmfp4.mmfp4_gemm_rowpacked(a[:1], rows, torch.ones((32, 64), dtype=torch.float16,
                                                           device="cuda"), 16)


@pytest.mark.parametrize("M,K,N,g", [(1, 4096, 4096, 128), (8, 14336, 4096, 128),
                                     (16, 512, 100, 32), (3, 4096, 6144, 64),
                                     (40, 512, 256, 128), (1, 1024, 8, 128), (24, 2048, 16, 128)])
def test_kernels_mmfp4_gemm_scale_layouts(M, K, N, g):
    """kernels.mmfp4_gemm (kernels_core.py:4804-4812 -> MetalKernels.mmfp4_gemm
    :4550-4633): Marlin-layout words with [K/g, N] scales, the layout the
    reference kernel reads (shaders/mmfp4_gemm.metal:570-588).  [N, K/g]
    scales are accepted when the shape is unambiguous (read in place at decode
    sizes, transposed above); a square tensor (N == K/g: the (1, 1024, 8) and
    (24, 2048, 16) cases) is read as [K/g, N].  Parity with the fp32
    reference, and dequantize_mmfp4 bit-exact with dequant_fp4."""
    import mmfp4
    gen = torch.Generator(device="cuda").manual_seed(M + 5 * K + N)
    w = (torch.randn((N, K), generator=gen, device="cuda") * 0.02).half()
    a = torch.randn((M, K), generator=gen, device="cuda").half()
    p, s = mmfp4.quantize_fp4(w, group_size=g)
    deq = mmfp4.dequant_fp4(p, s, K, N, g)
    ref = a.float() @ deq.float()
    announce(f"kernels.mmfp4_gemm M={M} K={K} N={N} g={g}")
    out = mmfp4.mmfp4_gemm(a, p, s, g)
    assert out.shape == (M, N)
    assert max_abs_rel(to_np(out), to_np(ref)) <= TOL
    assert torch.equal(out, mmfp4.marlin_gemm_fp4(a, p, s, g))
    assert torch.equal(mmfp4.dequantize_mmfp4(p, s, g).view(torch.int16), deq.view(torch.int16))
    if N != K // g:
        st = s.t().contiguous()
        out_t = mmfp4.mmfp4_gemm(a, p, st, g)
        assert max_abs_rel(to_np(out_t), to_np(ref)) <= TOL
        assert torch.equal(mmfp4.dequantize_mmfp4(p, st, g).view(torch.int16),
                           deq.view(torch.int16))
        if M <= 8 and K * N <= 4096 * 6144:
            # The two-slab decode kernel serves both scale layouts with the same
            # summation order: the results must agree bit for bit.
            assert torch.equal(out_t, out)
    else:
        # square: read as [K/g, N]; the transposed tensor is a different matrix
        other = mmfp4.mmfp4_gemm(a, p, s.t().contiguous(), g)
        ref_t = a.float() @ mmfp4.dequant_fp4(p, s.t().contiguous(), K, N, g).float()
        assert max_abs_rel(to_np(other), to_np(ref_t)) <= TOL


def test_mmfp4_gemm_rejects_mismatched_scales():
    import mmfp4
    a = torch.zeros((1, 512), dtype=torch.float16, device="cuda")
    p = torch.zeros((64, 96), dtype=torch.int32, device="cuda")
    with pytest.raises(ValueError, match="neither"):
        mmfp4.mmfp4_gemm(a, p, torch.ones((5, 96), dtype=torch.float16, device="cuda"), 128)


@pytest.mark.parametrize("g", [128, 32])
def test_mmfp4_linear_reloaded_weights_take_effect(rng, g):
    """load_state_dict with new weights changes MMFP4Linear's output at every
    M and matches the oracle of the new weights: g=128 reads the row-packed
    words in place at both sizes; g=32 in place at M=1 and, at M=40 (the
    prefill kernel needs a multiple of 64), through the Marlin-layout copy,
    which must follow writes to packed_weights."""
    import mmfp4
    out_f, in_f = 256, 512
    w1 = rng.normal(0, 0.02, (out_f, in_f)).astype(np.float16)
    w2 = rng.normal(0, 0.02, (out_f, in_f)).astype(np.float16)
    m1, s1 = ofp4.quantize_fp4(w1, g)
    m2, s2 = ofp4.quantize_fp4(w2, g)
    layer = mmfp4.MMFP4Linear(to_dev(np.ascontiguousarray(m1.T).view(np.int32)), to_dev(s1),
                              None, g)
    for M in (1, 40):
        x = rng.normal(0, 1, (M, in_f)).astype(np.float16)
        announce(f"MMFP4Linear reload M={M}")
        y1 = layer(to_dev(x))
        assert max_abs_rel(to_np(y1), ofp4.gemm_fp4_ref(x, m1, s1, g)) <= TOL
        sd = {"packed_weights": to_dev(np.ascontiguousarray(m2.T).view(np.int32)),
              "scales": to_dev(s2)}
        layer.load_state_dict(sd, strict=False)
        y2 = layer(to_dev(x))
        assert max_abs_rel(to_np(y2), ofp4.gemm_fp4_ref(x, m2, s2, g)) <= TOL
        layer.load_state_dict({"packed_weights": to_dev(np.ascontiguousarray(m1.T).view(np.int32)),
                               "scales": to_dev(s1)}, strict=False)


def test_mmfp4_linear_odd_width(rng):
    """out_features % 4 != 0: the layer pads its Marlin-layout copy (and its
    scales) to a multiple of 4 columns once, reuses it across calls, rebuilds
    it when the scales are written, and returns out_features columns that
    match the oracle."""
    import mmfp4
    out_f, in_f, g = 1002, 512, 64
    w = rng.normal(0, 0.02, (out_f, in_f)).astype(np.float16)
    m, s = ofp4.quantize_fp4(w, g)
    layer = mmfp4.MMFP4Linear(to_dev(np.ascontiguousarray(m.T).view(np.int32)), to_dev(s), None, g)
    for M in (1, 40):
        x = rng.normal(0, 1, (M, in_f)).astype(np.float16)
        announce(f"MMFP4Linear odd width M={M}")
        y = layer(to_dev(x))
        assert tuple(y.shape) == (M, out_f)
        assert max_abs_rel(to_np(y), ofp4.gemm_fp4_ref(x, m, s, g)) <= TOL
    kp = layer._kernel_packed_weights
    layer(to_dev(x))
    assert layer._kernel_packed_weights is kp            # reused, not re-padded
    s2 = (s * 2).astype(np.float16)
    layer.load_state_dict({"scales": to_dev(s2)}, strict=False)
    y2 = layer(to_dev(x))
    assert max_abs_rel(to_np(y2), ofp4.gemm_fp4_ref(x, m, s2, g)) <= TOL
