"""Accuracy checks in the terms of the reference's tests/test_kernel_accuracy.py
(:102-181): the same M, N, K and group-size grid and batch-shaped inputs,
scored by cosine similarity against dequant-then-matmul.  The reference's
test packs with kernels_core.pack_fp4_weights (a different LUT and scale);
here the library's own quantizer packs, and the reference is the bit-exact
dequant in fp32, so the thresholds are tighter than the reference's 0.999."""

from __future__ import annotations

import pytest
import torch

from gpu_helpers import TOL, announce, max_abs_rel, to_np

pytestmark = pytest.mark.gpu


def _cos(x, y):
    return torch.nn.functional.cosine_similarity(x.float().reshape(-1), y.float().reshape(-1),
                                                 dim=0).item()


@pytest.mark.parametrize("K", [1024, 2048])
@pytest.mark.parametrize("N", [64, 256])
@pytest.mark.parametrize("g", [32, 64])
def test_dequant_fp4_accuracy(K, N, g):
    import mmfp4
    gen = torch.Generator(device="cuda").manual_seed(42)
    w = torch.randn((N, K), generator=gen, device="cuda").half() * 2.0
    p, s = mmfp4.quantize_fp4(w, group_size=g)
    wd = mmfp4.dequant_fp4(p, s, K, N, g)
    announce(f"dequant accuracy K={K} N={N} g={g}")
    # the quantization error of E2M1 itself: cosine of the round trip
    assert _cos(wd, w.t()) > 0.99
    # the kernel against the per-element closed form fp16(E2M1[code] * scale)
    codes = torch.stack([(p >> (4 * i)) & 0xF for i in range(8)], 1).reshape(K, N)
    e2m1 = torch.tensor([0, .5, 1, 1.5, 2, 3, 4, 6, -0., -.5, -1, -1.5, -2, -3, -4, -6],
                        device="cuda")
    ref = (e2m1[codes.long()] * s.float().repeat_interleave(g, 0)).half()
    assert torch.equal(wd.view(torch.int16), ref.view(torch.int16))


@pytest.mark.parametrize("M", [1, 16, 33, 64])
@pytest.mark.parametrize("N", [64, 128])
@pytest.mark.parametrize("K", [512, 1024])
@pytest.mark.parametrize("g", [32, 64])
def test_marlin_gemm_fp4_accuracy(M, N, K, g):
    import mmfp4
    gen = torch.Generator(device="cuda").manual_seed(42)
    a = torch.randn((M, K), generator=gen, device="cuda").half()
    w = torch.randn((N, K), generator=gen, device="cuda").half()
    p, s = mmfp4.quantize_fp4(w, group_size=g)
    ref = a.float() @ mmfp4.dequant_fp4(p, s, K, N, g).float()
    announce(f"gemm accuracy M={M} N={N} K={K} g={g}")
    out = mmfp4.marlin_gemm_fp4(a, p, s, group_size=g)
    assert _cos(out, ref) > 0.99999
    assert max_abs_rel(to_np(out), to_np(ref)) <= TOL


@pytest.mark.parametrize("batch_dims", [(1,), (4,), (2, 8)])
def test_marlin_gemm_fp4_batch_shapes(batch_dims):
    import mmfp4
    N, K, g = 64, 1024, 32
    gen = torch.Generator(device="cuda").manual_seed(7)
    a = torch.randn((*batch_dims, K), generator=gen, device="cuda").half()
    w = torch.randn((N, K), generator=gen, device="cuda").half()
    p, s = mmfp4.quantize_fp4(w, group_size=g)
    announce(f"gemm batch shape {batch_dims}")
    out = mmfp4.marlin_gemm_fp4(a, p, s, g)
    assert out.shape == (*batch_dims, N)
    ref = a.float().reshape(-1, K) @ mmfp4.dequant_fp4(p, s, K, N, g).float()
    assert _cos(out.reshape(-1, N), ref) > 0.99999
