"""GPU parity of the fused gate/up operator (one launch over the gate and up
matrices): silu(x @ Wg) * (x @ Wu) and [x @ Wg | x @ Wu], against the fp32
reference built from the bit-exact dequant, on both kernels (decode M <= 32,
prefill M > 32), with and without a K split, and against the oracle on a
small case."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from gpu_helpers import TOL, announce, max_abs_rel, to_dev, to_np
from oracle import fp4 as ofp4

pytestmark = pytest.mark.gpu


def _weights(gen, K, N, g):
    import mmfp4
    w = (torch.randn((N, K), generator=gen, device="cuda") * 0.02).half()
    p, s = mmfp4.quantize_fp4(w, group_size=g)
    return p, s, mmfp4.dequant_fp4(p, s, K, N, g).float()


@pytest.mark.parametrize("M,K,N,g", [(1, 4096, 14336, 128), (5, 1024, 520, 64),
                                     (16, 14336, 512, 128), (17, 2048, 1024, 32),
                                     (32, 4096, 2048, 128), (33, 1024, 512, 128),
                                     (64, 4096, 1024, 64), (200, 2048, 1544, 128),
                                     (512, 4096, 4096, 128), (130, 256, 136, 32),
                                     (48, 200, 128, 8), (40, 1000, 264, 8), (1, 512, 1004, 64),
                                     (24, 1024, 300, 128), (64, 512, 1001, 64)])
def test_gate_up_vs_fp32_reference(M, K, N, g):
    import mmfp4
    gen = torch.Generator(device="cuda").manual_seed(M * 7 + N)
    gp, gs, wg = _weights(gen, K, N, g)
    up, us, wu = _weights(gen, K, N, g)
    x = torch.randn((M, K), generator=gen, device="cuda").half()
    hg, hu = x.float() @ wg, x.float() @ wu
    announce(f"gate_up M={M} K={K} N={N} g={g}")
    out = mmfp4.mmfp4_fused_gate_up_marlin(x, gp, gs, up, us, g)
    ref = torch.nn.functional.silu(hg) * hu
    assert max_abs_rel(to_np(out), to_np(ref)) <= TOL
    pair = mmfp4.fused_gate_up_gemm(x, gp, gs, up, us, g)
    assert tuple(pair.shape) == (M, 2 * N)
    assert max_abs_rel(to_np(pair[:, :N]), to_np(hg)) <= TOL
    assert max_abs_rel(to_np(pair[:, N:]), to_np(hu)) <= TOL
    # Deterministic: a second launch reproduces both outputs bit for bit.
    assert torch.equal(out, mmfp4.mmfp4_fused_gate_up_marlin(x, gp, gs, up, us, g))
    assert torch.equal(pair, mmfp4.fused_gate_up_gemm(x, gp, gs, up, us, g))


@pytest.mark.parametrize("M,K,N,g", [(3, 512, 256, 128), (1, 4096, 14336, 128),
                                     (16, 2048, 1024, 64), (40, 512, 256, 128),
                                     (300, 2048, 1000, 64), (64, 4096, 14336, 128),
                                     (40, 320, 256, 64), (1, 2880, 512, 64),
                                     (24, 1408, 256, 64), (1, 2048, 512, 32),
                                     (20, 1440, 264, 32), (48, 1024, 256, 32)])
def test_gate_up_rowpacked_vs_oracle(rng, M, K, N, g):
    """mmfp4_fused_gate_up on row-packed [N, K/8] weights (the reference's
    documented layout) against the numpy oracle: read in place by the decode
    kernel (M <= 16) and the pipelined prefill kernel (M > 16, including a
    ragged N, a split-K grid and K % 256 != 0); g=32 is read in place up to
    32 rows and transposed per call above."""
    import mmfp4
    wg = rng.normal(0, 0.02, (N, K)).astype(np.float16)
    wu = rng.normal(0, 0.02, (N, K)).astype(np.float16)
    gp, gs = ofp4.quantize_fp4(wg, g)
    up, us = ofp4.quantize_fp4(wu, g)
    x = rng.normal(0, 1, (M, K)).astype(np.float16)
    xf = x.astype(np.float32)
    hg = xf @ ofp4.dequant_fp4_f32(gp, gs, g)
    hu = xf @ ofp4.dequant_fp4_f32(up, us, g)
    ref = hg / (1.0 + np.exp(-hg)) * hu
    announce(f"gate_up row-packed vs oracle M={M} K={K} N={N} g={g}")
    out = mmfp4.mmfp4_fused_gate_up(to_dev(x), to_dev(np.ascontiguousarray(gp.T)), to_dev(gs),
                                    to_dev(np.ascontiguousarray(up.T)), to_dev(us), g)
    assert max_abs_rel(to_np(out), ref) <= TOL


def test_gate_up_errors():
    import mmfp4
    x = torch.zeros((2, 64), dtype=torch.float16, device="cuda")
    p = torch.zeros((8, 16), dtype=torch.int32, device="cuda")
    s = torch.zeros((1, 16), dtype=torch.float16, device="cuda")
    with pytest.raises(ValueError, match="up_packed must match"):
        mmfp4.fused_gate_up_gemm(x, p, s, p[:, :8], s, 64)
    with pytest.raises(ValueError, match="K mismatch"):
        mmfp4.fused_gate_up_gemm(x[:, :32], p, s, p, s, 64)

