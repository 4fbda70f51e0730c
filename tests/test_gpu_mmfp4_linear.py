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
