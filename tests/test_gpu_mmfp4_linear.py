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
