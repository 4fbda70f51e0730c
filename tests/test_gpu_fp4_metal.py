"""GPU parity of the flat-group FP4 surface (FP4Metal, metal_marlin/
fp4_metal.py:71-314) with the oracle: codes and scales bit-exact for f32,
fp16 and bf16 inputs over ragged sizes and group sizes, NaN/inf/-0 and tie
values, dequantize bit-exact, pack_pair, and numpy in -> numpy out."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from gpu_helpers import announce
from oracle import fp4 as ofp4

pytestmark = pytest.mark.gpu


def _same_f32(a: np.ndarray, b: np.ndarray) -> bool:
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32),
                          np.asarray(b, np.float32).view(np.uint32))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("shape,g", [((4096, 4096), 128), ((37, 53), 64), ((1,), 128),
                                     ((3, 5, 7), 32), ((1000,), 1000), ((129,), 1),
                                     ((8192,), 48)])
def test_fp4metal_quantize_dequantize_vs_oracle(dtype, shape, g):
    import mmfp4
    gen = torch.Generator(device="cuda").manual_seed(sum(shape) + g)
    x = (torch.randn(shape, generator=gen, device="cuda") * 0.5).to(dtype)
    announce(f"FP4Metal.quantize {shape} g={g} {dtype}")
    fp4 = mmfp4.FP4Metal()
    assert fp4.available
    codes, scales = fp4.quantize(x, group_size=g)
    assert codes.dtype == torch.uint8 and codes.shape == x.shape and codes.is_cuda
    assert scales.dtype == torch.float32
    xr = x.float().cpu().numpy()
    rc, rs = ofp4.flat_quantize(xr, g)
    assert np.array_equal(codes.cpu().numpy(), rc)
    assert _same_f32(scales.cpu().numpy(), rs)
    deq = fp4.dequantize(codes, scales, group_size=g)
    assert deq.dtype == torch.float32 and deq.shape == x.shape
    assert _same_f32(deq.cpu().numpy(), ofp4.flat_dequantize(rc, rs, g))


def test_fp4metal_special_values_and_numpy_io():
    import mmfp4
    x = np.array([6, -3, 0.25, 0.75, -0.0, 0, 1.25, 5,               # ties, -0
                  1, np.nan, -2, 3, 1, np.inf, -2, 3,                 # NaN group, inf group
                  0, 0, 0, 0, 3e-8, -6e-8, 1e-8, 0,                   # floor
                  1.5, -0.75], np.float32)

    announce("FP4Metal special values")
    codes, scales = mmfp4.FP4Metal().quantize(x, group_size=4)
    assert isinstance(codes, np.ndarray) and isinstance(scales, np.ndarray)
    rc, rs = ofp4.flat_quantize(x, 4)
    assert np.array_equal(codes, rc) and _same_f32(scales, rs)
    deq = mmfp4.FP4Metal().dequantize(codes, scales, group_size=4)
    assert isinstance(deq, np.ndarray)
    assert _same_f32(deq, ofp4.flat_dequantize(rc, rs, 4))
    # module-level convenience functions
    c2, s2 = mmfp4.quantize_fp4_metal(torch.from_numpy(x).cuda(), 4)
    assert np.array_equal(c2.cpu().numpy(), rc)
    d2 = mmfp4.dequantize_fp4_metal(c2, s2, 4)
    assert _same_f32(d2.cpu().numpy(), deq)


def test_fp4metal_pack_pair_and_errors():
    import mmfp4
    rng = np.random.default_rng(3)
    lo = rng.integers(0, 256, (1000,), dtype=np.uint8)
    hi = rng.integers(0, 256, (1000,), dtype=np.uint8)
    announce("FP4Metal.pack_pair")
    fp4 = mmfp4.FP4Metal()
    out = fp4.pack_pair(torch.from_numpy(lo).cuda(), torch.from_numpy(hi).cuda())
    assert out.dtype == torch.uint8
    assert np.array_equal(out.cpu().numpy(), ofp4.pack_pair(lo, hi))
    assert np.array_equal(fp4.pack_pair(lo, hi), ofp4.pack_pair(lo, hi))
    with pytest.raises(ValueError):
        fp4.dequantize(torch.zeros(300, dtype=torch.uint8, device="cuda"),
                       torch.ones(2, device="cuda"), 128)
    with pytest.raises(RuntimeError):
        fp4.quantize(torch.zeros(8), 4)             # host tensor: no CPU path
