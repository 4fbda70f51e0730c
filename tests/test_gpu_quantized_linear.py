"""GPU parity of the quantized-linear module layer against the oracle:
QuantizedLinear (metal_marlin/quantized_linear.py:12-78: flatten, optional
Hadamard rotation, fused GEMM, in-place bias add) for fp4 and int4,
MetalKernelLibrary.int4_gemm's constant zero point 8.0
(metal_dispatch.py:1863-1937), quantized_linear, MarlinLinear and
MarlinLinear.from_linear (metal_marlin.py:389-577)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from gpu_helpers import TOL, announce, max_abs_rel, to_dev, to_np
from oracle import fp4 as ofp4

pytestmark = pytest.mark.gpu


def _hadamard(n: int) -> np.ndarray:
    h = np.array([[1.0]])
    while h.shape[0] < n:
        h = np.block([[h, h], [h, -h]])
    return (h / np.sqrt(n)).astype(np.float32)


@pytest.mark.parametrize("M", [1, 6, 48])
@pytest.mark.parametrize("hadamard", [False, True])
def test_quantized_linear_fp4(rng, M, hadamard):
    import mmfp4
    N, K, g = 192, 256, 128
    w = rng.normal(0, 0.02, (N, K)).astype(np.float16)
    p, s = ofp4.quantize_fp4(w, g)
    bias = rng.normal(0, 1, (N,)).astype(np.float16)
    x = rng.normal(0, 1, (2, M, K)).astype(np.float16)
    H = _hadamard(K)
    qt = mmfp4.QuantizedTensor(data=to_dev(p), scales=to_dev(s), format="fp4", group_size=g,
                               original_shape=(N, K), needs_hadamard=hadamard,
                               hadamard_matrix=to_dev(H.astype(np.float16)) if hadamard else None)
    layer = mmfp4.QuantizedLinear(qt, bias=to_dev(bias))
    announce(f"QuantizedLinear fp4 M={M} hadamard={hadamard}")
    y = layer(to_dev(x))
    assert tuple(y.shape) == (2, M, N) and y.dtype == torch.float16
    xf = x.reshape(-1, K)
    if hadamard:
        xf = (xf.astype(np.float32) @ H.astype(np.float16).astype(np.float32)).astype(np.float16)
    ref = ofp4.gemm_fp4_ref(xf, p, s, g).astype(np.float32) + bias.astype(np.float32)
    assert max_abs_rel(to_np(y).reshape(-1, N), ref) <= TOL


@pytest.mark.parametrize("M", [1, 16, 40])
def test_quantized_linear_int4_constant_zero_point(rng, M):
    """The reference's int4 dispatch passes no zero points: int4_gemm fills
    them with 8.0 (metal_dispatch.py:1899-1908).  A QuantizedTensor that
    carries its quantizer's zeros uses them instead."""
    import mmfp4
    N, K, g = 256, 512, 128
    w = rng.normal(0, 0.02, (N, K)).astype(np.float16)
    p, s, z = ofp4.pack_u4_weights(w, g)
    x = rng.normal(0, 1, (M, K)).astype(np.float16)
    bias = rng.normal(0, 1, (N,)).astype(np.float16)
    z8 = np.full_like(s, 8.0)
    announce(f"QuantizedLinear int4 M={M}")
    qt = mmfp4.QuantizedTensor(data=to_dev(p), scales=to_dev(s), format="int4", group_size=g,
                               original_shape=(N, K))
    y = mmfp4.QuantizedLinear(qt, bias=to_dev(bias))(to_dev(x))
    ref8 = ofp4.gemm_u4_ref(x, p, s, z8, g).astype(np.float32) + bias.astype(np.float32)
    assert max_abs_rel(to_np(y), ref8) <= TOL
    lib = mmfp4.get_default_library()
    y2 = lib.int4_gemm(to_dev(x), to_dev(p), to_dev(s), N, K, g)
    assert max_abs_rel(to_np(y2), ofp4.gemm_u4_ref(x, p, s, z8, g)) <= TOL
    qz = mmfp4.QuantizedTensor(data=to_dev(p), scales=to_dev(s), format="int4", group_size=g,
                               original_shape=(N, K), zeros=to_dev(z))
    y3 = mmfp4.QuantizedLinear(qz)(to_dev(x))
    assert max_abs_rel(to_np(y3), ofp4.gemm_u4_ref(x, p, s, z, g)) <= TOL
    # fp4_gemm of the same library
    pf, sf = ofp4.quantize_fp4(w, g)
    y4 = lib.fp4_gemm(to_dev(x), to_dev(pf), to_dev(sf), N, K, g)
    assert max_abs_rel(to_np(y4), ofp4.gemm_fp4_ref(x, pf, sf, g)) <= TOL


def test_quantized_linear_rejects_unknown_format(rng):
    import mmfp4
    qt = mmfp4.QuantizedTensor(data=torch.zeros((32, 64), dtype=torch.int32, device="cuda"),
                               scales=torch.ones((2, 64), dtype=torch.float16, device="cuda"),
                               format="fp8", group_size=128, original_shape=(64, 256))
    with pytest.raises(ValueError, match="Unsupported quantized format"):
        mmfp4.QuantizedLinear(qt)(torch.zeros((1, 256), dtype=torch.float16, device="cuda"))


def test_quantized_linear_function_and_marlin_linear(rng):
    import mmfp4
    N, K, g = 128, 256, 32
    w = rng.normal(0, 0.02, (N, K)).astype(np.float16)
    p, s = ofp4.quantize_fp4(w, g)
    x = rng.normal(0, 1, (2, 3, K)).astype(np.float16)
    bias = rng.normal(0, 1, (N,)).astype(np.float16)
    ref = ofp4.gemm_fp4_ref(x.reshape(-1, K), p, s, g).astype(np.float32)
    announce("quantized_linear / MarlinLinear")
    y = mmfp4.quantized_linear(to_dev(x), to_dev(p), to_dev(s), g)
    assert tuple(y.shape) == (2, 3, N)
    assert max_abs_rel(to_np(y).reshape(-1, N), ref) <= TOL
    ml = mmfp4.MarlinLinear(to_dev(p), to_dev(s), to_dev(bias), group_size=g)
    y2 = ml(to_dev(x))
    assert max_abs_rel(to_np(y2).reshape(-1, N), ref + bias.astype(np.float32)) <= TOL


def test_marlin_linear_from_linear(rng):
    """from_linear quantizes the nn.Linear weight [out, in] with the FP4
    quantizer: same codes as the oracle's quantize_fp4, and the layer output
    matches the oracle GEMM of those codes plus the bias."""
    import mmfp4
    N, K, g = 96, 512, 64
    lin = torch.nn.Linear(K, N, bias=True)
    with torch.no_grad():
        lin.weight.copy_(torch.from_numpy(rng.normal(0, 0.02, (N, K)).astype(np.float32)))
        lin.bias.copy_(torch.from_numpy(rng.normal(0, 1, (N,)).astype(np.float32)))
    lin = lin.half()
    announce("MarlinLinear.from_linear")
    ml = mmfp4.MarlinLinear.from_linear(lin, group_size=g, device="cuda")
    p, s = ofp4.quantize_fp4(lin.weight.detach().numpy(), g)
    assert np.array_equal(to_np(ml.weight_packed).view(np.uint32), p)
    assert np.array_equal(to_np(ml.scales).view(np.uint16), s.view(np.uint16))
    x = rng.normal(0, 1, (5, K)).astype(np.float16)
    y = ml(to_dev(x))
    ref = ofp4.gemm_fp4_ref(x, p, s, g).astype(np.float32) + \
        lin.bias.detach().numpy().astype(np.float32)
    assert max_abs_rel(to_np(y), ref) <= TOL
    with pytest.raises(NotImplementedError):
        mmfp4.MarlinLinear.from_linear(lin, quant_type="int4")
