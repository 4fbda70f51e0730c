"""Quantized linear layers (the reference's `metal_marlin.quantized_linear`,
`QuantizedTensor`, `MarlinLinear` and `MetalKernelLibrary.fp4_gemm/int4_gemm`
surface) over libmmfp4.so."""

from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn as nn

from . import kernels
from .quantize_fp4 import quantize_fp4


@dataclass
class QuantizedTensor:
    """A quantized weight and its metadata (quantized_loader.py:17-27)."""

    data: torch.Tensor
    scales: torch.Tensor
    format: str
    group_size: int
    original_shape: tuple[int, ...]
    needs_hadamard: bool = False
    hadamard_matrix: torch.Tensor | None = None
    zeros: torch.Tensor | None = None


class KernelLibrary:
    """The GEMM methods QuantizedLinear dispatches to
    (metal_dispatch.py:1791-1937, MetalKernelLibrary.fp4_gemm / int4_gemm)."""

    def fp4_gemm(self, input: torch.Tensor, weight: torch.Tensor, scales: torch.Tensor, N: int,
                 K: int, group_size: int = 128) -> torch.Tensor:
        if weight.shape[1] != N or weight.shape[0] * 8 != K:
            raise ValueError(f"weight shape {tuple(weight.shape)} != ({K // 8}, {N})")
        return kernels.marlin_gemm_fp4(input, weight, scales, group_size).to(input.dtype)

    def int4_gemm(self, input: torch.Tensor, weight: torch.Tensor, scales: torch.Tensor, N: int,
                  K: int, group_size: int = 128, zeros: torch.Tensor | None = None) -> torch.Tensor:
        """Asymmetric INT4 GEMM.  Without `zeros` the zero point is the
        constant 8.0, as the reference's int4_gemm dispatches
        (metal_dispatch.py:1899-1908)."""
        if weight.shape[1] != N or weight.shape[0] * 8 != K:
            raise ValueError(f"weight shape {tuple(weight.shape)} != ({K // 8}, {N})")
        if zeros is None:
            zeros = torch.full(scales.shape, 8.0, dtype=torch.float16, device=scales.device)
        return kernels.marlin_gemm_int4(input, weight, scales, zeros, group_size).to(input.dtype)


_LIB: KernelLibrary | None = None


def get_default_library() -> KernelLibrary:
    """metal_dispatch.py:5456 (get_default_library)."""
    global _LIB
    if _LIB is None:
        _LIB = KernelLibrary()
    return _LIB


class QuantizedLinear(nn.Module):
    """Linear layer over FP4/INT4 weights (quantized_linear.py:12-78): flatten,
    optional Hadamard rotation, fused dequant-GEMM, in-place bias add."""

    def __init__(self, quantized_weight: QuantizedTensor, bias: torch.Tensor | None = None):
        super().__init__()
        self.weight_data = quantized_weight.data
        self.weight_scales = quantized_weight.scales
        self.weight_zeros = quantized_weight.zeros
        self.format = quantized_weight.format
        self.group_size = quantized_weight.group_size
        self.out_features, self.in_features = quantized_weight.original_shape
        self.bias = bias
        self.needs_hadamard = quantized_weight.needs_hadamard
        self.hadamard = quantized_weight.hadamard_matrix
        self._lib = get_default_library()

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        batch_shape = x.shape[:-1]
        x_flat = x.reshape(-1, self.in_features)
        if self.needs_hadamard and self.hadamard is not None:
            x_flat = x_flat @ self.hadamard.to(x.device, x.dtype)
        out = self._dispatch_quantized_gemm(x_flat)
        if self.bias is not None:
            out.add_(self.bias)
        return out.view(*batch_shape, self.out_features)

    def _dispatch_quantized_gemm(self, x: torch.Tensor) -> torch.Tensor:
        if self.format == "fp4":
            return self._lib.fp4_gemm(x, self.weight_data, self.weight_scales, self.out_features,
                                      self.in_features, self.group_size)
        if self.format == "int4":
            return self._lib.int4_gemm(x, self.weight_data, self.weight_scales, self.out_features,
                                       self.in_features, self.group_size, self.weight_zeros)
        raise ValueError(f"Unsupported quantized format: {self.format}")


def quantized_linear(x: torch.Tensor, weight_packed: torch.Tensor, scales: torch.Tensor,
                     group_size: int = 32, dtype_config=None) -> torch.Tensor:
    """x @ dequant(weight_packed, scales) with weight_packed in the Marlin
    layout [K/8, N] (metal_marlin.py:389-438).  The reference's docstring
    mentions an N-packed [K, N/8] layout but its body calls marlin_gemm_fp4,
    which takes [K/8, N]; this follows the body.  Output dtype = x.dtype."""
    return kernels.marlin_gemm_fp4(x, weight_packed, scales, group_size).to(x.dtype)


class MarlinLinear:
    """Callable FP4 linear (metal_marlin.py:501-577)."""

    def __init__(self, weight_packed: torch.Tensor, scales: torch.Tensor,
                 bias: torch.Tensor | None = None, group_size: int = 32, dtype_config=None):
        self.weight_packed = weight_packed
        self.scales = scales
        self.bias = bias
        self.group_size = group_size
        self.dtype_config = dtype_config

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        out = quantized_linear(x, self.weight_packed, self.scales, self.group_size)
        if self.bias is not None:
            out.add_(self.bias)
        return out

    @staticmethod
    def from_linear(linear: nn.Linear, quant_type: str = "fp4", group_size: int = 32,
                    device: torch.device | str | None = None) -> "MarlinLinear":
        """Quantize an nn.Linear (weight [out, in]) with quantize_fp4 (Marlin
        layout; the reference uses its N-packed pack_fp4_weights here)."""
        if quant_type != "fp4":
            raise NotImplementedError(
                f"from_linear only supports quant_type='fp4', got {quant_type!r}")
        dev = torch.device(device) if device is not None else (
            linear.weight.device if linear.weight.is_cuda else torch.device("cuda"))
        packed, scales = quantize_fp4(linear.weight.data.to(dev), group_size=group_size)
        bias = linear.bias.data.to(dev, torch.float16) if linear.bias is not None else None
        return MarlinLinear(packed, scales, bias, group_size=group_size)


def dequant_fp4_bulk(packed: torch.Tensor, scales: torch.Tensor, K: int,
                     group_size: int = 128) -> torch.Tensor:
    """[K/8, N] -> [K, N] fp16 (metal_marlin.py:580-612)."""
    k_blocks, N = packed.shape
    if k_blocks != (K + 7) // 8:
        raise ValueError(f"packed.shape[0]={k_blocks} inconsistent with K={K}")
    return kernels.dequant_fp4(packed, scales, K, N, group_size)


def dequant_int4_bulk(packed: torch.Tensor, scales: torch.Tensor, zeros: torch.Tensor, K: int,
                      group_size: int = 128) -> torch.Tensor:
    """[K/8, N] -> [K, N] fp16, (q - z) * s (metal_marlin.py:615-678)."""
    k_blocks, N = packed.shape
    if k_blocks != (K + 7) // 8:
        raise ValueError(f"packed.shape[0]={k_blocks} inconsistent with K={K}")
    return kernels.dequant_int4(packed, scales, zeros, K, N, group_size)
