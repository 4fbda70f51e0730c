"""Operator-style entry points of the reference's dispatch layer for this
path: `metal_dispatch.dispatch_gemm_fp4` (metal_dispatch.py:4045-4181) and
`ops.GemmFp4` (ops/gemm_fp4.py:20-91), over the FP4 kernels.  The `lib`
argument is accepted for signature parity; there is one kernel library."""

from __future__ import annotations

from typing import Any

import torch

from . import kernels

__all__ = ["GemmFp4", "dispatch_gemm_fp4"]


def dispatch_gemm_fp4(lib: Any, A: torch.Tensor, B_packed: torch.Tensor, scales: torch.Tensor,
                      M: int, N: int, K: int, group_size: int = 32,
                      enable_padding: bool | None = None,
                      out: torch.Tensor | None = None) -> torch.Tensor:
    """C[M, N] = A[M, K] @ dequant(B_packed [K/8, N], scales [K/g, N]).
    `enable_padding` is accepted and unused: the kernels take any M and
    N % 4 == 0 without padding.  With `out`, the result is written there."""
    if tuple(A.shape[-2:]) != (M, K) and not (A.dim() == 1 and M == 1 and A.shape[0] == K):
        raise ValueError(f"A shape {tuple(A.shape)} does not match M={M}, K={K}")
    if B_packed.shape[-1] != N:
        raise ValueError(f"B_packed has {B_packed.shape[-1]} columns, expected N={N}")
    C = kernels.marlin_gemm_fp4(A.reshape(M, K), B_packed, scales, group_size)
    if out is not None:
        out.copy_(C)
        return out
    return C


class GemmFp4:
    """Callable FP4 GEMM (ops/gemm_fp4.py:20-91): forward(x [..., K],
    packed_weight [K/8, N], scales [K/g, N], group_size) -> [..., N].
    The output width is packed_weight.shape[-1] (the Marlin column count);
    the reference computes it as shape[-1] * 8."""

    def __init__(self, library: Any | None = None) -> None:
        self._library = library

    def forward(self, x: torch.Tensor, packed_weight: torch.Tensor, scales: torch.Tensor,
                group_size: int = 32) -> torch.Tensor:
        return kernels.marlin_gemm_fp4(x, packed_weight, scales, group_size)

    def __call__(self, *args, **kwargs) -> torch.Tensor:
        return self.forward(*args, **kwargs)
