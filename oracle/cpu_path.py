"""The reference's CPU path, restated in torch-CPU: the timed `cpu_baseline`
of bench.py (test infrastructure; see oracle/__init__.py).

kernels_core.py:1860-1905 (FP4) and :1989-2017 (INT4): an fp32 E2M1 LUT
gather per nibble plane, `scales.repeat_interleave(group_size)`, then
`A_f32 @ B_f32` cast to fp16.  Dequant is redone on every call, as in the
reference.
"""

from __future__ import annotations

import torch

_E2M1 = torch.tensor([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0,
                      -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0], dtype=torch.float32)


def marlin_gemm_fp4_cpu(a: torch.Tensor, b_packed: torch.Tensor, scales: torch.Tensor,
                        group_size: int) -> torch.Tensor:
    """a [M, K] fp16, b_packed [K/8, N] int32/uint32 bits, scales [K/g, N] fp16."""
    m, k = a.shape
    kp, n = b_packed.shape
    if kp * 8 != k:
        raise ValueError(f"Packed K {kp * 8} does not match activations K {k}")
    words = b_packed.view(torch.int32).to(torch.int64) & 0xFFFFFFFF
    s = scales.to(torch.float32).repeat_interleave(group_size, dim=0)
    b = torch.empty((k, n), dtype=torch.float32)
    for j in range(8):
        nib = (words >> (4 * j)) & 0xF
        rows = torch.arange(j, k, 8)
        b[rows, :] = _E2M1[nib] * s[rows, :]
    return (a.to(torch.float32) @ b).to(torch.float16)


def marlin_gemm_int4_cpu(a: torch.Tensor, b_packed: torch.Tensor, scales: torch.Tensor,
                         zeros: torch.Tensor, group_size: int) -> torch.Tensor:
    m, k = a.shape
    kp, n = b_packed.shape
    words = b_packed.view(torch.int32).to(torch.int64) & 0xFFFFFFFF
    s = scales.to(torch.float32).repeat_interleave(group_size, dim=0)
    z = zeros.to(torch.float32).repeat_interleave(group_size, dim=0)
    b = torch.empty((k, n), dtype=torch.float32)
    for j in range(8):
        nib = ((words >> (4 * j)) & 0xF).to(torch.float32)
        rows = torch.arange(j, k, 8)
        b[rows, :] = (nib - z[rows]) * s[rows]
    return (a.to(torch.float32) @ b).to(torch.float16)
