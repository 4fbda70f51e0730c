"""MMFP4 linear layer on row-packed FP4 weights (metal_marlin/layers/
mmfp4_linear.py:414-478, 549-598, 600-960).

Row-packed means `packed_weights` uint32 [out_features, in_features // 8],
word (n, j) holding inputs 8j..8j+7 of output n (LSB first); scales are
[n_groups, out_features] or [out_features, n_groups].  Both the functional
`mmfp4_gemm` and `MMFP4Linear` read the row-packed words in place
(mm_fp4_gemm_rowpacked): the decode kernels up to 32 rows (group size a
multiple of 32), the pipelined prefill kernel above (group size a multiple
of 64, out_features % 8 == 0), so the layer holds one copy of its weights.  Other shapes run the Marlin-layout kernels
on [in // 8, out] words: the functional form converts per call (as the
reference does on every call); the layer converts once on the device and
keeps the copy as a non-persistent buffer (the reference's
`_kernel_packed_weights`), rebuilt whenever `packed_weights` is written or
replaced.  The reference's M <= 16 path dequantises the whole weight to fp16
and calls F.linear.
"""

from __future__ import annotations

import torch
import torch.nn as nn

from .. import kernels

__all__ = ["MMFP4Linear", "mmfp4_gemm", "rowpacked_to_marlin"]


def _as_words(t: torch.Tensor) -> torch.Tensor:
    if t.dtype in (torch.int32, torch.uint32):
        return t
    if t.dtype == torch.int64:      # word values 0 .. 2^32-1 held in int64
        t = t & 0xFFFFFFFF
        return torch.where(t >= 2**31, t - 2**32, t).to(torch.int32)
    raise TypeError(f"packed weights must be uint32/int32/int64 words, got {t.dtype}")


def rowpacked_to_marlin(packed_weights: torch.Tensor) -> torch.Tensor:
    """[out, in // 8] row-packed words -> [in // 8, out] Marlin layout
    (mmfp4_linear.py:414-478, _rowpacked_to_gpu_layout), on the device."""
    return _as_words(packed_weights).t().contiguous()


def _scales_groups_first(scales: torch.Tensor, out_features: int, n_groups: int) -> torch.Tensor:
    """Scales as [n_groups, out_features] (accepting the transposed layout)."""
    s = scales
    if s.shape[1] != out_features and s.shape[0] == out_features:
        s = s.t()
    if s.shape[1] != out_features:
        raise ValueError("scales second dimension must match out_features; "
                         f"got scales.shape={tuple(s.shape)}, out_features={out_features}")
    if s.shape[0] != n_groups:
        raise ValueError(f"scales first dimension must match n_groups; expected {n_groups}, "
                         f"got {s.shape[0]}")
    return s.to(torch.float16).contiguous()


def mmfp4_gemm(x: torch.Tensor, packed_weights: torch.Tensor, scales: torch.Tensor,
               group_size: int) -> torch.Tensor:
    """x [M, in] @ dequant(row-packed W [out, in // 8])^T -> [M, out] fp16
    (mmfp4_linear.py:549-598)."""
    if x.dim() != 2:
        raise ValueError(f"x must be rank-2 [M, K], got shape={tuple(x.shape)}")
    if packed_weights.dim() != 2:
        raise ValueError("packed_weights must be rank-2 [out, in//8], "
                         f"got shape={tuple(packed_weights.shape)}")
    if x.shape[1] != packed_weights.shape[1] * 8:
        raise ValueError("Input feature mismatch: "
                         f"x.shape[1]={x.shape[1]} vs packed in_features="
                         f"{packed_weights.shape[1] * 8}")
    out_f, in_f = packed_weights.shape[0], packed_weights.shape[1] * 8
    n_groups = -(-in_f // group_size)
    if kernels.rowpacked_gemm_supported(x.shape[0], out_f, in_f, group_size):
        # the row-packed words are read in place, no transpose
        return kernels.mmfp4_gemm_rowpacked(x, _as_words(packed_weights), scales, group_size)
    s = _scales_groups_first(scales, out_f, n_groups)
    return kernels.marlin_gemm_fp4(x, rowpacked_to_marlin(packed_weights), s, group_size)


class MMFP4Linear(nn.Module):
    """y = x @ W^T (+ bias) with row-packed FP4 weights
    (mmfp4_linear.py:600-960).  Same constructor arguments, validation and
    errors as the reference.  `activation` is stored and, as in the
    reference's forward, not applied."""

    def __init__(self, packed_weights: torch.Tensor, scales: torch.Tensor,
                 bias: torch.Tensor | None = None, group_size: int = 128,
                 activation: str | None = None) -> None:
        super().__init__()
        if group_size <= 0:
            raise ValueError(f"group_size must be > 0, got {group_size}")
        if packed_weights.dim() != 2:
            raise ValueError("packed_weights must be rank-2 [out_features, in_features//8], "
                             f"got shape={tuple(packed_weights.shape)}")
        if scales.dim() != 2:
            raise ValueError("scales must be rank-2 [n_groups, out_features], "
                             f"got shape={tuple(scales.shape)}")
        if scales.dtype not in (torch.float16, torch.bfloat16, torch.float32):
            raise ValueError(f"scales must be fp16/bf16/fp32, got dtype={scales.dtype}")
        words = _as_words(packed_weights).contiguous()
        out_f, in_f = int(words.shape[0]), int(words.shape[1] * 8)
        n_groups = -(-in_f // group_size)
        s = _scales_groups_first(scales, out_f, n_groups)
        if bias is not None and (bias.dim() != 1 or bias.shape[0] != out_f):
            raise ValueError(f"bias must be shape [{out_f}], got shape={tuple(bias.shape)}")
        self.register_buffer("packed_weights", words)
        self.register_buffer("scales", s)
        self.register_buffer("bias", None if bias is None else bias.contiguous())
        self.register_buffer("_kernel_packed_weights", None, persistent=False)
        self.register_buffer("_kernel_scales", None, persistent=False)
        self.group_size = int(group_size)
        self.in_features = in_f
        self.out_features = out_f
        self.activation = activation

    def _kernel_weights(self, device: torch.device):
        """(Marlin-layout words, scales or None).  The copy is keyed on the
        source buffers' identity and version counters, so load_state_dict /
        copy_ into packed_weights or scales (or new tensors assigned to them)
        rebuilds it.  With out_features % 4 != 0 the words and scales are
        padded to a multiple of 4 columns here, once, instead of per call."""
        src, sc = self.packed_weights, self.scales
        pad = -self.out_features % 4
        key = (src.data_ptr(), src._version, device) + \
            ((sc.data_ptr(), sc._version) if pad else ())
        kp = self._kernel_packed_weights
        if kp is None or getattr(self, "_kernel_key", None) != key:
            kp = rowpacked_to_marlin(src.to(device))
            self._kernel_scales = None
            if pad:
                kp = torch.nn.functional.pad(kp.view(torch.int32), (0, pad))
                self._kernel_scales = torch.nn.functional.pad(
                    sc.to(device=device, dtype=torch.float16), (0, pad), value=1.0)
            self._kernel_packed_weights = kp
            self._kernel_key = key
        return kp, self._kernel_scales

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if x.shape[-1] != self.in_features:
            raise ValueError(f"Expected input last dim={self.in_features}, got {x.shape[-1]}")
        if not x.is_floating_point():
            raise ValueError(f"x must be a floating tensor, got dtype={x.dtype}")
        x2 = x.reshape(-1, self.in_features)
        if kernels.rowpacked_gemm_supported(x2.shape[0], self.out_features, self.in_features,
                                            self.group_size):
            # row-packed words and [n_groups, out] scales in place
            out = kernels.mmfp4_gemm_rowpacked(x2, self.packed_weights.to(x.device),
                                               self.scales.to(x.device), self.group_size)
        else:
            kp, ks = self._kernel_weights(x.device)
            if ks is None:
                out = kernels.marlin_gemm_fp4(x2, kp, self.scales.to(x.device), self.group_size)
            else:
                out = kernels.marlin_gemm_fp4(x2, kp, ks, self.group_size)[:, :self.out_features]
        if self.bias is not None:
            out = out + self.bias.to(device=out.device, dtype=out.dtype)
        out = out.reshape(*x.shape[:-1], self.out_features)
        return out.to(x.dtype) if out.dtype != x.dtype else out
