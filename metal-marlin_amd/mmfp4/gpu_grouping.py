"""Expert grouping manager API (the reference's `metal_marlin.moe.gpu_grouping`
surface), backed by the device counting sort of libmmfp4.so (`mm_moe_sort`).

Reference: metal_marlin/moe/gpu_grouping.py:30-75 (GPUGroupingResult),
:96-152 (group_tokens_by_expert_gpu_optimized), :155-221
(group_tokens_by_expert_fast), :224-280 (group_tokens_by_expert_auto),
:283-410 (GPUExpertGrouping).  Every variant yields the same stable order
(ties keep ascending flat index t*k+slot), so all of them route to the one
sort kernel.  The reference falls back to a CPU sort off its GPU; here the
tensors must live on the ROCm device and a CPU tensor raises.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from .moe_dispatch import (MoEDispatchInfo, group_tokens_by_expert_full,
                           scatter_expert_outputs)

__all__ = [
    "GPUGroupingResult",
    "GPUExpertGrouping",
    "group_tokens_by_expert_gpu_optimized",
    "group_tokens_by_expert_fast",
    "group_tokens_by_expert_auto",
]


@dataclass
class GPUGroupingResult:
    """Indices of one grouping (gpu_grouping.py:30-75); int64 tensors."""

    sorted_token_indices: torch.Tensor
    sorted_expert_indices: torch.Tensor
    expert_offsets: torch.Tensor
    inverse_indices: torch.Tensor
    num_tokens: int
    top_k: int
    num_experts: int

    @property
    def total_assignments(self) -> int:
        return self.num_tokens * self.top_k

    def to_dispatch_info(self) -> MoEDispatchInfo:
        return MoEDispatchInfo(
            sorted_token_indices=self.sorted_token_indices,
            sorted_expert_indices=self.sorted_expert_indices,
            expert_offsets=self.expert_offsets, inverse_indices=self.inverse_indices,
            num_tokens=self.num_tokens, top_k=self.top_k, num_experts=self.num_experts)


def _num_experts(expert_ids: torch.Tensor, num_experts: int | None) -> int:
    # max+1 as the reference infers it; this reads one value back to the host.
    if num_experts is not None:
        return int(num_experts)
    if expert_ids.numel() == 0:
        raise ValueError("num_experts must be given for an empty expert_ids tensor")
    return int(expert_ids.max().item()) + 1


def _group(expert_ids: torch.Tensor, num_experts: int | None) -> GPUGroupingResult:
    info = group_tokens_by_expert_full(expert_ids, _num_experts(expert_ids, num_experts))
    return GPUGroupingResult(
        sorted_token_indices=info.sorted_token_indices,
        sorted_expert_indices=info.sorted_expert_indices,
        expert_offsets=info.expert_offsets, inverse_indices=info.inverse_indices,
        num_tokens=info.num_tokens, top_k=info.top_k, num_experts=info.num_experts)


def group_tokens_by_expert_gpu_optimized(expert_ids: torch.Tensor,
                                         expert_probs: torch.Tensor | None = None,
                                         num_experts: int | None = None) -> GPUGroupingResult:
    """gpu_grouping.py:96-152.  `expert_probs` does not affect the order."""
    del expert_probs
    return _group(expert_ids, num_experts)


def group_tokens_by_expert_fast(expert_ids: torch.Tensor,
                                num_experts: int | None = None) -> GPUGroupingResult:
    """gpu_grouping.py:155-221 (its bincount + one-hot cumsum gives the same
    stable order as the counting sort)."""
    return _group(expert_ids, num_experts)


def group_tokens_by_expert_auto(expert_ids: torch.Tensor,
                                expert_probs: torch.Tensor | None = None,
                                num_experts: int | None = None,
                                force_gpu: bool = False) -> GPUGroupingResult:
    """gpu_grouping.py:224-280.  There is one implementation, on the device,
    so `force_gpu` changes nothing."""
    del expert_probs, force_gpu
    return _group(expert_ids, num_experts)


class GPUExpertGrouping:
    """Grouping manager (gpu_grouping.py:283-410): group, gather the sorted
    activations, scatter-combine the expert outputs."""

    def __init__(self, num_experts: int, device: torch.device | str | None = None,
                 prefer_gpu: bool = True) -> None:
        self.num_experts = int(num_experts)
        self.prefer_gpu = prefer_gpu
        self.device = torch.device("cuda") if device is None else torch.device(device)
        if self.device.type != "cuda":
            raise ValueError(f"GPUExpertGrouping needs a ROCm device, got {self.device}")

    def group(self, expert_ids: torch.Tensor,
              expert_probs: torch.Tensor | None = None) -> GPUGroupingResult:
        del expert_probs
        if expert_ids.device.type != "cuda" or (self.device.index is not None
                                                and expert_ids.device != self.device):
            expert_ids = expert_ids.to(self.device)
        return _group(expert_ids, self.num_experts)

    def gather_activations(self, hidden_states: torch.Tensor,
                           grouping_result: GPUGroupingResult) -> torch.Tensor:
        return hidden_states[grouping_result.sorted_token_indices]

    def scatter_outputs(self, expert_outputs: torch.Tensor, expert_probs: torch.Tensor,
                        grouping_result: GPUGroupingResult) -> torch.Tensor:
        return scatter_expert_outputs(expert_outputs, expert_probs,
                                      grouping_result.to_dispatch_info())
