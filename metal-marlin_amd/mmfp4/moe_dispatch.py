"""MoE token grouping, gather, grouped FP4 expert GEMM and weighted combine
(the reference's `metal_marlin.moe_dispatch` and `kernels.moe_expert_gemm_fp4`
surface), on the GPU through libmmfp4.so.

The whole routed-expert pass is one stream of four launches with no host
synchronisation: stable device counting sort -> grouped gate_up GEMM (token
gather + SwiGLU fused) -> grouped down GEMM -> deterministic combine.
"""

from __future__ import annotations

from collections.abc import Sequence
from dataclasses import dataclass

import torch
import torch.nn as nn

from . import _lib


@dataclass
class MoEDispatchInfo:
    """Indexing tensors of a grouped MoE pass (moe_dispatch.py:453-490)."""

    sorted_token_indices: torch.Tensor  # [T*k] token of each sorted assignment
    sorted_expert_indices: torch.Tensor  # [T*k] slot (0..k-1) of each sorted assignment
    expert_offsets: torch.Tensor  # [E+1]
    inverse_indices: torch.Tensor  # [T*k]
    num_tokens: int
    top_k: int
    num_experts: int
    sorted_indices: torch.Tensor | None = None  # [T*k] int32 flat index t*k+slot

    @property
    def total_assignments(self) -> int:
        return self.num_tokens * self.top_k


def _sort(expert_ids: torch.Tensor, num_experts: int):
    """Device counting sort -> (sorted_idx, offsets, inverse), all int32."""
    dev = _lib.require_device(expert_ids)
    if expert_ids.dim() != 2:
        raise ValueError("expert_ids must be [batch, top_k]")
    T, k = expert_ids.shape
    if expert_ids.dtype == torch.int64:
        ids, entry = expert_ids.contiguous(), "mm_moe_sort_i64"
    else:
        ids, entry = expert_ids.to(torch.int32).contiguous(), "mm_moe_sort"
    offsets = torch.empty(num_experts + 1, dtype=torch.int32, device=dev)
    sorted_idx = torch.empty(T * k, dtype=torch.int32, device=dev)
    inverse = torch.empty(T * k, dtype=torch.int32, device=dev)
    _lib.call(entry, _lib.ptr(ids), T, k, num_experts, _lib.ptr(offsets),
              _lib.ptr(sorted_idx), _lib.ptr(inverse), _lib.stream_of(ids))
    return sorted_idx, offsets, inverse


def group_tokens_by_expert(expert_ids: torch.Tensor, num_experts: int):
    """Stable counting sort of the flattened assignments by expert
    (moe_dispatch.py:493-555).  Returns int64 (sorted_indices, expert_offsets
    [E+1], inverse_indices)."""
    s, o, inv = _sort(expert_ids, num_experts)
    return s.to(torch.int64), o.to(torch.int64), inv.to(torch.int64)


def group_tokens_by_expert_full(expert_ids: torch.Tensor, num_experts: int,
                                use_gpu: bool = True) -> MoEDispatchInfo:
    """moe_dispatch.py:726-786.  `use_gpu` is accepted for signature
    compatibility; the sort always runs on the device."""
    T, k = expert_ids.shape
    s, o, inv = _sort(expert_ids, num_experts)
    s64 = s.to(torch.int64)
    return MoEDispatchInfo(
        sorted_token_indices=s64 // k, sorted_expert_indices=s64 % k,
        expert_offsets=o.to(torch.int64), inverse_indices=inv.to(torch.int64),
        num_tokens=T, top_k=k, num_experts=num_experts, sorted_indices=s)


def gather_for_experts(activations: torch.Tensor, dispatch_info: MoEDispatchInfo) -> torch.Tensor:
    """X_sorted = X[sorted_token_indices] (moe_dispatch.py:789-809)."""
    return activations[dispatch_info.sorted_token_indices]


def scatter_expert_outputs(expert_outputs: torch.Tensor, expert_probs: torch.Tensor,
                           dispatch_info: MoEDispatchInfo) -> torch.Tensor:
    """out[t] = sum_j p[t, j] * y[(t, j)], summed in fp32 in slot order
    (moe_dispatch.py:812-925)."""
    dev = _lib.require_device(expert_outputs, expert_probs)
    T, k = dispatch_info.num_tokens, dispatch_info.top_k
    H = expert_outputs.shape[1]
    y = expert_outputs.to(torch.float16).contiguous()
    p = expert_probs.to(torch.float32).contiguous()
    inv = dispatch_info.inverse_indices.to(torch.int32).contiguous()
    out = torch.empty((T, H), dtype=torch.float16, device=dev)
    _lib.call("mm_moe_combine", _lib.ptr(y), _lib.ptr(p), _lib.ptr(inv), T, k, H, _lib.ptr(out),
              _lib.stream_of(y))
    return out if expert_outputs.dtype == torch.float16 else out.to(expert_outputs.dtype)


def compute_expert_load(expert_ids: torch.Tensor, num_experts: int) -> torch.Tensor:
    """Tokens per expert (moe_dispatch.py:930-948)."""
    return torch.bincount(expert_ids.reshape(-1).to(torch.int64), minlength=num_experts)


def compute_load_balancing_loss(expert_probs_pre_topk: torch.Tensor, expert_ids: torch.Tensor,
                                num_experts: int) -> torch.Tensor:
    """Switch-Transformer balance loss E * sum_e f_e P_e (moe_dispatch.py:951-982)."""
    f = compute_expert_load(expert_ids, num_experts).to(torch.float32) / expert_ids.numel()
    return num_experts * (f * expert_probs_pre_topk.mean(dim=0)).sum()


# The one-launch router kernel wins while the gate GEMM is small (decode-sized
# T); above that the GEMM goes to the vendor library (hipBLASLt through
# torch's linear, the same fp16 logits the reference's nn.Linear gives) and
# softmax/top-k to mm_softmax_topk.  Measured on MI355X at E=128, H=2048,
# top-8: T=32 13.0 us fused vs 14.9 us two-step; T=1024 19.7 vs 16.0 us;
# T=8192 74.9 vs 24.1 us (the reference's torch sequence: 99 us).
_FUSED_ROUTER_MAX_T = 64
_FUSED_ROUTER_MAX_WORK = 1 << 25        # T * H * E


def _router(hidden: torch.Tensor, weight_eh: torch.Tensor, bias: torch.Tensor | None,
            top_k: int, renormalize: bool):
    """logits = hidden @ weight_eh^T (+ bias), rounded to fp16 as the gate's
    fp16 output is, then fp32 softmax -> top-k -> optional renormalisation.
    Decode-sized T: one launch (`mm_moe_router`); larger T: the library GEMM
    then `mm_softmax_topk`.  Returns (probs fp32 [T, k], ids int64 [T, k])."""
    dev = _lib.require_device(hidden, weight_eh, bias)
    H = hidden.shape[-1]
    x = _half(hidden.reshape(-1, H))
    if weight_eh.dim() != 2 or weight_eh.shape[1] != H:
        raise ValueError(f"router weight must be [num_experts, {H}], got {tuple(weight_eh.shape)}")
    T, E = x.shape[0], weight_eh.shape[0]
    if T > _FUSED_ROUTER_MAX_T or T * H * E > _FUSED_ROUTER_MAX_WORK:
        w16 = weight_eh.to(torch.float16).contiguous()
        b16 = None if bias is None else bias.to(torch.float16)
        return _softmax_topk(torch.nn.functional.linear(x, w16, b16), top_k, renormalize)
    w = _half(weight_eh)
    b = None if bias is None else bias.to(torch.float32).contiguous()
    ids = torch.empty((T, top_k), dtype=torch.int64, device=dev)
    probs = torch.empty((T, top_k), dtype=torch.float32, device=dev)
    ws = _lib.workspace(dev, int(_lib.load().mm_moe_router_workspace_bytes(T, H, E)))
    _lib.call("mm_moe_router", _lib.ptr(x), _lib.ptr(w), _lib.ptr(b), T, H, E, top_k,
              int(renormalize), _lib.ptr(ids), _lib.ptr(probs), _lib.ptr(ws), ws.numel(),
              _lib.stream_of(x))
    return probs, ids


def moe_router_topk(hidden: torch.Tensor, router_weights: torch.Tensor, top_k: int = 2):
    """softmax(hidden @ router_weights) -> top-k -> renormalise
    (kernels/moe.py:729-740), router_weights [H, E], in one launch.
    Returns (ids int64, probs fp32)."""
    probs, ids = _router(hidden, router_weights.t(), None, top_k, True)
    return ids, probs


def fused_router_topk(hidden_states: torch.Tensor, gate: nn.Linear, top_k: int,
                      training: bool = False, use_metal: bool = True):
    """Router GEMV + softmax + top-k + renormalise in one launch
    (moe_dispatch.py:178-219, _fused_router_topk; the math of its torch path,
    gate(hidden) -> _router_softmax_fusion(renormalize=True)).  gate.weight is
    [num_experts, hidden]; returns (topk_weights in the gate's dtype,
    topk_indices int64).  `training` and `use_metal` are accepted for
    signature parity; there is one implementation."""
    probs, ids = _router(hidden_states, gate.weight.detach(),
                         None if gate.bias is None else gate.bias.detach(), top_k, True)
    return probs.to(gate.weight.dtype), ids


def _softmax_topk(gate_logits: torch.Tensor, top_k: int, renormalize: bool):
    """mm_softmax_topk over logits [..., E] -> (probs fp32 [T, k], ids int64 [T, k])."""
    dev = _lib.require_device(gate_logits)
    E = gate_logits.shape[-1]
    lg = gate_logits.reshape(-1, E)
    f32 = lg.dtype != torch.float16
    lg = (lg.to(torch.float32) if f32 else lg).contiguous()
    T = lg.shape[0]
    ids = torch.empty((T, top_k), dtype=torch.int64, device=dev)
    probs = torch.empty((T, top_k), dtype=torch.float32, device=dev)
    _lib.call("mm_softmax_topk", _lib.ptr(lg), int(f32), T, E, top_k, int(renormalize),
              _lib.ptr(ids), _lib.ptr(probs), _lib.stream_of(lg))
    return probs, ids


def router_softmax_topk(gate_logits: torch.Tensor, top_k: int, renormalize: bool = True):
    """fp32 softmax -> top-k (descending) -> optional renormalisation of given
    logits [T, E] in one launch (moe_dispatch.py:99-151,
    _router_softmax_fusion).  Returns (topk_probs in the logits' dtype,
    topk_indices int64)."""
    probs, ids = _softmax_topk(gate_logits, top_k, renormalize)
    lead = tuple(gate_logits.shape[:-1])
    return probs.to(gate_logits.dtype).reshape(*lead, top_k), ids.reshape(*lead, top_k)


def mmfp4_softmax_topk(logits: torch.Tensor, top_k: int = 4):
    """Softmax over the experts then top-k, no renormalisation
    (kernels_core.py:241-247 -> the mmfp4_softmax_topk kernel :966):
    logits [B, E] -> (probs fp16 [B, k], indices int64 [B, k])."""
    probs, ids = router_softmax_topk(logits, top_k, renormalize=False)
    return probs.to(torch.float16), ids


def moe_fused_router_sorted(hidden_states: torch.Tensor, gate: nn.Linear, top_k: int):
    """Router -> softmax -> top-k -> renormalise, then the stable expert sort:
    two launches and no host synchronisation (moe_dispatch.py:328-449,
    _fused_router_topk_metal with the moe_fused_router_sorted kernel, whose
    grouping is not stable; this one is).  Returns (topk_weights, topk_ids,
    MoEDispatchInfo)."""
    w, ids = fused_router_topk(hidden_states, gate, top_k)
    info = group_tokens_by_expert_full(ids, gate.weight.shape[0])
    return w, ids, info


def _grouped(x, sorted_idx, offsets, gather: bool, k: int, T: int, packed, scales,
             group_size: int, act: int) -> torch.Tensor:
    E, KP, N = packed.shape
    K = KP * 8
    if tuple(scales.shape) != (E, K // group_size, N):
        raise ValueError(f"scales shape {tuple(scales.shape)} != ({E}, {K // group_size}, {N})")
    if x.shape[-1] != K:
        raise ValueError(f"activations K={x.shape[-1]} != packed K={K}")
    out = torch.empty((T * k, N // 2 if act else N), dtype=torch.float16, device=x.device)
    _lib.call("mm_moe_grouped_gemm", _lib.ptr(x), _lib.ptr(sorted_idx), _lib.ptr(offsets),
              int(gather), k, T, _lib.ptr(packed.contiguous()), _lib.ptr(scales.contiguous()),
              E, K, N, group_size, act, _lib.ptr(out), _lib.stream_of(x))
    return out


def _half(t: torch.Tensor) -> torch.Tensor:
    return (t if t.dtype == torch.float16 else t.to(torch.float16)).contiguous()


def moe_expert_gemm_fp4(activations: torch.Tensor, expert_weights: torch.Tensor,
                        scales: torch.Tensor, expert_ids: torch.Tensor,
                        expert_probs: torch.Tensor, group_size: int = 128) -> torch.Tensor:
    """out[t] = sum_j p[t, j] * (x[t] @ dequant(W[e(t, j)])) (kernels/moe.py:583-727).
    activations [T, K]; expert_weights [E, K/8, N]; scales [E, K/g, N];
    expert_ids / expert_probs [T, k].  Returns [T, N] in activations' dtype."""
    _lib.require_device(activations, expert_weights, scales, expert_ids, expert_probs)
    T, k = expert_ids.shape
    E = expert_weights.shape[0]
    x = _half(activations)
    s_idx, offs, inv = _sort(expert_ids, E)
    y = _grouped(x, s_idx, offs, True, k, T, expert_weights, _half(scales), group_size, 0)
    info = MoEDispatchInfo(s_idx, s_idx, offs, inv, T, k, E, s_idx)
    out = scatter_expert_outputs(y, expert_probs, info)
    return out.to(activations.dtype)


def moe_mlp_fp4(hidden: torch.Tensor, gate_up_packed: torch.Tensor, gate_up_scales: torch.Tensor,
                down_packed: torch.Tensor, down_scales: torch.Tensor, expert_ids: torch.Tensor,
                expert_probs: torch.Tensor, group_size: int = 128) -> torch.Tensor:
    """Routed-expert SwiGLU MLP over all experts, one library call
    (`mm_moe_mlp_fp4`):
        h = x @ W_gu[e];  a = silu(h[:, :I]) * h[:, I:];  y = a @ W_dn[e];
        out[t] = sum_j p[t, j] * y[(t, j)]
    (moe_dispatch.py:1241-1431 per expert, combined as :812-925).
    gate_up_packed [E, H/8, 2I], down_packed [E, I/8, H]; scales alike.
    Four launches on the caller's stream (sort, gate_up, down, combine)."""
    dev = _lib.require_device(hidden, gate_up_packed, gate_up_scales, down_packed, down_scales,
                              expert_ids, expert_probs)
    T, k = expert_ids.shape
    E, HP, N2 = gate_up_packed.shape
    H, I = HP * 8, N2 // 2
    if tuple(down_packed.shape) != (E, I // 8, H):
        raise ValueError(f"down_packed shape {tuple(down_packed.shape)} != ({E}, {I // 8}, {H})")
    for name, sc, kk, nn in (("gate_up_scales", gate_up_scales, H, N2),
                             ("down_scales", down_scales, I, H)):
        if tuple(sc.shape) != (E, kk // group_size, nn):
            raise ValueError(f"{name} shape {tuple(sc.shape)} != ({E}, {kk // group_size}, {nn})")
    x = _half(hidden.reshape(T, -1))
    if x.shape[-1] != H:
        raise ValueError(f"hidden size {x.shape[-1]} != packed K={H}")
    i64 = expert_ids.dtype == torch.int64
    ids = expert_ids.contiguous() if i64 else expert_ids.to(torch.int32).contiguous()
    p = expert_probs.to(torch.float32).contiguous()
    act = torch.empty((T * k, I), dtype=torch.float16, device=dev)
    y = torch.empty((T * k, H), dtype=torch.float16, device=dev)
    sort_buf = torch.empty(E + 1 + 2 * T * k, dtype=torch.int32, device=dev)
    out = torch.empty((T, H), dtype=torch.float16, device=dev)
    _lib.call("mm_moe_mlp_fp4", _lib.ptr(x), _lib.ptr(ids), int(i64), _lib.ptr(p), T, k, E, H, I,
              _lib.ptr(gate_up_packed.contiguous()), _lib.ptr(_half(gate_up_scales)),
              _lib.ptr(down_packed.contiguous()), _lib.ptr(_half(down_scales)), group_size,
              _lib.ptr(act), _lib.ptr(y), _lib.ptr(sort_buf), _lib.ptr(out), _lib.stream_of(x))
    return out if hidden.dtype == torch.float16 else out.to(hidden.dtype)


class MoEDispatcher(nn.Module):
    """Top-k MoE with optional shared expert (moe_dispatch.py:1025-1108):
    softmax -> top-k (no renormalisation) -> group -> per-expert callables ->
    weighted combine.  Expert offsets reach the host with one copy per call
    (the reference does one .item() sync per expert)."""

    def __init__(self, num_experts: int, num_experts_per_tok: int, experts: Sequence,
                 shared_expert=None, shared_expert_weight: float = 1.0) -> None:
        super().__init__()
        self.num_experts = num_experts
        self.num_experts_per_tok = num_experts_per_tok
        self.experts = nn.ModuleList(experts)  # type: ignore[arg-type]
        self.shared_expert = shared_expert
        self.shared_expert_weight = shared_expert_weight

    def forward(self, hidden: torch.Tensor, gate_logits: torch.Tensor) -> torch.Tensor:
        if hidden.dim() == 3:
            batch, seq, hd = hidden.shape
            flat = hidden.view(-1, hd)
        else:
            flat, batch, seq = hidden, None, None
        if gate_logits.dim() != 2:
            raise ValueError("gate_logits must be [tokens, num_experts]")
        if gate_logits.shape[0] != flat.shape[0]:
            raise ValueError("gate_logits batch must match hidden tokens")
        topk_w, topk_i = router_softmax_topk(gate_logits, self.num_experts_per_tok,
                                             renormalize=False)
        info = group_tokens_by_expert_full(topk_i, self.num_experts)
        xin = gather_for_experts(flat, info)
        out_dim = getattr(self.experts[0], "out_features", flat.shape[-1])
        y = flat.new_empty((xin.shape[0], out_dim))
        offs = info.expert_offsets.cpu().tolist()
        for e in range(self.num_experts):
            a, b = offs[e], offs[e + 1]
            if a != b:
                y[a:b] = self.experts[e](xin[a:b])
        combined = scatter_expert_outputs(y, topk_w, info)
        if self.shared_expert is not None:
            combined = combined + self.shared_expert_weight * self.shared_expert(flat)
        if batch is not None:
            return combined.view(batch, seq, -1)
        return combined
