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

FP4_PER_UINT = 8


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
             group_size: int, act: int, zero_rows: bool = False) -> torch.Tensor:
    """mm_moe_grouped_gemm -> [T*k, N (N/2 with act)] in sorted order.  Rows
    of dropped assignments (ids outside [0, E)) are not written by the
    kernel; zero_rows makes them zero."""
    E, KP, N = packed.shape
    K = KP * 8
    if tuple(scales.shape) != (E, K // group_size, N):
        raise ValueError(f"scales shape {tuple(scales.shape)} != ({E}, {K // group_size}, {N})")
    if x.shape[-1] != K:
        raise ValueError(f"activations K={x.shape[-1]} != packed K={K}")
    alloc = torch.zeros if zero_rows else torch.empty
    out = alloc((T * k, N // 2 if act else N), dtype=torch.float16, device=x.device)
    # converted copies are bound to names so they outlive the launch
    w, s = packed.contiguous(), scales.contiguous()
    _lib.call("mm_moe_grouped_gemm", _lib.ptr(x), _lib.ptr(sorted_idx), _lib.ptr(offsets),
              int(gather), k, T, _lib.ptr(w), _lib.ptr(s), E, K, N, group_size, act,
              _lib.ptr(out), _lib.stream_of(x))
    return out


def _half(t: torch.Tensor) -> torch.Tensor:
    return (t if t.dtype == torch.float16 else t.to(torch.float16)).contiguous()


def _packed_words(t: torch.Tensor) -> torch.Tensor:
    if t.dtype not in (torch.int32, torch.uint32):
        raise TypeError(f"packed weights must be int32/uint32 words, got {t.dtype}")
    return t.contiguous()


def moe_expert_gemm_fp4(activations: torch.Tensor, expert_weights: torch.Tensor,
                        scales: torch.Tensor, expert_ids: torch.Tensor,
                        expert_probs: torch.Tensor, group_size: int = 128) -> torch.Tensor:
    """out[t] = sum_j p[t, j] * (x[t] @ dequant(W[e(t, j)])) (kernels/moe.py:583-727).
    activations [T, K]; expert_weights [E, K/8, N]; scales [E, K/g, N];
    expert_ids / expert_probs [T, k].  Returns [T, N] in activations' dtype.
    Ids outside [0, E) contribute nothing (the reference kernel skips them)."""
    _lib.require_device(activations, expert_weights, scales, expert_ids, expert_probs)
    T, k = expert_ids.shape
    E = expert_weights.shape[0]
    x = _half(activations)
    s_idx, offs, inv = _sort(expert_ids, E)
    y = _grouped(x, s_idx, offs, True, k, T, expert_weights, _half(scales), group_size, 0,
                 zero_rows=True)
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
    # converted copies are bound to names so they outlive the launch
    gu, gus = gate_up_packed.contiguous(), _half(gate_up_scales)
    dn, dns = down_packed.contiguous(), _half(down_scales)
    _lib.call("mm_moe_mlp_fp4", _lib.ptr(x), _lib.ptr(ids), int(i64), _lib.ptr(p), T, k, E, H, I,
              _lib.ptr(gu), _lib.ptr(gus), _lib.ptr(dn), _lib.ptr(dns), group_size,
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


# ---------------------------------------------------------------------------
# Expert MLP entry points with the reference's names, and the shared expert.
# ---------------------------------------------------------------------------
def _marlin_words(packed: torch.Tensor, K: int, N: int, name: str) -> torch.Tensor:
    """[K/8, N] words; a row-packed [N, K/8] tensor (what the reference's
    torch path also accepts, moe_dispatch.py:1397-1406) is transposed."""
    if tuple(packed.shape) == (K // 8, N):
        return packed.contiguous()
    if tuple(packed.shape) == (N, K // 8):
        return packed.t().contiguous()
    raise ValueError(f"{name} shape {tuple(packed.shape)} is neither ({K // 8}, {N}) nor "
                     f"({N}, {K // 8})")


def _moe_mlp_shared(hidden: torch.Tensor, routed, shared, expert_ids, expert_probs,
                    shared_weight: float, base: torch.Tensor | None, group_size: int
                    ) -> torch.Tensor:
    """One mm_moe_mlp_shared_fp4 call.  routed: (gu, gus, dn, dns) stacked
    [E, ...] or None; shared: (gu, gus, dn, dns) of one expert."""
    sgu, sgus, sdn, sdns = shared
    x = _half(hidden)
    T, H = x.shape
    if sgus.dim() != 2 or sgus.shape[1] % 2 != 0:
        raise ValueError(f"shared gate_up scales must be [H/g, 2I], got {tuple(sgus.shape)}")
    I = sgus.shape[1] // 2
    if H % group_size or I % group_size:
        raise ValueError(f"hidden ({H}) and intermediate ({I}) must be divisible by "
                         f"group_size ({group_size})")
    sgu = _marlin_words(sgu, H, 2 * I, "shared gate_up packed")
    sdn = _marlin_words(sdn, I, H, "shared down packed")
    if tuple(sgus.shape) != (H // group_size, 2 * I) or \
            tuple(sdns.shape) != (I // group_size, H):
        raise ValueError("shared expert scales must be [H/g, 2I] and [I/g, H]")
    dev = _lib.require_device(x, sgu, sgus, sdn, sdns, expert_ids, expert_probs, base)
    if routed is None:
        k, E = 0, 0
        gu = gus = dn = dns = ids = p = None
        i64 = 1
    else:
        gu, gus, dn, dns = routed
        E = gu.shape[0]
        if tuple(gu.shape) != (E, H // 8, 2 * I) or tuple(dn.shape) != (E, I // 8, H):
            raise ValueError(f"routed weights must be [E, {H // 8}, {2 * I}] and "
                             f"[E, {I // 8}, {H}] (the shared expert's intermediate size)")
        if tuple(gus.shape) != (E, H // group_size, 2 * I) or \
                tuple(dns.shape) != (E, I // group_size, H):
            raise ValueError("routed scales must be [E, H/g, 2I] and [E, I/g, H]")
        if expert_ids.dim() != 2 or expert_ids.shape[0] != T:
            raise ValueError(f"expert_ids must be [{T}, top_k], got {tuple(expert_ids.shape)}")
        k = expert_ids.shape[1]
        i64 = int(expert_ids.dtype == torch.int64)
        ids = expert_ids.contiguous() if i64 else expert_ids.to(torch.int32).contiguous()
        p = expert_probs.to(torch.float32).contiguous()
        gu, dn = gu.contiguous(), dn.contiguous()
        gus, dns = _half(gus), _half(dns)
    kt = k + 1
    b = None if base is None else _half(base.reshape(T, H))
    act = torch.empty((T * kt, I), dtype=torch.float16, device=dev)
    y = torch.empty((T * kt, H), dtype=torch.float16, device=dev)
    sort_buf = torch.empty(E + 2 + 2 * T * kt, dtype=torch.int32, device=dev)
    out = torch.empty((T, H), dtype=torch.float16, device=dev)
    sgus_h, sdns_h = _half(sgus), _half(sdns)   # bound: they must outlive the launch
    _lib.call("mm_moe_mlp_shared_fp4", _lib.ptr(x), _lib.ptr(ids), i64, _lib.ptr(p), T, k, E, H,
              I, _lib.ptr(gu), _lib.ptr(gus), _lib.ptr(dn), _lib.ptr(dns), _lib.ptr(sgu),
              _lib.ptr(sgus_h), _lib.ptr(sdn), _lib.ptr(sdns_h), float(shared_weight),
              _lib.ptr(b), group_size, _lib.ptr(act), _lib.ptr(y), _lib.ptr(sort_buf),
              _lib.ptr(out), _lib.stream_of(x))
    return out


def _flatten_hidden(hidden: torch.Tensor):
    if hidden.dim() < 2:
        raise ValueError(f"hidden_states must be [..., hidden], got {tuple(hidden.shape)}")
    return hidden.reshape(-1, hidden.shape[-1]), hidden.shape


def _fused_expert_mlp(x: torch.Tensor, gate_up_packed: torch.Tensor,
                      gate_up_scales: torch.Tensor, down_packed: torch.Tensor,
                      down_scales: torch.Tensor, group_size: int) -> torch.Tensor:
    """One expert's SwiGLU MLP (moe_dispatch.py:1241-1431):
    h = x @ W_gu ([H/8, 2I] packed; the row-packed [2I, H/8] is accepted too),
    a = silu(h[:, :I]) * h[:, I:], y = a @ W_dn ([I/8, H]).  x [batch, H];
    returns [batch, H] in x's dtype.  The gate_up product and the SwiGLU are
    one launch, the down product a second (the sort is a trivial one-group
    launch)."""
    if x.dim() != 2:
        raise ValueError(f"x must be [batch, hidden], got {tuple(x.shape)}")
    out = _moe_mlp_shared(x, None, (gate_up_packed, gate_up_scales, down_packed, down_scales),
                          None, None, 1.0, None, group_size)
    return out if x.dtype == torch.float16 else out.to(x.dtype)


def moe_shared_expert_fp4(hidden_states: torch.Tensor, gate_up_packed: torch.Tensor,
                          gate_up_scales: torch.Tensor, down_packed: torch.Tensor,
                          down_scales: torch.Tensor, group_size: int = 128,
                          shared_prob: float = 1.0) -> torch.Tensor:
    """shared_prob * SwiGLU-MLP(hidden) for a shared expert (kernels/moe.py:
    442-582): gate_up [H/8, 2I], down [I/8, H].  fp16 [..., H]."""
    x, shape = _flatten_hidden(hidden_states)
    out = _moe_mlp_shared(x, None, (gate_up_packed, gate_up_scales, down_packed, down_scales),
                          None, None, shared_prob, None, group_size)
    return out.reshape(*shape[:-1], out.shape[-1])


def moe_add_shared_expert_fp4(hidden_states: torch.Tensor, moe_output: torch.Tensor,
                              shared_gate_up_packed: torch.Tensor,
                              shared_gate_up_scales: torch.Tensor,
                              shared_down_packed: torch.Tensor, shared_down_scales: torch.Tensor,
                              group_size: int = 128) -> torch.Tensor:
    """moe_output + SwiGLU-MLP_shared(hidden) (kernels/moe.py:858-930); the
    addition happens in the combine launch, in fp32.  fp16 [..., H]."""
    x, shape = _flatten_hidden(hidden_states)
    if moe_output.shape != x.shape and moe_output.shape != shape:
        raise ValueError(f"moe_output shape {tuple(moe_output.shape)} doesn't match hidden "
                         f"shape {tuple(x.shape)}")
    out = _moe_mlp_shared(x, None, (shared_gate_up_packed, shared_gate_up_scales,
                                    shared_down_packed, shared_down_scales),
                          None, None, 1.0, moe_output, group_size)
    return out.reshape(*shape[:-1], out.shape[-1])


def moe_shared_expert_fused_fp4(hidden_states: torch.Tensor, shared_expert_packed: torch.Tensor,
                                shared_expert_scales: torch.Tensor,
                                routed_expert_packed: torch.Tensor,
                                routed_expert_scales: torch.Tensor, router_probs: torch.Tensor,
                                router_indices: torch.Tensor,
                                group_size: int = 128) -> torch.Tensor:
    """Shared + routed aggregation of one FP4 projection (kernels/moe.py:
    182-329, src/moe_shared_expert.metal:604-):
        out[t] = x[t] @ W_sh + sum_j p[t, j] * (x[t] @ W_{e(t, j)})
    shared_expert_packed [H/8, I] Marlin layout, scales [H/g, I]; routed
    [E, H/8, I] / [E, H/g, I]; router_probs / router_indices [T, top_k].
    Indices outside [0, E) contribute nothing (the reference kernel skips
    them).  One library call: the shared matrix is one more group of the
    grouped launch.  fp16 [..., I]."""
    x, shape = _flatten_hidden(hidden_states)
    T, H = x.shape
    if H % FP4_PER_UINT != 0:
        raise ValueError(f"hidden_dim ({H}) must be divisible by {FP4_PER_UINT}")
    if H % group_size != 0:
        raise ValueError(f"hidden_dim ({H}) must be divisible by group_size ({group_size})")
    if shared_expert_packed.dim() != 2:
        raise ValueError("shared_expert_packed must be [hidden/8, intermediate]")
    packed_k = int(shared_expert_packed.shape[0])
    if packed_k * FP4_PER_UINT != H:
        raise ValueError("shared_expert_packed hidden dim mismatch")
    I = int(shared_expert_packed.shape[1])
    rows = H // group_size
    if tuple(shared_expert_scales.shape) != (rows, I):
        raise ValueError("shared_expert_scales shape mismatch")
    if routed_expert_packed.dim() != 3:
        raise ValueError("routed_expert_packed must be [num_experts, hidden/8, intermediate]")
    if routed_expert_packed.shape[1] != packed_k or routed_expert_packed.shape[2] != I:
        raise ValueError("routed_expert_packed shape mismatch")
    if routed_expert_scales.dim() != 3:
        raise ValueError("routed_expert_scales must be [num_experts, hidden/group, intermediate]")
    if routed_expert_scales.shape[1] != rows or routed_expert_scales.shape[2] != I:
        raise ValueError("routed_expert_scales shape mismatch")
    if router_probs.dim() != 2 or router_probs.shape[0] != T:
        raise ValueError("router_probs must be [tokens, top_k]")
    if router_indices.dim() != 2 or router_indices.shape[0] != T:
        raise ValueError("router_indices must be [tokens, top_k]")
    k = int(router_probs.shape[1])
    if router_indices.shape[1] != k:
        raise ValueError("router_probs and router_indices must have same top_k")
    if I % 8 != 0:
        raise ValueError(f"intermediate_dim ({I}) must be divisible by 8")
    dev = _lib.require_device(x, shared_expert_packed, shared_expert_scales, routed_expert_packed,
                              routed_expert_scales, router_probs, router_indices)
    E = int(routed_expert_packed.shape[0])
    i64 = int(router_indices.dtype == torch.int64)
    ids = router_indices.contiguous() if i64 else router_indices.to(torch.int32).contiguous()
    p = router_probs.to(torch.float32).contiguous()
    sp, rp = _packed_words(shared_expert_packed), _packed_words(routed_expert_packed)
    ss, rs = _half(shared_expert_scales), _half(routed_expert_scales)
    kt = k + 1
    y = torch.empty((T * kt, I), dtype=torch.float16, device=dev)
    sort_buf = torch.empty(E + 2 + 2 * T * kt, dtype=torch.int32, device=dev)
    out = torch.empty((T, I), dtype=torch.float16, device=dev)
    _lib.call("mm_moe_gemm_shared_fp4", _lib.ptr(x), _lib.ptr(ids), i64, _lib.ptr(p), T, k, E,
              H, I, _lib.ptr(sp), _lib.ptr(ss), _lib.ptr(rp), _lib.ptr(rs), group_size,
              _lib.ptr(y), _lib.ptr(sort_buf), _lib.ptr(out), _lib.stream_of(x))
    return out.reshape(*shape[:-1], I)


def moe_fused_dispatch_shared_fp4(hidden_states: torch.Tensor,
                                  shared_gate_up_packed: torch.Tensor,
                                  shared_gate_up_scales: torch.Tensor,
                                  shared_down_packed: torch.Tensor,
                                  shared_down_scales: torch.Tensor,
                                  routed_gate_up_packed: torch.Tensor,
                                  routed_gate_up_scales: torch.Tensor,
                                  routed_down_packed: torch.Tensor,
                                  routed_down_scales: torch.Tensor,
                                  expert_ids: torch.Tensor, expert_probs: torch.Tensor,
                                  group_size: int = 128) -> torch.Tensor:
    """Routed experts plus a shared expert (kernels/moe.py:742-856):
    out[t] = MLP_shared(x[t]) + sum_j p[t, j] * MLP_{e(t, j)}(x[t]).
    Shared weights [H/8, 2I] / [I/8, H], routed [E, H/8, 2I] / [E, I/8, H]
    (same intermediate size, as the reference requires).  The shared expert is
    one more group of the two grouped launches.  fp16 [..., H]."""
    x, shape = _flatten_hidden(hidden_states)
    H = x.shape[-1]
    if H % 8 != 0:
        raise ValueError(f"hidden_dim ({H}) must be divisible by 8")
    if H % group_size != 0:
        raise ValueError(f"hidden_dim ({H}) must be divisible by group_size ({group_size})")
    out = _moe_mlp_shared(
        x, (routed_gate_up_packed, routed_gate_up_scales, routed_down_packed, routed_down_scales),
        (shared_gate_up_packed, shared_gate_up_scales, shared_down_packed, shared_down_scales),
        expert_ids, expert_probs, 1.0, None, group_size)
    return out.reshape(*shape[:-1], H)


class FusedMoEDispatcher(nn.Module):
    """MoE with a shared expert in one fused pass (moe_dispatch.py:1111-1238):
    output = shared_expert(x) + sum_k prob[k] * routed_expert_k(x), with
    softmax -> top-k (no renormalisation) routing of the given logits.
    Weights: routed gate_up [E, H/8, 2I] (scales [E, H/g, 2I]), down
    [E, I/8, H] (scales [E, I/g, H]); shared gate_up [H/8, 2I], down [I/8, H]."""

    def __init__(self, num_experts: int, num_experts_per_tok: int,
                 expert_gate_up_weights: torch.Tensor, expert_gate_up_scales: torch.Tensor,
                 expert_down_weights: torch.Tensor, expert_down_scales: torch.Tensor,
                 shared_gate_up_weights: torch.Tensor, shared_gate_up_scales: torch.Tensor,
                 shared_down_weights: torch.Tensor, shared_down_scales: torch.Tensor,
                 group_size: int = 128) -> None:
        super().__init__()
        self.num_experts = num_experts
        self.num_experts_per_tok = num_experts_per_tok
        self.group_size = group_size
        self.register_buffer("expert_gate_up_weights", expert_gate_up_weights)
        self.register_buffer("expert_gate_up_scales", expert_gate_up_scales)
        self.register_buffer("expert_down_weights", expert_down_weights)
        self.register_buffer("expert_down_scales", expert_down_scales)
        self.register_buffer("shared_gate_up_weights", shared_gate_up_weights)
        self.register_buffer("shared_gate_up_scales", shared_gate_up_scales)
        self.register_buffer("shared_down_weights", shared_down_weights)
        self.register_buffer("shared_down_scales", shared_down_scales)

    def forward(self, hidden: torch.Tensor, gate_logits: torch.Tensor) -> torch.Tensor:
        if hidden.dim() == 3:
            batch, seq, hd = hidden.shape
            flat = hidden.reshape(-1, hd)
        else:
            flat, batch, seq = hidden, None, None
        if gate_logits.dim() != 2:
            raise ValueError("gate_logits must be [tokens, num_experts]")
        if gate_logits.shape[0] != flat.shape[0]:
            raise ValueError("gate_logits batch must match hidden tokens")
        probs, ids = _softmax_topk(gate_logits, self.num_experts_per_tok, False)
        out = moe_fused_dispatch_shared_fp4(
            flat, self.shared_gate_up_weights, self.shared_gate_up_scales,
            self.shared_down_weights, self.shared_down_scales, self.expert_gate_up_weights,
            self.expert_gate_up_scales, self.expert_down_weights, self.expert_down_scales,
            ids, probs, self.group_size)
        if batch is not None:
            return out.view(batch, seq, -1)
        return out


def _expert_tensors(expert) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """One expert module's weights as Marlin-layout gate_up [H/8, 2I] with
    scales [H/g, 2I] and down [I/8, H] with scales [I/g, H].  Experts hold
    row-packed layers ([out, in/8] words, [n_groups, out] scales): either
    gate_proj and up_proj (what moe_dispatch.py:2623-2636 stacks) or one fused
    gate_up_proj (layers/mmfp4_expert.py:193-250)."""
    if hasattr(expert, "gate_up_proj"):
        gu_rows = expert.gate_up_proj.packed_weights
        gu_s = expert.gate_up_proj.scales
    else:
        gu_rows = torch.cat([expert.gate_proj.packed_weights, expert.up_proj.packed_weights], 0)
        gu_s = torch.cat([expert.gate_proj.scales, expert.up_proj.scales], 1)
    dn = expert.down_proj
    return (gu_rows.t().contiguous(), gu_s.to(torch.float16).contiguous(),
            dn.packed_weights.t().contiguous(), dn.scales.to(torch.float16).contiguous())


def _stacked_expert_weights(experts, n_experts: int):
    """[E, ...] Marlin-layout stacks of every expert's weights, built once and
    kept on the ModuleList until one of the source tensors is replaced or
    written (keyed on data pointers and version counters)."""
    srcs = []
    for e in range(n_experts):
        ex = experts[e]
        layers = ([ex.gate_up_proj] if hasattr(ex, "gate_up_proj")
                  else [ex.gate_proj, ex.up_proj]) + [ex.down_proj]
        for lyr in layers:
            for t in (lyr.packed_weights, lyr.scales):
                srcs.append((t.data_ptr(), t._version))
    key = tuple(srcs)
    cached = getattr(experts, "_mmfp4_stacked", None)
    if cached is not None and cached[0] == key:
        return cached[1]
    parts = [_expert_tensors(experts[e]) for e in range(n_experts)]
    stacked = tuple(torch.stack([p[i] for p in parts], 0) for i in range(4))
    experts._mmfp4_stacked = (key, stacked)
    return stacked


def dispatch_experts_batched(expert_inputs: torch.Tensor, experts, dispatch_info: MoEDispatchInfo,
                             n_experts: int, batch_size: int = 16) -> torch.Tensor:
    """Every expert's SwiGLU MLP over its rows of the expert-sorted inputs
    (moe_dispatch.py:2546-2676): expert_inputs [T*k, H] in sorted order (the
    output of gather_for_experts), rows offsets[e]..offsets[e+1] go to
    experts[e].  Returns [T*k, H] in sorted order, expert_inputs' dtype.
    The reference stacks weights per batch of `batch_size` experts and runs
    one fused MLP per expert; here the stacked weights are cached and all
    experts run in two grouped launches (gate_up + SwiGLU, down), so
    `batch_size` has no effect."""
    del batch_size
    dev = _lib.require_device(expert_inputs)
    total, H = expert_inputs.shape
    out_dtype = expert_inputs.dtype
    if total == 0:
        return expert_inputs.new_empty((0, H))
    gs = {int(experts[e].group_size) for e in range(n_experts)}
    if len(gs) != 1:
        raise ValueError(f"experts use different group sizes {sorted(gs)}")
    g = gs.pop()
    gu, gus, dn, dns = _stacked_expert_weights(experts, n_experts)
    if gu.device != dev:
        raise RuntimeError(f"expert weights on {gu.device}, inputs on {dev}")
    E, HP, N2 = gu.shape
    if HP * 8 != H:
        raise ValueError(f"expert hidden size {HP * 8} != inputs' {H}")
    I = N2 // 2
    offs = dispatch_info.expert_offsets.to(device=dev, dtype=torch.int32).contiguous()
    if offs.numel() != n_experts + 1:
        raise ValueError(f"dispatch_info has {offs.numel() - 1} experts, expected {n_experts}")
    x = _half(expert_inputs)
    act = torch.empty((total, I), dtype=torch.float16, device=dev)
    y = torch.empty((total, H), dtype=torch.float16, device=dev)
    st = _lib.stream_of(x)
    _lib.call("mm_moe_grouped_gemm", _lib.ptr(x), None, _lib.ptr(offs), 0, 1, total,
              _lib.ptr(gu), _lib.ptr(gus), E, H, N2, g, 1, _lib.ptr(act), st)
    _lib.call("mm_moe_grouped_gemm", _lib.ptr(act), None, _lib.ptr(offs), 0, 1, total,
              _lib.ptr(dn), _lib.ptr(dns), E, I, H, g, 0, _lib.ptr(y), st)
    return y if out_dtype == torch.float16 else y.to(out_dtype)
