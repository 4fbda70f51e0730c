"""numpy restatement of the reference's MoE routing, grouping, gather, expert
MLP and weighted combine (test infrastructure; see oracle/__init__.py)."""

from __future__ import annotations

import numpy as np

from .fp4 import dequant_fp4_f32


def router_topk(logits: np.ndarray, top_k: int, renormalize: bool = True):
    """fp32 softmax -> top-k (descending, lower expert id first on ties) ->
    optional renormalisation.  moe_dispatch.py:99-151 (_router_softmax_fusion,
    renormalize=True) and kernels/moe.py:729-740 (moe_router_topk);
    renormalize=False is MoEDispatcher.forward (moe_dispatch.py:1077-1080).
    Returns (ids int32 [T, k], probs float32 [T, k])."""
    x = np.asarray(logits, dtype=np.float32)
    x = x - x.max(axis=-1, keepdims=True)
    e = np.exp(x)
    p = e / e.sum(axis=-1, keepdims=True)
    order = np.argsort(-p, axis=-1, kind="stable")[:, :top_k]
    probs = np.take_along_axis(p, order, axis=-1)
    if renormalize:
        probs = probs / probs.sum(axis=-1, keepdims=True)
    return order.astype(np.int32), probs.astype(np.float32)


def group_tokens_by_expert(expert_ids: np.ndarray, num_experts: int):
    """Stable counting sort of the flattened (token, slot) assignments by
    expert.  moe_dispatch.py:493-555: offsets = exclusive cumsum of bincount;
    within an expert, assignments keep ascending flat index t*k+slot (the
    one-hot cumsum rank).  Returns (sorted_indices, offsets[E+1], inverse)."""
    flat = np.asarray(expert_ids).reshape(-1).astype(np.int64)
    counts = np.bincount(flat, minlength=num_experts)
    offsets = np.zeros(num_experts + 1, dtype=np.int64)
    offsets[1:] = np.cumsum(counts)
    # explicit counting-sort scatter (rank = number of earlier equal ids)
    fill = offsets[:-1].copy()
    sorted_idx = np.empty(flat.shape[0], dtype=np.int64)
    for i, e in enumerate(flat):
        sorted_idx[fill[e]] = i
        fill[e] += 1
    inverse = np.empty_like(sorted_idx)
    inverse[sorted_idx] = np.arange(flat.shape[0], dtype=np.int64)
    return sorted_idx, offsets, inverse


def gather_for_experts(x: np.ndarray, sorted_idx: np.ndarray, top_k: int) -> np.ndarray:
    """X_sorted = X[sorted_idx // k].  moe_dispatch.py:789-809."""
    return np.asarray(x)[sorted_idx // top_k]


def combine(expert_out: np.ndarray, probs: np.ndarray, sorted_idx: np.ndarray,
            num_tokens: int, top_k: int) -> np.ndarray:
    """out[t] = sum_j p[t, j] * y[(t, j)] in fp32.  moe_dispatch.py:812-894."""
    out = np.zeros((num_tokens, expert_out.shape[1]), dtype=np.float32)
    p = np.asarray(probs, dtype=np.float32).reshape(-1)
    for pos, idx in enumerate(sorted_idx):
        out[idx // top_k] += p[idx] * expert_out[pos].astype(np.float32)
    return out


def silu(x: np.ndarray) -> np.ndarray:
    return x / (1.0 + np.exp(-x))


def expert_mlp_ref(x: np.ndarray, gu_packed, gu_scales, dn_packed, dn_scales,
                   group_size: int) -> np.ndarray:
    """fp32 expert MLP: h = x @ W_gu; a = silu(h[:, :I]) * h[:, I:]; y = a @ W_dn.
    moe_dispatch.py:1341-1431 (_fused_expert_mlp PyTorch reference)."""
    w_gu = dequant_fp4_f32(gu_packed, gu_scales, group_size)
    w_dn = dequant_fp4_f32(dn_packed, dn_scales, group_size)
    h = np.asarray(x, dtype=np.float32) @ w_gu
    inter = h.shape[1] // 2
    a = silu(h[:, :inter]) * h[:, inter:]
    return a @ w_dn


def moe_forward_ref(x, gu_packed, gu_scales, dn_packed, dn_scales, expert_ids, probs,
                    group_size: int) -> np.ndarray:
    """Per-token brute force: y[t] = sum_j p[t,j] * MLP_{e(t,j)}(x[t]) in fp32.
    Semantics of the per-expert fallback kernels/moe.py:690-727 composed with
    the expert MLP of moe_dispatch.py:1341-1431.  Weights are indexed [E, ...]."""
    x = np.asarray(x, dtype=np.float32)
    t_count, top_k = expert_ids.shape
    out = np.zeros((t_count, dn_packed.shape[-1]), dtype=np.float32)
    cache = {}
    for e in np.unique(expert_ids):
        rows = np.nonzero(expert_ids == e)
        toks = rows[0]
        if e not in cache:
            cache[e] = expert_mlp_ref(x[toks], gu_packed[e], gu_scales[e], dn_packed[e],
                                      dn_scales[e], group_size)
        y = cache[e]
        for r, (t, j) in enumerate(zip(*rows)):
            out[t] += probs[t, j] * y[r]
    return out
