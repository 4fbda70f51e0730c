"""GPU parity of the fused router (router GEMM + softmax + top-k +
renormalisation in one launch) and of the softmax/top-k kernel against the
oracle's fp32 softmax and stable top-k on the fp16-rounded logits."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from gpu_helpers import announce, to_dev, to_np
from oracle import moe as omoe

pytestmark = pytest.mark.gpu


def _check_topk(ids, probs, ref_full, k, renorm):
    """ids/probs against the reference probabilities ref_full [T, E] (fp32):
    where the k-th and (k+1)-th reference probabilities are apart by more than
    a logit-rounding margin the ids must match exactly (in order); elsewhere
    the chosen set must still be a top-k set within that margin."""
    ids, probs = to_np(ids), to_np(probs).astype(np.float64)
    T, E = ref_full.shape
    order = np.argsort(-ref_full, axis=1, kind="stable")
    for t in range(T):
        r = ref_full[t]
        ref_ids = order[t, :k]
        kth = r[ref_ids[-1]]
        nxt = r[order[t, k]] if k < E else -1.0
        margin = 2e-3 * max(r.max(), 1e-30)
        if kth - nxt > margin:
            assert set(ids[t]) == set(ref_ids), (t, ids[t], ref_ids)
        else:
            assert r[ids[t]].min() >= nxt - margin, (t, ids[t], ref_ids)
        sel = r[ids[t]]
        want = sel / sel.sum() if renorm else sel
        np.testing.assert_allclose(probs[t], want, rtol=5e-3, atol=1e-6)
        assert np.all(np.diff(probs[t]) <= 1e-7), "descending order"


def _ref_probs(logits16):
    x = logits16.astype(np.float32)
    x = x - x.max(axis=1, keepdims=True)
    e = np.exp(x)
    return e / e.sum(axis=1, keepdims=True)


@pytest.mark.parametrize("T,H,E,k", [(1, 2048, 128, 8), (15, 2048, 128, 8), (17, 2048, 128, 8),
                                     (1024, 2048, 128, 8), (33, 4096, 8, 2), (40, 512, 60, 4),
                                     (9, 256, 1000, 8), (300, 7168, 256, 8), (5, 96, 16, 1),
                                     (4100, 2048, 128, 8)])
@pytest.mark.parametrize("path", ["auto", "one_launch"])
def test_fused_router_vs_oracle(rng, monkeypatch, path, T, H, E, k):
    """`auto` takes the size dispatch (one launch for decode-sized T, the
    library GEMM + softmax/top-k kernel above it); `one_launch` forces the
    single-kernel router at every size."""
    import mmfp4
    from mmfp4 import moe_dispatch
    if path == "one_launch":
        monkeypatch.setattr(moe_dispatch, "_FUSED_ROUTER_MAX_T", 1 << 30)
        monkeypatch.setattr(moe_dispatch, "_FUSED_ROUTER_MAX_WORK", 1 << 62)
    x = rng.normal(0, 1, (T, H)).astype(np.float16)
    w = (rng.normal(0, 1, (E, H)) / np.sqrt(H)).astype(np.float16)
    logits16 = (x.astype(np.float32) @ w.astype(np.float32).T).astype(np.float16)
    ref = _ref_probs(logits16)
    gate = torch.nn.Linear(H, E, bias=False).to("cuda").half()
    with torch.no_grad():
        gate.weight.copy_(to_dev(w))
    announce(f"fused router {path} T={T} H={H} E={E} k={k}")
    wts, ids = mmfp4.fused_router_topk(to_dev(x), gate, k)
    assert wts.dtype == torch.float16 and ids.dtype == torch.int64
    _check_topk(ids, wts.float(), ref, k, True)
    # the [H, E] router-weights entry (kernels/moe.py:729) is the same op
    ids2, p2 = mmfp4.moe_router_topk(to_dev(x), to_dev(np.ascontiguousarray(w.T)), k)
    assert torch.equal(ids2, ids)
    _check_topk(ids2, p2, ref, k, True)


@pytest.mark.parametrize("dtype", [np.float16, np.float32])
@pytest.mark.parametrize("renorm", [True, False])
def test_softmax_topk_vs_oracle(rng, dtype, renorm):
    import mmfp4
    T, E, k = 300, 128, 8
    logits = rng.normal(0, 2, (T, E)).astype(dtype)
    logits[0, :] = 1.0                        # all equal: lowest ids win
    logits[1, 5] = logits[1, 9] = 40.0        # a tie at the top
    announce(f"softmax_topk {np.dtype(dtype).name} renorm={renorm}")
    p, ids = mmfp4.router_softmax_topk(to_dev(logits), k, renormalize=renorm)
    ref = _ref_probs(logits)
    _check_topk(ids, p.float(), ref, k, renorm)
    assert to_np(ids)[0].tolist() == list(range(k))
    assert to_np(ids)[1, :2].tolist() == [5, 9]
    oid, op = omoe.router_topk(logits.astype(np.float32), k, renormalize=renorm)
    np.testing.assert_array_equal(to_np(ids)[:2], oid[:2])


def test_moe_fused_router_sorted():
    import mmfp4
    gen = torch.Generator(device="cuda").manual_seed(4)
    T, H, E, k = 64, 1024, 32, 4
    x = torch.randn((T, H), generator=gen, device="cuda").half()
    gate = torch.nn.Linear(H, E, bias=False).to("cuda").half()
    announce("moe_fused_router_sorted")
    w, ids, info = mmfp4.moe_fused_router_sorted(x, gate, k)
    ref = mmfp4.group_tokens_by_expert_full(ids, E)
    assert torch.equal(info.expert_offsets, ref.expert_offsets)
    assert torch.equal(info.sorted_token_indices, ref.sorted_token_indices)
    assert torch.allclose(w.float().sum(-1), torch.ones(T, device="cuda"), atol=2e-3)


def test_moe_dispatcher_forward_matches_torch():
    """MoEDispatcher (moe_dispatch.py:1025-1108): softmax -> top-k (no
    renormalisation) -> per-expert callables -> weighted combine, against the
    same steps in torch."""
    import mmfp4
    gen = torch.Generator(device="cuda").manual_seed(8)
    T, H, E, k = 48, 256, 8, 2
    experts = [torch.nn.Linear(H, H, bias=False).to("cuda").half() for _ in range(E)]
    x = torch.randn((T, H), generator=gen, device="cuda").half()
    logits = torch.randn((T, E), generator=gen, device="cuda").half()
    announce("MoEDispatcher forward")
    disp = mmfp4.MoEDispatcher(E, k, experts)
    with torch.no_grad():
        out = disp(x, logits).float()
        p = logits.softmax(-1)
        w, i = torch.topk(p, k, -1)
        ref = torch.zeros((T, H), device="cuda")
        for t in range(T):
            for j in range(k):
                ref[t] += w[t, j].float() * experts[int(i[t, j])](x[t:t + 1]).float()[0]
    assert (out - ref).abs().max().item() <= 1e-2 * ref.abs().max().item()


@pytest.mark.parametrize("E,k,dtype", [(16, 1, np.float32), (16, 16, np.float16), (128, 64, np.float32),
                                       (200, 8, np.float16), (300, 16, np.float32),
                                       (1000, 8, np.float16), (2000, 32, np.float32)])
def test_softmax_topk_layouts(rng, E, k, dtype):
    """Every selection layout of the softmax/top-k kernel: 16 lanes per token
    (E <= 256, up to 16 slots per lane, k up to 64), 64 lanes per token with
    registers (E <= 1024) and the per-round path (E > 1024); odd token counts
    so the last wave holds fewer than four tokens."""
    import mmfp4
    T = 37
    logits = rng.normal(0, 2, (T, E)).astype(dtype)
    logits[3, :] = 0.5                          # all equal: the lowest ids win
    announce(f"softmax_topk layouts E={E} k={k} {np.dtype(dtype).name}")
    p, ids = mmfp4.router_softmax_topk(to_dev(logits), k, renormalize=True)
    ref = _ref_probs(logits)
    _check_topk(ids, p.float(), ref, k, True)
    assert to_np(ids)[3].tolist() == list(range(k))


@pytest.mark.parametrize("T,H,E,k", [(40, 256, 300, 8), (19, 512, 64, 64), (33, 128, 16, 3)])
def test_fused_router_bias_and_layouts(rng, T, H, E, k):
    """Router with a gate bias (added to the fp32 logits before the fp16
    rounding, as nn.Linear does) over the 16-lane and 64-lane top-k layouts."""
    import mmfp4
    x = rng.normal(0, 1, (T, H)).astype(np.float16)
    w = (rng.normal(0, 1, (E, H)) / np.sqrt(H)).astype(np.float16)
    b = rng.normal(0, 0.5, E).astype(np.float16)
    logits16 = (x.astype(np.float32) @ w.astype(np.float32).T + b.astype(np.float32)).astype(np.float16)
    ref = _ref_probs(logits16)
    gate = torch.nn.Linear(H, E, bias=True).to("cuda").half()
    with torch.no_grad():
        gate.weight.copy_(to_dev(w))
        gate.bias.copy_(to_dev(b))
    announce(f"fused router bias T={T} H={H} E={E} k={k}")
    wts, ids = mmfp4.fused_router_topk(to_dev(x), gate, k)
    _check_topk(ids, wts.float(), ref, k, True)
