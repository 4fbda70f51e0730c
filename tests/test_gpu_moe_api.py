"""GPU parity of the expert-MLP entry points with the reference's names and
of the shared-expert path, against the oracle's fp32 brute force:

* _fused_expert_mlp (moe_dispatch.py:1241-1431), Marlin and row-packed
  weight orientations;
* moe_shared_expert_fp4 / moe_add_shared_expert_fp4 (kernels/moe.py:442-582,
  858-930);
* moe_fused_dispatch_shared_fp4 (kernels/moe.py:742-856) and
  FusedMoEDispatcher (moe_dispatch.py:1111-1238): routed experts plus a
  shared expert, decode- and prefill-sized groups;
* dispatch_experts_batched (moe_dispatch.py:2546-2676) over expert modules,
  including the stacked-weight cache following a weight reload."""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn as nn

from gpu_helpers import TOL, announce, max_abs_rel, to_dev, to_np
from oracle import fp4 as ofp4
from oracle import moe as omoe

pytestmark = pytest.mark.gpu


def _expert(rng, H, I, g):
    gu = rng.normal(0, 0.02, (2 * I, H)).astype(np.float16)
    dn = rng.normal(0, 0.02, (H, I)).astype(np.float16)
    gp, gs = ofp4.quantize_fp4(gu, g)             # [H/8, 2I], [H/g, 2I]
    dp, ds = ofp4.quantize_fp4(dn, g)             # [I/8, H], [I/g, H]
    return gp, gs, dp, ds


def _experts(rng, E, H, I, g):
    parts = [_expert(rng, H, I, g) for _ in range(E)]
    return tuple(np.stack([p[i] for p in parts]) for i in range(4))


@pytest.mark.parametrize("M", [1, 7, 64, 300])
@pytest.mark.parametrize("rowpacked", [False, True])
def test_fused_expert_mlp(rng, M, rowpacked):
    import mmfp4
    H, I, g = 512, 256, 128
    gp, gs, dp, ds = _expert(rng, H, I, g)
    x = rng.normal(0, 1, (M, H)).astype(np.float16)
    ref = omoe.expert_mlp_ref(x, gp, gs, dp, ds, g)
    gpt = np.ascontiguousarray(gp.T) if rowpacked else gp
    dpt = np.ascontiguousarray(dp.T) if rowpacked else dp
    announce(f"_fused_expert_mlp M={M} rowpacked={rowpacked}")
    out = mmfp4._fused_expert_mlp(to_dev(x), to_dev(gpt), to_dev(gs), to_dev(dpt), to_dev(ds), g)
    assert out.shape == (M, H) and out.dtype == torch.float16
    assert max_abs_rel(to_np(out), ref) <= TOL
    out32 = mmfp4._fused_expert_mlp(to_dev(x).float(), to_dev(gp), to_dev(gs), to_dev(dp),
                                    to_dev(ds), g)
    assert out32.dtype == torch.float32


def test_shared_expert_and_add(rng):
    import mmfp4
    H, I, g, T = 256, 384, 128, 20
    gp, gs, dp, ds = _expert(rng, H, I, g)
    x = rng.normal(0, 1, (2, T // 2, H)).astype(np.float16)
    ref = omoe.expert_mlp_ref(x.reshape(T, H), gp, gs, dp, ds, g)
    announce("moe_shared_expert_fp4 / moe_add_shared_expert_fp4")
    out = mmfp4.moe_shared_expert_fp4(to_dev(x), to_dev(gp), to_dev(gs), to_dev(dp), to_dev(ds),
                                      g, shared_prob=0.5)
    assert out.shape == (2, T // 2, H)
    assert max_abs_rel(to_np(out).reshape(T, H), 0.5 * ref) <= TOL
    base = rng.normal(0, 1, (T, H)).astype(np.float16)
    out2 = mmfp4.moe_add_shared_expert_fp4(to_dev(x), to_dev(base.reshape(2, T // 2, H)),
                                           to_dev(gp), to_dev(gs), to_dev(dp), to_dev(ds), g)
    assert max_abs_rel(to_np(out2).reshape(T, H), ref + base.astype(np.float32)) <= TOL


@pytest.mark.parametrize("T,E,k", [(32, 16, 4), (1, 8, 2), (400, 6, 2), (64, 128, 8), (2800, 8, 2)])
def test_fused_dispatch_shared(rng, T, E, k):
    """Routed experts plus a shared expert in the same grouped launches; the
    (400, 6, 2) case gives every group prefill-sized row counts, and the
    shared group holds all T rows."""
    import mmfp4
    H, I, g = 256, 128, 128
    GU, GS, DP, DS = _experts(rng, E, H, I, g)
    sgp, sgs, sdp, sds = _expert(rng, H, I, g)
    x = rng.normal(0, 1, (T, H)).astype(np.float16)
    ids, probs = omoe.router_topk(rng.normal(0, 1, (T, E)), k, renormalize=False)
    ref = omoe.moe_forward_ref(x, GU, GS, DP, DS, ids, probs, g) + \
        omoe.expert_mlp_ref(x, sgp, sgs, sdp, sds, g)
    announce(f"moe_fused_dispatch_shared_fp4 T={T} E={E} k={k}")
    for ids_t in (to_dev(ids), to_dev(ids.astype(np.int64))):
        out = mmfp4.moe_fused_dispatch_shared_fp4(
            to_dev(x), to_dev(sgp), to_dev(sgs), to_dev(sdp), to_dev(sds), to_dev(GU),
            to_dev(GS), to_dev(DP), to_dev(DS), ids_t, to_dev(probs), g)
        assert out.shape == (T, H)
        assert max_abs_rel(to_np(out), ref) <= TOL
    # FusedMoEDispatcher: softmax -> top-k (no renormalisation) of the logits
    logits = rng.normal(0, 1, (T, E)).astype(np.float32)
    lid, lp = omoe.router_topk(logits, k, renormalize=False)
    ref2 = omoe.moe_forward_ref(x, GU, GS, DP, DS, lid, lp, g) + \
        omoe.expert_mlp_ref(x, sgp, sgs, sdp, sds, g)
    disp = mmfp4.FusedMoEDispatcher(E, k, to_dev(GU), to_dev(GS), to_dev(DP), to_dev(DS),
                                    to_dev(sgp), to_dev(sgs), to_dev(sdp), to_dev(sds), g)
    out2 = disp(to_dev(x), to_dev(logits))
    assert max_abs_rel(to_np(out2), ref2) <= TOL
    out3 = disp(to_dev(x).reshape(1, T, H), to_dev(logits))
    assert out3.shape == (1, T, H) and torch.equal(out3[0], out2)


class _Expert(nn.Module):
    def __init__(self, gate, up, down, g):
        super().__init__()
        self.gate_proj, self.up_proj, self.down_proj = gate, up, down
        self.group_size = g


def _layer(mmfp4, packed, scales, g):
    # Marlin [in/8, out] -> the row-packed layer's [out, in/8]; scales [in/g, out]
    return mmfp4.MMFP4Linear(to_dev(np.ascontiguousarray(packed.T).view(np.int32)),
                             to_dev(scales), None, g)


@pytest.mark.parametrize("T,k", [(32, 8), (512, 8)])
def test_dispatch_experts_batched(rng, T, k):
    import mmfp4
    E, H, I, g = 16, 256, 128, 128
    GU, GS, DP, DS = _experts(rng, E, H, I, g)
    experts = nn.ModuleList([
        _Expert(_layer(mmfp4, GU[e][:, :I], GS[e][:, :I], g),
                _layer(mmfp4, GU[e][:, I:], GS[e][:, I:], g),
                _layer(mmfp4, DP[e], DS[e], g), g) for e in range(E)])
    x = rng.normal(0, 1, (T, H)).astype(np.float16)
    ids, _ = omoe.router_topk(rng.normal(0, 1, (T, E)), k)
    info = mmfp4.group_tokens_by_expert_full(to_dev(ids), E)
    xs = mmfp4.gather_for_experts(to_dev(x), info)
    announce(f"dispatch_experts_batched T={T} k={k}")
    y = mmfp4.dispatch_experts_batched(xs, experts, info, E)
    s, off, _ = omoe.group_tokens_by_expert(ids, E)
    xs_ref = omoe.gather_for_experts(x, s, k)
    ref = np.zeros((T * k, H), np.float32)
    for e in range(E):
        if off[e + 1] > off[e]:
            ref[off[e]:off[e + 1]] = omoe.expert_mlp_ref(xs_ref[off[e]:off[e + 1]], GU[e], GS[e],
                                                         DP[e], DS[e], g)
    assert y.shape == (T * k, H)
    assert max_abs_rel(to_np(y), ref) <= TOL
    # a weight written in place (load_state_dict) is picked up by the cache
    e0 = int(ids[0, 0])
    new_gp, new_gs, new_dp, new_ds = _expert(rng, H, I, g)
    experts[e0].down_proj.load_state_dict(
        {"packed_weights": to_dev(np.ascontiguousarray(new_dp.T).view(np.int32)),
         "scales": to_dev(new_ds)}, strict=False)
    y2 = mmfp4.dispatch_experts_batched(xs, experts, info, E)
    a, b = int(off[e0]), int(off[e0 + 1])
    ref[a:b] = omoe.expert_mlp_ref(xs_ref[a:b], GU[e0], GS[e0], new_dp, new_ds, g)
    assert max_abs_rel(to_np(y2), ref) <= TOL


def _proj(rng, K, N, g):
    w = rng.normal(0, 0.02, (N, K)).astype(np.float16)
    return ofp4.quantize_fp4(w, g)                 # [K/8, N], [K/g, N]


@pytest.mark.parametrize("T,E,k,i64", [(32, 16, 4, False), (512, 8, 2, True), (1, 4, 3, False),
                                        (3000, 8, 2, False)])
def test_shared_expert_fused_fp4(rng, T, E, k, i64):
    """moe_shared_expert_fused_fp4 (kernels/moe.py:182-329): one projection,
    out = x @ W_sh + sum_j p_j x @ W_e(j), against the fp32 brute force; one
    slot per token is given an out-of-range id, which contributes nothing
    (T=512 gives the routed groups prefill-sized row counts)."""
    import mmfp4
    H, I, g = 512, 256, 128
    sp, ss = _proj(rng, H, I, g)
    parts = [_proj(rng, H, I, g) for _ in range(E)]
    RP, RS = np.stack([q[0] for q in parts]), np.stack([q[1] for q in parts])
    x = rng.normal(0, 1, (T, H)).astype(np.float16)
    ids, probs = omoe.router_topk(rng.normal(0, 1, (T, E)), k)
    ids = ids.astype(np.int64)
    ids[:, -1] = np.where(np.arange(T) % 2 == 0, -1, E)       # dropped slots
    ref = ofp4.gemm_fp4_ref(x, sp, ss, g).astype(np.float32)
    for t in range(T):
        for j in range(k):
            e = int(ids[t, j])
            if 0 <= e < E:
                ref[t] += probs[t, j] * ofp4.gemm_fp4_ref(x[t:t + 1], RP[e], RS[e], g)[0]
    dids = to_dev(ids if i64 else ids.astype(np.int32))
    announce(f"moe_shared_expert_fused_fp4 T={T} E={E} k={k} i64={i64}")
    out = mmfp4.moe_shared_expert_fused_fp4(to_dev(x.reshape(1, T, H)), to_dev(sp), to_dev(ss),
                                            to_dev(RP), to_dev(RS), to_dev(probs), dids, g)
    assert out.shape == (1, T, I) and out.dtype == torch.float16
    assert max_abs_rel(to_np(out[0]), ref) <= TOL


@pytest.mark.parametrize("T,E,k", [(32, 16, 4), (600, 8, 2), (2100, 8, 4)])
def test_dropped_expert_ids(rng, T, E, k):
    """Ids outside [0, E): the sort places them after every expert's rows in
    index order (the stable argsort of the ids with those mapped to E), and
    offsets[E] counts the valid ones; moe_mlp_fp4 and moe_expert_gemm_fp4
    give them no contribution."""
    import mmfp4
    H, I, g = 256, 128, 128
    ids, probs = omoe.router_topk(rng.normal(0, 1, (T, E)), k)
    ids = ids.astype(np.int64)
    bad = rng.random((T, k)) < 0.2
    ids[bad] = rng.choice([-1, -7, E, E + 5, 1 << 40], size=int(bad.sum()))
    announce(f"dropped ids sort T={T} E={E} k={k}")
    s, o, inv = mmfp4.group_tokens_by_expert(to_dev(ids), E)
    keys = np.where((ids >= 0) & (ids < E), ids, E).reshape(-1)
    want = np.argsort(keys, kind="stable")
    assert np.array_equal(to_np(s), want)
    assert np.array_equal(to_np(inv)[want], np.arange(T * k))
    cnt = np.bincount(keys, minlength=E + 1)
    assert np.array_equal(to_np(o), np.concatenate([[0], np.cumsum(cnt[:E])]))
    # the MLP and the single-projection entry: dropped slots contribute zero
    GU, GS, DP, DS = _experts(rng, E, H, I, g)
    x = rng.normal(0, 1, (T, H)).astype(np.float16)
    safe = np.where(bad, 0, ids).astype(np.int32)
    p0 = np.where(bad, 0.0, probs).astype(np.float32)
    ref = omoe.moe_forward_ref(x, GU, GS, DP, DS, safe, p0, g)
    out = mmfp4.moe_mlp_fp4(to_dev(x), to_dev(GU), to_dev(GS), to_dev(DP), to_dev(DS),
                            to_dev(ids), to_dev(probs), g)
    assert max_abs_rel(to_np(out), ref) <= TOL
    WP, WS = GU[:, :, :I], np.ascontiguousarray(GS[:, :, :I])
    WP = np.ascontiguousarray(WP)
    ref1 = np.zeros((T, I), np.float32)
    for t in range(T):
        for j in range(k):
            if not bad[t, j]:
                ref1[t] += probs[t, j] * ofp4.gemm_fp4_ref(x[t:t + 1], WP[ids[t, j]],
                                                           WS[ids[t, j]], g)[0]
    out1 = mmfp4.moe_expert_gemm_fp4(to_dev(x), to_dev(WP), to_dev(WS), to_dev(ids),
                                     to_dev(probs), g)
    assert max_abs_rel(to_np(out1), ref1) <= TOL
