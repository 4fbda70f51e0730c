"""GPU parity of the MoE path: device sort exact vs the oracle, grouped expert
GEMM + SwiGLU + combine vs the oracle's per-token fp32 brute force."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from gpu_helpers import TOL, announce, max_abs_rel, to_dev, to_np
from oracle import fp4 as ofp4
from oracle import moe as omoe

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("T,k,E", [(3, 2, 3), (1, 1, 4), (32, 8, 128), (1024, 8, 128),
                                   (37, 3, 1000), (2000, 2, 8), (70, 1, 1), (8192, 8, 1024),
                                   (0, 4, 16)])
@pytest.mark.parametrize("dtype", [np.int32, np.int64])
def test_sort_exact(rng, T, k, E, dtype):
    import mmfp4
    ids = rng.integers(0, E, (T, k)).astype(np.int32)
    if E > 4:
        ids[ids == 1] = 0          # leave some experts empty
    announce(f"moe sort T={T} k={k} E={E} {np.dtype(dtype).name}")
    s, off, inv = mmfp4.group_tokens_by_expert(to_dev(ids.astype(dtype)), E)
    rs, roff, rinv = omoe.group_tokens_by_expert(ids, E)
    assert np.array_equal(to_np(s), rs)
    assert np.array_equal(to_np(off), roff)
    assert np.array_equal(to_np(inv), rinv)


def _experts(rng, E, K, N, g):
    ps, ss = [], []
    for _ in range(E):
        w = rng.normal(0, 0.02, (N, K)).astype(np.float16)
        p, s = ofp4.quantize_fp4(w, g)
        ps.append(p)
        ss.append(s)
    return np.stack(ps), np.stack(ss)


def test_moe_expert_gemm_vs_oracle(rng):
    import mmfp4
    E, T, k, K, N, g = 8, 20, 2, 256, 192, 128
    P, S = _experts(rng, E, K, N, g)
    x = rng.normal(0, 1, (T, K)).astype(np.float16)
    ids, probs = omoe.router_topk(rng.normal(0, 1, (T, E)), k)
    ref = np.zeros((T, N), np.float32)
    for t in range(T):
        for j in range(k):
            e = ids[t, j]
            ref[t] += probs[t, j] * (x[t].astype(np.float32) @ ofp4.dequant_fp4_f32(P[e], S[e], g))
    announce("moe_expert_gemm_fp4 small")
    out = mmfp4.moe_expert_gemm_fp4(to_dev(x), to_dev(P), to_dev(S), to_dev(ids), to_dev(probs), g)
    assert max_abs_rel(to_np(out), ref) <= TOL


@pytest.mark.parametrize("E,T,k,H,I", [(8, 16, 2, 256, 128), (16, 40, 4, 512, 256),
                                       (128, 32, 8, 2048, 768), (8, 256, 2, 256, 128),
                                       (16, 200, 4, 512, 384), (16, 100, 4, 256, 128)])
def test_moe_mlp_vs_oracle(rng, E, T, k, H, I):
    import mmfp4
    g = 128
    GU, GS = _experts(rng, E, H, 2 * I, g)
    DP, DS = _experts(rng, E, I, H, g)
    x = rng.normal(0, 1, (T, H)).astype(np.float16)
    ids, probs = omoe.router_topk(rng.normal(0, 1, (T, E)).astype(np.float32), k)
    ref = omoe.moe_forward_ref(x, GU, GS, DP, DS, ids, probs, g)
    announce(f"moe mlp E={E} T={T} k={k} H={H} I={I}")
    out = mmfp4.moe_mlp_fp4(to_dev(x), to_dev(GU), to_dev(GS), to_dev(DP), to_dev(DS),
                            to_dev(ids), to_dev(probs), g)
    assert max_abs_rel(to_np(out), ref) <= TOL


@pytest.mark.parametrize("g", [32, 64, 128])
def test_moe_mlp_prefill_skewed(rng, g):
    """MFMA tile path with ragged groups: expert 0 takes 300 of 400 tokens
    (two full 128-row tiles and a partial one), expert 5 none, the rest a few
    dozen; group sizes below, at and above the 64-k chunk."""
    import mmfp4
    E, T, k, H, I = 6, 400, 2, 256, 128
    GU, GS = _experts(rng, E, H, 2 * I, g)
    DP, DS = _experts(rng, E, I, H, g)
    x = rng.normal(0, 1, (T, H)).astype(np.float16)
    ids = np.zeros((T, k), np.int32)
    ids[:, 0] = np.where(np.arange(T) < 300, 0, rng.integers(1, 5, T))
    ids[:, 1] = (ids[:, 0] + rng.integers(1, 4, T)) % 5
    ids[:, 1] = np.where(ids[:, 1] == ids[:, 0], 4, ids[:, 1])
    assert (ids[:, 0] != ids[:, 1]).all() and not (ids == 5).any()
    probs = rng.uniform(0.1, 1.0, (T, k)).astype(np.float32)
    probs /= probs.sum(1, keepdims=True)
    ref = omoe.moe_forward_ref(x, GU, GS, DP, DS, ids, probs, g)
    announce(f"moe mlp prefill skewed g={g}")
    out = mmfp4.moe_mlp_fp4(to_dev(x), to_dev(GU), to_dev(GS), to_dev(DP), to_dev(DS),
                            to_dev(ids), to_dev(probs), g)
    assert max_abs_rel(to_np(out), ref) <= TOL


def test_moe_expert_gemm_prefill_vs_oracle(rng):
    """moe_expert_gemm_fp4 with prefill-sized groups (gathered rows, no
    activation) against the per-token fp32 brute force."""
    import mmfp4
    E, T, k, K, N, g = 4, 200, 2, 256, 200, 128
    P, S = _experts(rng, E, K, N, g)
    x = rng.normal(0, 1, (T, K)).astype(np.float16)
    ids, probs = omoe.router_topk(rng.normal(0, 1, (T, E)), k)
    W = [ofp4.dequant_fp4_f32(P[e], S[e], g) for e in range(E)]
    ref = np.zeros((T, N), np.float32)
    for t in range(T):
        for j in range(k):
            ref[t] += probs[t, j] * (x[t].astype(np.float32) @ W[ids[t, j]])
    announce("moe_expert_gemm_fp4 prefill")
    out = mmfp4.moe_expert_gemm_fp4(to_dev(x), to_dev(P), to_dev(S), to_dev(ids), to_dev(probs), g)
    assert max_abs_rel(to_np(out), ref) <= TOL


def test_moe_prefill_config5_properties():
    """T=1024 prefill at the Qwen3-30B-A3B shape: deterministic, and equal to
    the same pipeline run expert-by-expert through the dense GEMM."""
    import mmfp4
    E, T, k, H, I, g = 128, 1024, 8, 2048, 768, 128
    gen = torch.Generator(device="cuda").manual_seed(11)
    wgu = (torch.randn((E, 2 * I, H), generator=gen, device="cuda") * 0.02).half()
    wdn = (torch.randn((E, H, I), generator=gen, device="cuda") * 0.02).half()
    GU = torch.empty((E, H // 8, 2 * I), dtype=torch.int32, device="cuda")
    GS = torch.empty((E, H // g, 2 * I), dtype=torch.float16, device="cuda")
    DP = torch.empty((E, I // 8, H), dtype=torch.int32, device="cuda")
    DS = torch.empty((E, I // g, H), dtype=torch.float16, device="cuda")
    for e in range(E):
        GU[e], GS[e] = mmfp4.quantize_fp4(wgu[e], group_size=g)
        DP[e], DS[e] = mmfp4.quantize_fp4(wdn[e], group_size=g)
    x = torch.randn((T, H), generator=gen, device="cuda").half()
    logits = torch.randn((T, E), generator=gen, device="cuda")
    p = torch.softmax(logits, -1)
    probs, ids = torch.topk(p, k, -1)
    probs = probs / probs.sum(-1, keepdim=True)
    announce("moe prefill T=1024 full config")
    out = mmfp4.moe_mlp_fp4(x, GU, GS, DP, DS, ids, probs, g)
    out2 = mmfp4.moe_mlp_fp4(x, GU, GS, DP, DS, ids, probs, g)
    assert torch.equal(out.view(torch.int16), out2.view(torch.int16))
    ref = torch.zeros((T, H), dtype=torch.float32, device="cuda")
    for e in range(E):
        tok, slot = torch.nonzero(ids == e, as_tuple=True)
        if tok.numel() == 0:
            continue
        h = mmfp4.marlin_gemm_fp4(x[tok], GU[e], GS[e], g).float()
        a = (torch.nn.functional.silu(h[:, :I]) * h[:, I:]).half()
        y = mmfp4.marlin_gemm_fp4(a, DP[e], DS[e], g).float()
        ref.index_add_(0, tok, y * probs[tok, slot, None].float())
    assert max_abs_rel(to_np(out), to_np(ref)) <= TOL


def test_moe_prefill_config5_vs_oracle_subset():
    """Config 5 at T=1024 (Qwen3-30B-A3B: E=128, H=2048, I=768, top-8) against
    the oracle's per-token fp32 brute force on a seeded subset of 24 tokens
    (each token's output depends only on its own routing, so the subset is
    exact).  Weights come from the GPU quantizer, which is bit-exact with the
    oracle's (test_gpu_dequant_quant.py)."""
    import mmfp4
    E, T, k, H, I, g = 128, 1024, 8, 2048, 768, 128
    gen = torch.Generator(device="cuda").manual_seed(12)
    GU = torch.empty((E, H // 8, 2 * I), dtype=torch.int32, device="cuda")
    GS = torch.empty((E, H // g, 2 * I), dtype=torch.float16, device="cuda")
    DP = torch.empty((E, I // 8, H), dtype=torch.int32, device="cuda")
    DS = torch.empty((E, I // g, H), dtype=torch.float16, device="cuda")
    for e in range(E):
        w1 = (torch.randn((2 * I, H), generator=gen, device="cuda") * 0.02).half()
        w2 = (torch.randn((H, I), generator=gen, device="cuda") * 0.02).half()
        GU[e], GS[e] = mmfp4.quantize_fp4(w1, group_size=g)
        DP[e], DS[e] = mmfp4.quantize_fp4(w2, group_size=g)
    x = torch.randn((T, H), generator=gen, device="cuda").half()
    logits = torch.randn((T, E), generator=gen, device="cuda")
    probs, ids = mmfp4.router_softmax_topk(logits, k)
    announce("moe prefill T=1024 vs oracle subset")
    out = to_np(mmfp4.moe_mlp_fp4(x, GU, GS, DP, DS, ids, probs, g))
    sub = np.random.default_rng(5).choice(T, 24, replace=False)
    ids_s = to_np(ids)[sub]
    ref = omoe.moe_forward_ref(to_np(x)[sub], to_np(GU).view(np.uint32), to_np(GS),
                               to_np(DP).view(np.uint32), to_np(DS), ids_s, to_np(probs)[sub], g)
    assert max_abs_rel(out[sub], ref) <= TOL


@pytest.mark.parametrize("T,k,E", [(5, 2, 4), (256, 8, 128), (1, 4, 64)])
def test_gpu_grouping_api(rng, T, k, E):
    """moe/gpu_grouping.py surface: every variant gives the oracle's stable order;
    the manager's gather/scatter match the per-token weighted sum."""
    import mmfp4
    ids = rng.integers(0, E, (T, k)).astype(np.int64)
    announce(f"gpu_grouping T={T} k={k} E={E}")
    rs, roff, rinv = omoe.group_tokens_by_expert(ids, E)
    d_ids = to_dev(ids)
    E_inf = int(ids.max()) + 1
    for res, e_want in [(mmfp4.group_tokens_by_expert_fast(d_ids, E), E),
                        (mmfp4.group_tokens_by_expert_fast(d_ids), E_inf),
                        (mmfp4.group_tokens_by_expert_gpu_optimized(d_ids, None, E), E),
                        (mmfp4.group_tokens_by_expert_auto(d_ids, num_experts=E), E)]:
        assert res.num_experts == e_want and res.num_tokens == T and res.top_k == k
        assert res.total_assignments == T * k
        assert np.array_equal(to_np(res.sorted_token_indices), rs // k)
        assert np.array_equal(to_np(res.sorted_expert_indices), rs % k)
        assert np.array_equal(to_np(res.expert_offsets)[:e_want + 1], roff[:e_want + 1])
        assert np.array_equal(to_np(res.inverse_indices), rinv)
    grp = mmfp4.GPUExpertGrouping(E, device="cuda")
    res = grp.group(torch.from_numpy(ids))          # host ids are moved to the device
    h = rng.normal(0, 1, (T, 64)).astype(np.float16)
    xs = grp.gather_activations(to_dev(h), res)
    assert np.array_equal(to_np(xs), h[rs // k])
    p = rng.random((T, k)).astype(np.float32)
    out = to_np(grp.scatter_outputs(xs, to_dev(p), res)).astype(np.float32)
    ref = (h.astype(np.float32)[:, None, :] * p[:, :, None]).sum(1)
    assert max_abs_rel(out, ref) <= TOL
    with pytest.raises(ValueError):
        mmfp4.GPUExpertGrouping(E, device="cpu")



@pytest.mark.parametrize("E,T,k,H,I,i64", [(128, 32, 8, 2048, 768, True), (16, 1, 4, 256, 128, False),
                                          (64, 256, 8, 512, 256, True), (8, 3, 8, 256, 128, False),
                                          (1, 4, 1, 384, 128, False), (128, 5, 8, 2048, 768, False),
                                          (256, 24, 8, 512, 256, True), (256, 512, 8, 256, 128, False),
                                          (64, 1100, 8, 256, 128, True), (32, 2500, 4, 256, 128, False)])
def test_moe_mlp_one_call_matches_steps(rng, E, T, k, H, I, i64):
    """mm_moe_mlp_fp4 (one library call) is bit-identical to the sort ->
    grouped GEMM -> grouped GEMM -> combine steps on the same inputs (above
    8192 assignments the call sorts in blocks of 1024 over two launches, the
    step path in one block)."""
    import mmfp4
    from mmfp4 import moe_dispatch as md
    g = 128
    GU, GS = _experts(rng, E, H, 2 * I, g)
    DP, DS = _experts(rng, E, I, H, g)
    x = to_dev(rng.normal(0, 1, (T, H)).astype(np.float16))
    ids, probs = omoe.router_topk(rng.normal(0, 1, (T, E)).astype(np.float32), k)
    dids = to_dev(ids.astype(np.int64 if i64 else np.int32))
    dp = to_dev(probs)
    announce(f"moe mlp one call vs steps E={E} T={T} k={k} i64={i64}")
    fused = mmfp4.moe_mlp_fp4(x, to_dev(GU), to_dev(GS), to_dev(DP), to_dev(DS), dids, dp, g)
    s_idx, offs, inv = md._sort(dids, E)
    a = md._grouped(x, s_idx, offs, True, k, T, to_dev(GU), to_dev(GS), g, 1)
    y = md._grouped(a, s_idx, offs, False, k, T, to_dev(DP), to_dev(DS), g, 0)
    ref = md.scatter_expert_outputs(y, dp, md.MoEDispatchInfo(s_idx, s_idx, offs, inv, T, k, E, s_idx))
    assert torch.equal(fused, ref)


def test_moe_mlp_back_to_back_calls(rng):
    """Consecutive decode-sized calls of different sizes on one stream (the
    sort, grouped GEMMs and combine reuse nothing between calls) each match
    their step-by-step result."""
    import mmfp4
    from mmfp4 import moe_dispatch as md
    E, H, I, k, g = 32, 512, 256, 4, 128
    GU, GS = _experts(rng, E, H, 2 * I, g)
    DP, DS = _experts(rng, E, I, H, g)
    dGU, dGS, dDP, dDS = to_dev(GU), to_dev(GS), to_dev(DP), to_dev(DS)
    outs, refs = [], []
    for T in (16, 3, 16, 1):
        x = to_dev(rng.normal(0, 1, (T, H)).astype(np.float16))
        ids, probs = omoe.router_topk(rng.normal(0, 1, (T, E)).astype(np.float32), k)
        dids, dp = to_dev(ids.astype(np.int32)), to_dev(probs)
        announce(f"moe mlp back-to-back T={T}")
        outs.append(mmfp4.moe_mlp_fp4(x, dGU, dGS, dDP, dDS, dids, dp, g))
        s_idx, offs, inv = md._sort(dids, E)
        a = md._grouped(x, s_idx, offs, True, k, T, dGU, dGS, g, 1)
        y = md._grouped(a, s_idx, offs, False, k, T, dDP, dDS, g, 0)
        refs.append(md.scatter_expert_outputs(
            y, dp, md.MoEDispatchInfo(s_idx, s_idx, offs, inv, T, k, E, s_idx)))
    for o, r in zip(outs, refs):
        assert torch.equal(o, r)


def test_moe_mlp_all_dropped_tokens_and_scale_dtypes(rng):
    """Decode-sized groups: tokens whose every id is outside [0, E) come out
    as exact zero rows, the others match the oracle with their dropped slots
    contributing nothing; fp32 and bf16 scales (converted copies inside the
    call, which must outlive the launches) give the same bits as fp16
    scales."""
    import mmfp4
    E, T, k, H, I, g = 16, 24, 4, 512, 256, 128
    GU, GS = _experts(rng, E, H, 2 * I, g)
    DP, DS = _experts(rng, E, I, H, g)
    x = rng.normal(0, 1, (T, H)).astype(np.float16)
    ids, probs = omoe.router_topk(rng.normal(0, 1, (T, E)).astype(np.float32), k)
    ids = ids.astype(np.int64)
    bad = np.zeros((T, k), bool)
    bad[[3, 7, 20]] = True                       # every slot of three tokens
    bad[5, 1] = bad[11, 0] = bad[11, 3] = True   # some slots of others
    ids[bad] = rng.choice([-1, E, E + 3], size=int(bad.sum()))
    safe = np.where(bad, 0, ids).astype(np.int32)
    ref = omoe.moe_forward_ref(x, GU, GS, DP, DS, safe, np.where(bad, 0.0, probs).astype(np.float32), g)
    announce("moe mlp all-dropped tokens")
    dx, dGU, dDP, dids, dp = to_dev(x), to_dev(GU), to_dev(DP), to_dev(ids), to_dev(probs)
    out = mmfp4.moe_mlp_fp4(dx, dGU, to_dev(GS), dDP, to_dev(DS), dids, dp, g)
    o = to_np(out)
    assert np.array_equal(o[[3, 7, 20]], np.zeros((3, H), np.float16))
    assert max_abs_rel(o, ref) <= TOL
    for dt in (torch.float32, torch.bfloat16):
        gs32, ds32 = to_dev(GS).to(dt), to_dev(DS).to(dt)
        if dt == torch.bfloat16:                 # bf16 rounds the scales: compare with those
            gs16, ds16 = gs32.half(), ds32.half()
            want = mmfp4.moe_mlp_fp4(dx, dGU, gs16, dDP, ds16, dids, dp, g)
        else:
            want = out
        got = mmfp4.moe_mlp_fp4(dx, dGU, gs32, dDP, ds32, dids, dp, g)
        assert torch.equal(got, want), dt


@pytest.mark.parametrize("T", [32, 1024])
def test_moe_mlp_out_aliases_hidden(rng, T):
    """mm_moe_mlp_fp4 with out == hidden (in place through the C ABI): the
    combine, the only launch that writes out, runs after every read of the
    hidden states, so the result matches the out-of-place call."""
    import mmfp4
    from mmfp4 import _lib
    E, k, H, I, g = 32, 8, 512, 256, 128
    GU, GS = _experts(rng, E, H, 2 * I, g)
    DP, DS = _experts(rng, E, I, H, g)
    ids, probs = omoe.router_topk(rng.normal(0, 1, (T, E)).astype(np.float32), k)
    x = to_dev(rng.normal(0, 1, (T, H)).astype(np.float16))
    dGU, dGS, dDP, dDS = to_dev(GU), to_dev(GS), to_dev(DP), to_dev(DS)
    dids, dp = to_dev(ids.astype(np.int32)), to_dev(probs)
    announce(f"moe mlp in place T={T}")
    want = mmfp4.moe_mlp_fp4(x, dGU, dGS, dDP, dDS, dids, dp, g)
    xin = x.clone()
    act = torch.empty((T * k, I), dtype=torch.float16, device="cuda")
    y = torch.empty((T * k, H), dtype=torch.float16, device="cuda")
    sort_buf = torch.empty(E + 1 + 2 * T * k, dtype=torch.int32, device="cuda")
    _lib.call("mm_moe_mlp_fp4", _lib.ptr(xin), _lib.ptr(dids), 0, _lib.ptr(dp), T, k, E, H, I,
              _lib.ptr(dGU), _lib.ptr(dGS), _lib.ptr(dDP), _lib.ptr(dDS), g, _lib.ptr(act),
              _lib.ptr(y), _lib.ptr(sort_buf), _lib.ptr(xin), _lib.stream_of(xin))
    assert torch.equal(xin, want)
