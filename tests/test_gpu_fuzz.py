"""Seeded random-shape parity sweep of the FP4 and INT4 GEMMs (every kernel
family: strip, skinny with and without split-K, both prefill kernels) and of
the fused gate/up and QKV operators, against fp32 references built from the
bit-exact dequant.  Shapes cover ragged M and N, K not a multiple of 64, and
group sizes 8..256."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from gpu_helpers import TOL, announce, max_abs_rel, to_np

pytestmark = pytest.mark.gpu


def _shapes(seed, n):
    r = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        g = int(r.choice([8, 16, 32, 64, 128, 256]))
        K = g * int(r.integers(1, max(2, 4096 // g)))
        if K % 8:
            continue
        N = 4 * int(r.integers(1, 1200))
        M = int(r.choice([1, 2, 3, 7, 16, 17, 31, 32, 33, 64, 65, 127, 200, 300]))
        out.append((M, K, N, g))
    return out


@pytest.mark.parametrize("M,K,N,g", _shapes(123, 40))
def test_fuzz_fp4(M, K, N, g):
    import mmfp4
    gen = torch.Generator(device="cuda").manual_seed(M * 131 + K * 7 + N)
    w = (torch.randn((N, K), generator=gen, device="cuda") * 0.02).half()
    a = torch.randn((M, K), generator=gen, device="cuda").half()
    p, s = mmfp4.quantize_fp4(w, group_size=g)
    ref = a.float() @ mmfp4.dequant_fp4(p, s, K, N, g).float()
    announce(f"fuzz fp4 M={M} K={K} N={N} g={g}")
    out = mmfp4.marlin_gemm_fp4(a, p, s, g)
    assert max_abs_rel(to_np(out), to_np(ref)) <= TOL


@pytest.mark.parametrize("M,K,N,g", _shapes(456, 16))
def test_fuzz_int4(M, K, N, g):
    import mmfp4
    gen = torch.Generator(device="cuda").manual_seed(M * 17 + K + N * 3)
    w = (torch.randn((N, K), generator=gen, device="cuda") * 0.02).half()
    a = torch.randn((M, K), generator=gen, device="cuda").half()
    p, s, z = mmfp4.pack_u4_weights(w, group_size=g)
    ref = a.float() @ mmfp4.dequant_int4(p, s, z, K, N, g).float()
    announce(f"fuzz int4 M={M} K={K} N={N} g={g}")
    out = mmfp4.marlin_gemm_int4(a, p, s, z, g)
    assert max_abs_rel(to_np(out), to_np(ref)) <= TOL


@pytest.mark.parametrize("M,K,N,g", [s for s in _shapes(789, 30) if s[2] % 8 == 0
                                     and (s[0] <= 32 or s[1] % 64 == 0)][:12])
def test_fuzz_gate_up(M, K, N, g):
    import mmfp4
    gen = torch.Generator(device="cuda").manual_seed(M + K + N)
    wg = (torch.randn((N, K), generator=gen, device="cuda") * 0.02).half()
    wu = (torch.randn((N, K), generator=gen, device="cuda") * 0.02).half()
    a = torch.randn((M, K), generator=gen, device="cuda").half()
    gp, gs = mmfp4.quantize_fp4(wg, group_size=g)
    up, us = mmfp4.quantize_fp4(wu, group_size=g)
    hg = a.float() @ mmfp4.dequant_fp4(gp, gs, K, N, g).float()
    hu = a.float() @ mmfp4.dequant_fp4(up, us, K, N, g).float()
    announce(f"fuzz gate_up M={M} K={K} N={N} g={g}")
    out = mmfp4.mmfp4_fused_gate_up_marlin(a, gp, gs, up, us, g)
    assert max_abs_rel(to_np(out), to_np(torch.nn.functional.silu(hg) * hu)) <= TOL


def _rowpacked_shapes(seed, n):
    r = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        g = int(r.choice([64, 128, 256]))
        K = 256 * int(r.integers(1, 17))
        if K % g:
            continue
        N = 8 * int(r.integers(1, 700))
        M = int(r.choice([1, 5, 16, 17, 31, 33, 64, 100, 257, 600]))
        out.append((M, K, N, g))
    return out


@pytest.mark.parametrize("M,K,N,g", _rowpacked_shapes(321, 16))
def test_fuzz_rowpacked(M, K, N, g):
    """Row-packed [N, K/8] words read in place (decode and prefill kernels),
    the plain product and the gate/up pair, both scale layouts."""
    import mmfp4
    gen = torch.Generator(device="cuda").manual_seed(M * 7 + K * 3 + N)
    wg = (torch.randn((N, K), generator=gen, device="cuda") * 0.02).half()
    wu = (torch.randn((N, K), generator=gen, device="cuda") * 0.02).half()
    a = torch.randn((M, K), generator=gen, device="cuda").half()
    gp, gs = mmfp4.quantize_fp4(wg, group_size=g)
    up, us = mmfp4.quantize_fp4(wu, group_size=g)
    hg = a.float() @ mmfp4.dequant_fp4(gp, gs, K, N, g).float()
    hu = a.float() @ mmfp4.dequant_fp4(up, us, K, N, g).float()
    rg, ru = gp.t().contiguous(), up.t().contiguous()
    announce(f"fuzz row-packed M={M} K={K} N={N} g={g}")
    out = mmfp4.mmfp4_gemm_rowpacked(a, rg, gs, g)
    assert max_abs_rel(to_np(out), to_np(hg)) <= TOL
    out_t = mmfp4.mmfp4_gemm_rowpacked(a, rg, gs.t().contiguous(), g)
    assert torch.equal(out_t.view(torch.int16), out.view(torch.int16))
    pair = mmfp4.mmfp4_fused_gate_up(a, rg, gs, ru, us, g)
    assert max_abs_rel(to_np(pair), to_np(torch.nn.functional.silu(hg) * hu)) <= TOL


def _moe_shapes(seed, n):
    r = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        g = int(r.choice([32, 64, 128]))
        H = g * int(r.integers(1, max(2, 1024 // g)))
        I = g * int(r.integers(1, max(2, 512 // g)))
        if H % 8 or I % 8:
            continue
        E = int(r.choice([1, 3, 8, 17, 64]))
        k = int(r.integers(1, min(E, 8) + 1))
        T = int(r.choice([1, 5, 32, 97, 300, 700]))
        out.append((T, E, k, H, I, g))
    return out


@pytest.mark.parametrize("T,E,k,H,I,g", _moe_shapes(2024, 12))
def test_fuzz_moe_mlp(T, E, k, H, I, g):
    """Seeded random MoE shapes (decode- and prefill-sized groups, K not a
    multiple of 64, int32 and int64 ids, a few out-of-range ids) through
    moe_mlp_fp4, against an fp32 torch reference built from the bit-exact
    dequant: sum_j p_j * SwiGLU-MLP_{e_j}(x), dropped slots contributing 0."""
    import mmfp4
    gen = torch.Generator(device="cuda").manual_seed(T * 7 + E * 3 + H + I + k)
    gp, gs, dp, ds = [], [], [], []
    for _ in range(E):
        w = (torch.randn((2 * I, H), generator=gen, device="cuda") * 0.02).half()
        p, s = mmfp4.quantize_fp4(w, group_size=g)
        gp.append(p); gs.append(s)
        w = (torch.randn((H, I), generator=gen, device="cuda") * 0.02).half()
        p, s = mmfp4.quantize_fp4(w, group_size=g)
        dp.append(p); ds.append(s)
    GP, GS, DP, DS = (torch.stack(v) for v in (gp, gs, dp, ds))
    x = torch.randn((T, H), generator=gen, device="cuda").half()
    logits = torch.randn((T, E), generator=gen, device="cuda")
    probs, ids = torch.topk(torch.softmax(logits, -1), k, -1)
    probs = probs / probs.sum(-1, keepdim=True)
    drop = torch.rand((T, k), generator=gen, device="cuda") < 0.05
    ids = torch.where(drop, torch.full_like(ids, E + 3), ids)
    if T % 2:
        ids = ids.to(torch.int32)
    ref = torch.zeros((T, H), dtype=torch.float32, device="cuda")
    xf = x.float()
    for e in range(E):
        wgu = mmfp4.dequant_fp4(GP[e], GS[e], H, 2 * I, g).float()
        wdn = mmfp4.dequant_fp4(DP[e], DS[e], I, H, g).float()
        h = xf @ wgu
        y = (torch.nn.functional.silu(h[:, :I]) * h[:, I:]) @ wdn
        w_e = (probs * (ids == e)).sum(-1, keepdim=True)
        ref += w_e * y
    announce(f"fuzz moe T={T} E={E} k={k} H={H} I={I} g={g}")
    out = mmfp4.moe_mlp_fp4(x, GP, GS, DP, DS, ids, probs, g)
    assert max_abs_rel(to_np(out), to_np(ref)) <= TOL
