"""HIP graph capture of the hot path.

The library's launches take the caller's stream and allocate nothing once a
stream's workspace exists, and the split-K arrival counters are returned to
zero by the last block of each tile (no memset node).  So a caller can
capture them: the four Llama-layer GEMMs (two-slab, skinny and split-K
hand-off at M=1; the pipelined prefill kernel with and without its K split
at M=128) and the MoE MLP (sort, grouped GEMMs, combine; decode- and
prefill-sized groups), and the row-packed GEMM and gate/up pair, are
captured once and replayed several times, with new inputs copied into the
captured buffers and eager launches of the same entry points in between.  Every replay must equal the eager result on the
same inputs bit for bit (the kernels are deterministic)."""

from __future__ import annotations

import pytest
import torch

from gpu_helpers import announce

pytestmark = pytest.mark.gpu

G = 128
LAYER = [(4096, 6144), (4096, 4096), (4096, 14336), (14336, 4096)]


def _words(gen, K, N):
    p = torch.randint(-2**31, 2**31 - 1, (K // 8, N), generator=gen, dtype=torch.int32,
                      device="cuda")
    s = (torch.rand((K // G, N), generator=gen, device="cuda") * 0.01 + 1e-3).half()
    return p, s


def _capture(fn, warmup=2):
    """Warm up on a side stream (so every workspace exists), then capture."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(warmup):
            fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        outs = fn()
    torch.cuda.synchronize()
    return g, outs


@pytest.mark.parametrize("M", [1, 128])
def test_layer_gemms_graph_replay(M):
    import mmfp4
    gen = torch.Generator(device="cuda").manual_seed(11 + M)
    ws = [_words(gen, K, N) for K, N in LAYER]
    xs = {K: torch.empty((M, K), dtype=torch.float16, device="cuda") for K, _ in LAYER}

    def layer():
        return [mmfp4.marlin_gemm_fp4(xs[K], w[0], w[1], G) for (K, _), w in zip(LAYER, ws)]

    for x in xs.values():
        x.copy_(torch.randn(x.shape, generator=gen, device="cuda").half())
    announce(f"graph capture of the layer GEMMs M={M}")
    g, outs = _capture(layer)
    for rep in range(4):
        for x in xs.values():
            x.copy_(torch.randn(x.shape, generator=gen, device="cuda").half())
        torch.cuda.synchronize()
        ref = layer()                                   # eager, same inputs
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for (K, N), o, r in zip(LAYER, outs, ref):
            assert torch.equal(o.view(torch.int16), r.view(torch.int16)), (rep, K, N)
        # unrelated eager work on the same entry point between replays
        mmfp4.marlin_gemm_fp4(xs[4096][:1], ws[1][0], ws[1][1], G)


@pytest.mark.parametrize("T,E,k", [(32, 16, 4), (512, 16, 4), (1024, 16, 4)])
def test_moe_mlp_graph_replay(T, E, k):
    import mmfp4
    H, I = 512, 256
    gen = torch.Generator(device="cuda").manual_seed(T + E)
    gu = [_words(gen, H, 2 * I) for _ in range(E)]
    dn = [_words(gen, I, H) for _ in range(E)]
    gp, gs = torch.stack([w[0] for w in gu]), torch.stack([w[1] for w in gu])
    dp, ds = torch.stack([w[0] for w in dn]), torch.stack([w[1] for w in dn])
    x = torch.empty((T, H), dtype=torch.float16, device="cuda")
    ids = torch.empty((T, k), dtype=torch.int32, device="cuda")
    probs = torch.empty((T, k), dtype=torch.float32, device="cuda")

    def refill():
        x.copy_(torch.randn((T, H), generator=gen, device="cuda").half())
        logits = torch.randn((T, E), generator=gen, device="cuda")
        p, i = torch.topk(torch.softmax(logits, -1), k, -1)
        ids.copy_(i.to(torch.int32))
        probs.copy_(p / p.sum(-1, keepdim=True))

    def mlp():
        return mmfp4.moe_mlp_fp4(x, gp, gs, dp, ds, ids, probs, G)

    refill()
    announce(f"graph capture of the MoE MLP T={T} E={E} k={k}")
    g, out = _capture(mlp)
    for rep in range(4):
        refill()
        torch.cuda.synchronize()
        ref = mlp()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), rep


@pytest.mark.parametrize("M", [1, 24, 64])
def test_rowpacked_graph_replay(M):
    """Row-packed (MMFP4) words read in place: the GEMM (split-K at M=1 on
    14336 -> 4096, the two-row-block kernel at M=24, the pipelined kernel at
    M=64, both scale layouts) and the gate/up pair with its SwiGLU."""
    import mmfp4
    gen = torch.Generator(device="cuda").manual_seed(101 + M)
    shapes = [(14336, 4096), (4096, 6144)]
    rows, scl = [], []
    for K, N in shapes:
        rows.append(torch.randint(-2**31, 2**31 - 1, (N, K // 8), generator=gen,
                                  dtype=torch.int32, device="cuda"))
        scl.append((torch.rand((K // G, N), generator=gen, device="cuda") * 0.01 + 1e-3).half())
    gup = [torch.randint(-2**31, 2**31 - 1, (1536, 4096 // 8), generator=gen, dtype=torch.int32,
                         device="cuda") for _ in range(2)]
    gus = [(torch.rand((4096 // G, 1536), generator=gen, device="cuda") * 0.01 + 1e-3).half()
           for _ in range(2)]
    xs = {K: torch.empty((M, K), dtype=torch.float16, device="cuda") for K in (14336, 4096)}
    scl_t = [s.t().contiguous() for s in scl]

    def step():
        outs = [mmfp4.mmfp4_gemm_rowpacked(xs[K], r, s, G)
                for (K, _), r, s in zip(shapes, rows, scl)]
        if M <= 32:
            outs += [mmfp4.mmfp4_gemm_rowpacked(xs[K], r, s, G)
                     for (K, _), r, s in zip(shapes, rows, scl_t)]
        outs.append(mmfp4.mmfp4_fused_gate_up(xs[4096], gup[0], gus[0], gup[1], gus[1], G))
        return outs

    for x in xs.values():
        x.copy_(torch.randn(x.shape, generator=gen, device="cuda").half())
    announce(f"graph capture of the row-packed GEMMs M={M}")
    g, outs = _capture(step)
    for rep in range(4):
        for x in xs.values():
            x.copy_(torch.randn(x.shape, generator=gen, device="cuda").half())
        torch.cuda.synchronize()
        ref = step()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for i, (o, r) in enumerate(zip(outs, ref)):
            assert torch.equal(o.view(torch.int16), r.view(torch.int16)), (rep, i)
        mmfp4.mmfp4_gemm_rowpacked(xs[4096][:1], rows[1], scl[1], G)
