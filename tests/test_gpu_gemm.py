"""GPU parity of the fused FP4 / INT4 dequant-GEMM against the oracle's fp32
dequant+matmul (max-abs-rel <= 1e-2), plus the
size-independent properties at the BASELINE shapes."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from gpu_helpers import TOL, announce, max_abs_rel, to_dev, to_np
from oracle import fp4 as ofp4

pytestmark = pytest.mark.gpu


def _fp4_problem(rng, M, K, N, g):
    w = rng.normal(0, 0.02, (N, K)).astype(np.float16)
    packed, scales = ofp4.quantize_fp4(w, g)
    a = rng.normal(0, 1, (M, K)).astype(np.float16)
    return a, packed, scales


SMALL = [(1, 128, 128, 32), (2, 256, 192, 64), (5, 512, 256, 128), (16, 1024, 512, 128),
         (17, 256, 128, 32), (31, 1024, 1000, 8), (32, 4096, 256, 128), (33, 512, 384, 64),
         (64, 1024, 512, 128), (100, 768, 1024, 128), (128, 256, 256, 32),
         (129, 512, 260, 64), (256, 2048, 512, 128), (300, 384, 520, 128)]


@pytest.mark.parametrize("M,K,N,g", SMALL)
def test_fp4_gemm_vs_oracle(rng, M, K, N, g):
    import mmfp4
    a, packed, scales = _fp4_problem(rng, M, K, N, g)
    ref = ofp4.gemm_fp4_ref(a, packed, scales, g)
    announce(f"fp4 gemm M={M} K={K} N={N} g={g}")
    out = to_np(mmfp4.marlin_gemm_fp4(to_dev(a), to_dev(packed), to_dev(scales), g))
    assert out.shape == (M, N)
    assert max_abs_rel(out, ref) <= TOL


@pytest.mark.parametrize("M,K,N,g", [(1, 256, 128, 128), (16, 1024, 256, 128),
                                     (24, 512, 512, 64), (77, 512, 256, 128),
                                     (256, 1024, 512, 32)])
def test_u4_gemm_vs_oracle(rng, M, K, N, g):
    import mmfp4
    w = rng.normal(0, 0.02, (N, K)).astype(np.float16)
    packed, s, z = ofp4.pack_u4_weights(w, g)
    a = rng.normal(0, 1, (M, K)).astype(np.float16)
    ref = ofp4.gemm_u4_ref(a, packed, s, z, g)
    announce(f"u4 gemm M={M} K={K} N={N} g={g}")
    out = to_np(mmfp4.marlin_gemm_int4(to_dev(a), to_dev(packed), to_dev(s), to_dev(z), g))
    assert max_abs_rel(out, ref) <= TOL


def test_fp4_gemm_config1_vs_oracle(rng):
    """M=1, K=N=4096, g=128, against the CPU oracle."""
    import mmfp4
    a, packed, scales = _fp4_problem(rng, 1, 4096, 4096, 128)
    ref = ofp4.gemm_fp4_ref(a, packed, scales, 128)
    announce("fp4 gemm config1 M=1 4096x4096")
    out = to_np(mmfp4.marlin_gemm_fp4(to_dev(a), to_dev(packed), to_dev(scales), 128))
    assert max_abs_rel(out, ref) <= TOL


def _gpu_problem(M, K, N, g, seed=0):
    """Full-size problem built on the device by the (separately pinned) GPU
    quantizer; returns a, packed, scales and the unfused fp32 reference
    dequant(B) (bit-exact kernel) @ A in fp32."""
    import mmfp4
    gen = torch.Generator(device="cuda").manual_seed(seed)
    w = (torch.randn((N, K), generator=gen, device="cuda") * 0.02).half()
    a = torch.randn((M, K), generator=gen, device="cuda").half()
    packed, scales = mmfp4.quantize_fp4(w, group_size=g)
    wd = mmfp4.dequant_fp4(packed, scales, K, N, g).float()
    ref = a.float() @ wd
    return a, packed, scales, ref


LAYERS = [(4096, 6144), (4096, 4096), (4096, 28672), (14336, 4096)]


@pytest.mark.parametrize("M", [1, 8, 32])
@pytest.mark.parametrize("K,N", LAYERS)
def test_fp4_decode_llama_layers(M, K, N):
    import mmfp4
    a, packed, scales, ref = _gpu_problem(M, K, N, 128)
    announce(f"fp4 decode M={M} K={K} N={N}")
    out = mmfp4.marlin_gemm_fp4(a, packed, scales, 128)
    assert max_abs_rel(to_np(out), to_np(ref)) <= TOL


@pytest.mark.parametrize("M", [512, 2048, 8192])
@pytest.mark.parametrize("K,N", [(4096, 14336), (14336, 4096)])
def test_fp4_prefill_config4(M, K, N):
    import mmfp4
    a, packed, scales, ref = _gpu_problem(M, K, N, 128)
    announce(f"fp4 prefill M={M} K={K} N={N}")
    out = mmfp4.marlin_gemm_fp4(a, packed, scales, 128)
    assert max_abs_rel(to_np(out), to_np(ref)) <= TOL


@pytest.mark.parametrize("M", [1, 16])
@pytest.mark.parametrize("K,N", LAYERS)
def test_u4_llama_layers(M, K, N):
    import mmfp4
    gen = torch.Generator(device="cuda").manual_seed(3)
    w = (torch.randn((N, K), generator=gen, device="cuda") * 0.02).half()
    a = torch.randn((M, K), generator=gen, device="cuda").half()
    packed, s, z = mmfp4.pack_u4_weights(w, group_size=128)
    ref = a.float() @ mmfp4.dequant_int4(packed, s, z, K, N, 128).float()
    announce(f"u4 layer M={M} K={K} N={N}")
    out = mmfp4.marlin_gemm_int4(a, packed, s, z, 128)
    assert max_abs_rel(to_np(out), to_np(ref)) <= TOL


@pytest.mark.parametrize("M", [1, 16, 64])
def test_u4_outlier_activations(rng, M):
    """INT4 with LLM-like activations: a few channels at +-100 .. +-1000 over an
    N(0, 1) body.  The decode kernels sum a * (1024 + q) and subtract
    (1024 + z) * sum(a) per group, a cancellation whose rounding grows with
    1024 * sum|a|; the prefill kernel uses the dequantized weights.  Against
    the oracle's fp32 (q - z) * s matmul."""
    import mmfp4
    K, N, g = 4096, 1024, 128
    w = rng.normal(0, 0.02, (N, K)).astype(np.float16)
    packed, s, z = ofp4.pack_u4_weights(w, g)
    a = rng.normal(0, 1, (M, K)).astype(np.float32)
    chans = rng.choice(K, 24, replace=False)
    a[:, chans] = rng.choice([-1000.0, -300.0, -100.0, 100.0, 250.0, 1000.0], (M, 24))
    a = a.astype(np.float16)
    ref = ofp4.gemm_u4_ref(a, packed, s, z, g)
    announce(f"u4 outliers M={M}")
    out = to_np(mmfp4.marlin_gemm_int4(to_dev(a), to_dev(packed), to_dev(s), to_dev(z), g))
    assert max_abs_rel(out, ref) <= TOL
    # the body columns alone (outlier contributions removed) are still matched
    a2 = a.copy()
    a2[:, chans] = 0
    body = ofp4.gemm_u4_ref(a2, packed, s, z, g)
    out2 = to_np(mmfp4.marlin_gemm_int4(to_dev(a2), to_dev(packed), to_dev(s), to_dev(z), g))
    assert max_abs_rel(out2, body) <= TOL


@pytest.mark.parametrize("M", [1, 20, 64])
def test_zero_input_and_determinism(M):
    import mmfp4
    a, packed, scales, _ = _gpu_problem(M, 14336, 4096, 128, seed=5)
    announce(f"zero/determinism M={M}")
    z = mmfp4.marlin_gemm_fp4(torch.zeros_like(a), packed, scales, 128)
    assert torch.count_nonzero(z).item() == 0
    o1 = mmfp4.marlin_gemm_fp4(a, packed, scales, 128)
    o2 = mmfp4.marlin_gemm_fp4(a, packed, scales, 128)
    assert torch.equal(o1.view(torch.int16), o2.view(torch.int16))


@pytest.mark.parametrize("M", [1, 48])
def test_linearity(M):
    import mmfp4
    a, packed, scales, _ = _gpu_problem(M, 4096, 1024, 128, seed=6)
    b = torch.randn_like(a.float()).half()
    announce(f"linearity M={M}")
    lhs = mmfp4.marlin_gemm_fp4((a.float() + b.float()).half(), packed, scales, 128).float()
    rhs = (mmfp4.marlin_gemm_fp4(a, packed, scales, 128).float()
           + mmfp4.marlin_gemm_fp4(b, packed, scales, 128).float())
    assert max_abs_rel(to_np(lhs), to_np(rhs)) <= TOL


@pytest.mark.parametrize("M", [1, 32, 100])
def test_large_k_all_ones(M):
    """tests/test_gemm.py:531-556: K = 32768 ones against weights 1.0 * 0.5."""
    import mmfp4
    K, N = 32768, 256
    packed = torch.full((K // 8, N), 0x22222222, dtype=torch.int32, device="cuda")
    scales = torch.full((K // 128, N), 0.5, dtype=torch.float16, device="cuda")
    announce(f"all-ones K=32768 M={M}")
    out = mmfp4.marlin_gemm_fp4(torch.ones((M, K), dtype=torch.float16, device="cuda"), packed,
                                scales, 128)
    assert torch.all(out == 16384.0).item()


def test_split_k_workspace_reuse_across_shapes():
    """Counters left at zero: interleaved shapes reproduce their first result."""
    import mmfp4
    probs = [_gpu_problem(M, K, N, 128, seed=M + K) for M, K, N in
             [(1, 14336, 4096), (8, 4096, 6144), (32, 14336, 512), (3, 4096, 128),
              (32, 4096, 28672), (16, 14336, 4096)]]
    announce("workspace reuse")
    first = [mmfp4.marlin_gemm_fp4(a, p, s, 128) for a, p, s, _ in probs]
    for _ in range(3):
        for (a, p, s, _), f in zip(probs, first):
            assert torch.equal(mmfp4.marlin_gemm_fp4(a, p, s, 128).view(torch.int16),
                               f.view(torch.int16))


@pytest.mark.parametrize("M,K", [(1, 4096), (8, 14336), (32, 4096)])
def test_split_k_large_and_nonfinite_partials(M, K):
    """Split-K partials outside the fixed-point range (|p| >= 2^15), that
    cancel across splits, and inf / NaN inputs: same finite values (to the
    tolerance), same NaN and same signed-inf positions as the fp32 reference."""
    import mmfp4
    N, g = 256, 128
    gen = torch.Generator(device="cuda").manual_seed(9)
    packed = torch.randint(-2**31, 2**31 - 1, (K // 8, N), generator=gen, dtype=torch.int32,
                           device="cuda")
    scales = (torch.rand((K // g, N), generator=gen, device="cuda") + 0.5).half()
    a = torch.randn((M, K), generator=gen, device="cuda").half()
    a[0, 5] = 30000.0            # first split: |partial| >> 2^15 ...
    a[0, K - 7] = -30000.0       # ... cancelled by the last split
    if M > 1:
        a[1, 100] = float("inf")
        a[1, K - 100] = float("-inf")
        a[M - 1, K // 2] = float("nan")
    ref = (a.float() @ mmfp4.dequant_fp4(packed, scales, K, N, g).float()).half().float()
    announce(f"split-K big/non-finite partials M={M} K={K}")
    out = mmfp4.marlin_gemm_fp4(a, packed, scales, g).float()
    assert torch.equal(torch.isnan(out), torch.isnan(ref))
    assert torch.equal(torch.isposinf(out), torch.isposinf(ref))
    assert torch.equal(torch.isneginf(out), torch.isneginf(ref))
    fin = torch.isfinite(ref)
    err = (out[fin] - ref[fin]).abs().max().item()
    assert err <= TOL * ref[fin].abs().max().item()


def test_stream_read_measurement_aid():
    """mm_stream_read (bench.py's read-ceiling aid, libmmfp4_bench.so) reads
    and writes nothing in every order and load form; bad arguments are
    refused."""
    import bench_aids
    buf = torch.arange(1 << 18, dtype=torch.int32, device="cuda")
    sink = torch.zeros(8192 * 512, dtype=torch.int32, device="cuda")
    st = torch.cuda.current_stream().cuda_stream
    for blocks, threads, unroll, mode in ((0, 0, 4, 1), (64, 256, 1, 0), (300, 1024, 16, 3),
                                          (1000, 64, 8, 2)):
        announce(f"stream read blocks={blocks} threads={threads} unroll={unroll} mode={mode}")
        bench_aids.call("mm_stream_read", buf.data_ptr(), buf.numel() * 4, sink.data_ptr(),
                        sink.numel() * 4, blocks, threads, unroll, mode, st)
    torch.cuda.synchronize()
    assert int(sink.abs().sum()) == 0
    for bad in ((1000, 0, 0, 4, 1), (4096, 64, 100, 4, 1), (4096, 64, 256, 3, 1),
                (4096, 64, 256, 4, 4), (4096, 1 << 20, 1024, 4, 0)):
        with pytest.raises(ValueError):
            bench_aids.call("mm_stream_read", buf.data_ptr(), bad[0], sink.data_ptr(),
                            sink.numel() * 4, *bad[1:], st)


def test_mfma_ceiling_measurement_aid():
    """mm_mfma_ceiling's sums: with all-ones operands every accumulator gains
    16 per MFMA and 4 MFMAs per iteration, and a lane's 8 accumulators add to
    512 * iters; bad arguments are refused."""
    import bench_aids
    ones = torch.ones(4096, dtype=torch.float16, device="cuda")
    sink = torch.zeros(256 * 512, dtype=torch.float32, device="cuda")
    st = torch.cuda.current_stream().cuda_stream
    announce("mfma ceiling iters=3")
    bench_aids.call("mm_mfma_ceiling", ones.data_ptr(), ones.data_ptr(), ones.numel(), 3,
                    sink.data_ptr(), sink.numel() * 4, st)
    torch.cuda.synchronize()
    assert torch.all(sink == 512 * 3)
    with pytest.raises(ValueError):
        bench_aids.call("mm_mfma_ceiling", ones.data_ptr(), ones.data_ptr(), 12, 3,
                        sink.data_ptr(), sink.numel() * 4, st)
    with pytest.raises(ValueError):
        bench_aids.call("mm_mfma_ceiling", ones.data_ptr(), ones.data_ptr(), 4096, 3,
                        sink.data_ptr(), 1024, st)


@pytest.mark.parametrize("M,K,N,g,int4", [(1, 512, 3072, 128, False), (8, 4160, 3076, 64, False),
                                          (3, 1024, 4096, 256, False), (5, 576, 6144, 64, False),
                                          (1, 1024, 3072, 128, True), (7, 640, 4100, 64, True),
                                          (1, 4096, 4096, 128, False), (2, 4096, 6144, 128, True)])
def test_two_slab_decode_vs_oracle(rng, M, K, N, g, int4):
    """The two-slab decode kernel (M <= 8, 32-column blocks, each MFMA step 64 k
    split over operand rows 0-7 / 8-15): ragged last tile (N % 32 != 0), a
    partial last round (K = 65 x 64), group sizes 64..256, FP4 and INT4."""
    import mmfp4
    w = rng.normal(0, 0.02, (N, K)).astype(np.float16)
    a = rng.normal(0, 1, (M, K)).astype(np.float16)
    announce(f"two-slab decode M={M} K={K} N={N} g={g} int4={int4}")
    if int4:
        packed, s, z = ofp4.pack_u4_weights(w, g)
        ref = ofp4.gemm_u4_ref(a, packed, s, z, g)
        out = to_np(mmfp4.marlin_gemm_int4(to_dev(a), to_dev(packed), to_dev(s), to_dev(z), g))
    else:
        packed, scales = ofp4.quantize_fp4(w, g)
        ref = ofp4.gemm_fp4_ref(a, packed, scales, g)
        out = to_np(mmfp4.marlin_gemm_fp4(to_dev(a), to_dev(packed), to_dev(scales), g))
    assert out.shape == (M, N)
    assert max_abs_rel(out, ref) <= TOL


@pytest.mark.parametrize("M,K,N", [(1, 4096, 4096), (37, 512, 256)])
def test_binding_and_ctypes_paths_agree(M, K, N):
    """marlin_gemm_fp4 / marlin_gemm_int4 through the per-call C++ binding and
    through the ctypes path: the same C entry points, bit-identical outputs;
    errors raise the same exception types."""
    import mmfp4
    from mmfp4 import kernels
    assert kernels._binding(), "the per-call binding (_mmfp4_torch.so) is not built"
    a, packed, scales, _ = _gpu_problem(M, K, N, 128, seed=4)
    z = torch.full_like(scales, 8.0)
    announce(f"binding vs ctypes M={M}")
    fast = mmfp4.marlin_gemm_fp4(a, packed, scales, 128)
    fast4 = mmfp4.marlin_gemm_int4(a, packed, scales, z, 128)
    slow = kernels._gemm_ctypes("fp4", a, packed, scales, None, 128)
    slow4 = kernels._gemm_ctypes("u4", a, packed, scales, z, 128)
    assert torch.equal(fast.view(torch.int16), slow.view(torch.int16))
    assert torch.equal(fast4.view(torch.int16), slow4.view(torch.int16))
    a3 = a.reshape(1, M, K)
    assert mmfp4.marlin_gemm_fp4(a3, packed, scales, 128).shape == (1, M, N)
    for fn in (lambda *x: mmfp4.marlin_gemm_fp4(*x), lambda *x: kernels._gemm_ctypes("fp4", *x[:3], None, x[3])):
        with pytest.raises(ValueError, match="Packed K"):
            fn(a[:, :K - 8].contiguous(), packed, scales, 128)
        with pytest.raises(ValueError):
            fn(a, packed, scales, 64)
        with pytest.raises(RuntimeError, match="GPU only"):
            fn(a.cpu(), packed, scales, 128)


def test_odd_width_padding_is_cached_on_the_operands(rng):
    """N % 4 != 0: the padded copies are built once per operand tensor and
    rebuilt after an in-place write (the version counter moves)."""
    import mmfp4
    K, N, g = 512, 1002, 128
    w = rng.normal(0, 0.02, (N, K)).astype(np.float16)
    packed, scales = ofp4.quantize_fp4(w, g)
    a = rng.normal(0, 1, (3, K)).astype(np.float16)
    dp, ds, da = to_dev(packed), to_dev(scales), to_dev(a)
    announce("odd width padding cache")
    out1 = mmfp4.marlin_gemm_fp4(da, dp, ds, g)
    cached = dp._mmfp4_derived["pad4"][1]
    out2 = mmfp4.marlin_gemm_fp4(da, dp, ds, g)
    assert dp._mmfp4_derived["pad4"][1] is cached
    assert torch.equal(out1, out2)
    assert max_abs_rel(to_np(out1), ofp4.gemm_fp4_ref(a, packed, scales, g)) <= TOL
    ds.mul_(2)                                   # in-place write: rebuilt, result doubles
    out3 = mmfp4.marlin_gemm_fp4(da, dp, ds, g)
    assert torch.equal(out3, (out1.float() * 2).half())


def test_workspace_shared_between_call_paths_and_released():
    from mmfp4 import _lib
    import mmfp4
    dev = torch.device("cuda", torch.cuda.current_device())
    st = _lib.raw_stream(dev.index)
    w1 = _lib.workspace_on(dev.index, st, 4096)
    assert _lib.workspace(dev, 4096).data_ptr() == w1.data_ptr()
    b = _lib.binding()
    if b:
        assert b.workspace(dev.index, st, 4096).data_ptr() == w1.data_ptr()
    mmfp4.release_workspaces()
    torch.cuda.synchronize()
    w2 = _lib.workspace_on(dev.index, st, 4096)
    assert int(w2[:65536].count_nonzero()) == 0       # fresh, zeroed counters


@pytest.mark.parametrize("M,K,N,g", [(1, 4096, 6144, 128), (4, 4096, 4096, 64), (12, 4096, 4096, 128),
                                     (16, 4096, 28672, 128), (1, 14336, 4096, 128),
                                     (24, 2048, 3072, 32), (32, 4096, 1024, 256), (9, 1024, 2048, 8)])
def test_u4_interleaved_scales_zeros_bit_identical(rng, M, K, N, g):
    """mm_u4_gemm_sz (scales and zero points interleaved for the decode
    kernels) gives mm_u4_gemm's bits on every decode kernel family (two-slab,
    strip, 64- and 128-column skinny, split-K, pre-scale g=8), through the C
    ABI; marlin_gemm_int4 caches the interleaved copy on the scales tensor and
    rebuilds it when the zeros change."""
    import mmfp4
    from mmfp4 import _lib, kernels
    q, s, z = ofp4.pack_u4_weights(rng.normal(0, 0.02, (N, K)).astype(np.float16), g)
    a = to_dev(rng.normal(0, 1, (M, K)).astype(np.float16))
    dq, ds, dz = to_dev(q), to_dev(s), to_dev(z)
    sz = kernels._interleave_sz(ds, dz)
    ws = _lib.workspace(a.device, int(_lib.load().mm_gemm_workspace_bytes(M, N, K)))
    outs = []
    for name, extra in (("mm_u4_gemm", ()), ("mm_u4_gemm_sz", (_lib.ptr(sz),))):
        out = torch.empty((M, N), dtype=torch.float16, device=a.device)
        announce(f"{name} M={M} K={K} N={N} g={g}")
        _lib.call(name, _lib.ptr(a), _lib.ptr(dq), _lib.ptr(ds), _lib.ptr(dz), *extra,
                  _lib.ptr(out), M, N, K, g, _lib.ptr(ws), ws.numel(), _lib.stream_of(a))
        outs.append(out)
    assert torch.equal(outs[0], outs[1])
    assert torch.equal(mmfp4.marlin_gemm_int4(a, dq, ds, dz, g), outs[0])
    cached = ds._mmfp4_derived["sz"][1]
    dz.add_(1)                                   # new zero points: the copy is rebuilt
    out2 = mmfp4.marlin_gemm_int4(a, dq, ds, dz, g)
    assert ds._mmfp4_derived["sz"][1] is not cached
    ref = ofp4.gemm_u4_ref(to_np(a), q, s, z + 1, g)
    assert max_abs_rel(to_np(out2), ref) <= TOL
