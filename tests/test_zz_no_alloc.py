"""mm_fp4_gemm_noalloc: the no-allocation variant of mm_fp4_gemm (workspace in
a built-in device array) against mm_fp4_gemm with a caller workspace, through
the C ABI: bit-identical outputs on two calls in a row, the second smaller,
for shapes that use the split-K hand-off (decode) and the split-K partials
(prefill); oversize workspace requests are refused."""

from __future__ import annotations

import ctypes

import pytest
import torch

from gpu_helpers import announce

pytestmark = pytest.mark.gpu

MAX_SCRATCH = 32 << 20


def _problem(M, K, N, g, seed):
    import mmfp4
    gen = torch.Generator(device="cuda").manual_seed(seed)
    w = (torch.randn((N, K), generator=gen, device="cuda") * 0.02).half()
    a = torch.randn((M, K), generator=gen, device="cuda").half()
    p, s = mmfp4.quantize_fp4(w, group_size=g)
    return a, p, s


def _with_workspace(lib, a, p, s, M, N, K, g):
    ws = torch.zeros(int(lib.mm_gemm_workspace_bytes(M, N, K)), dtype=torch.uint8, device="cuda")
    out = torch.empty((M, N), dtype=torch.float16, device="cuda")
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = lib.mm_fp4_gemm(a.data_ptr(), p.data_ptr(), s.data_ptr(), out.data_ptr(), M, N, K, g,
                         ws.data_ptr(), ws.numel(), st)
    assert rc == 0, lib.mm_last_error()
    return out


def _noalloc(lib, a, p, s, M, N, K, g):
    out = torch.full((M, N), float("nan"), dtype=torch.float16, device="cuda")
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = lib.mm_fp4_gemm_noalloc(a.data_ptr(), p.data_ptr(), s.data_ptr(), out.data_ptr(), M, N, K,
                                 g, st)
    assert rc == 0, lib.mm_last_error()
    return out


@pytest.mark.parametrize("first,second", [
    ((8, 14336, 4096), (1, 14336, 4096)),        # decode split-K (counters + partials)
    ((32, 4096, 28672), (3, 4096, 6144)),        # MT=2 skinny, then two-slab
    ((192, 4096, 4096), (100, 14336, 4096)),     # prefill split-K partials, then smaller M
    ((2048, 4096, 14336), (64, 1024, 512)),      # prefill (no split), then small
])
def test_noalloc_matches_workspace_entry(first, second):
    from mmfp4 import _lib
    lib = _lib.load()
    g = 128
    for i, (M, K, N) in enumerate((first, second)):
        assert lib.mm_gemm_workspace_bytes(M, N, K) <= MAX_SCRATCH
        a, p, s = _problem(M, K, N, g, seed=M + N + i)
        announce(f"noalloc call {i} M={M} K={K} N={N}")
        ref = _with_workspace(lib, a, p, s, M, N, K, g)
        out = _noalloc(lib, a, p, s, M, N, K, g)
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16))


def test_noalloc_refuses_oversize_workspace():
    from mmfp4 import _lib
    lib = _lib.load()
    M, N, K = 256, 4096, 4096                    # 32 MiB of split-K partials + counters
    need = lib.mm_gemm_workspace_bytes(M, N, K)
    assert need > MAX_SCRATCH
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = lib.mm_fp4_gemm_noalloc(0, 0, 0, 0, M, N, K, 128, st)
    assert rc == 1 and b"built-in scratch" in lib.mm_last_error()
