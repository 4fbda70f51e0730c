"""Drop-in FP4 / INT4 dequant-GEMM entry points (the reference's
`metal_marlin.kernels` GEMM surface), backed by libmmfp4.so on gfx950.

Same names, argument meaning and errors as metal_marlin/kernels_core.py;
outputs are fp16 like the reference.  Calls are asynchronous on the current
torch stream (the reference blocks on `waitUntilCompleted`); there is no CPU
fallback: host tensors raise.
"""

from __future__ import annotations

import functools

import torch

from . import _lib

__all__ = [
    "marlin_gemm_fp4", "marlin_gemm_fp4_tuned", "marlin_gemm_fused_fp4",
    "marlin_gemm_int4", "marlin_gemm_fused_u4", "dequant_fp4", "dequant_int4",
    "dequant_fp4_decode_gemv", "decode_gemv_fp4", "mmfp4_gemm", "dequantize_mmfp4",
    "select_decode_kernel", "fused_gate_up_gemm", "mmfp4_fused_gate_up",
    "mmfp4_gemm_rowpacked", "rowpacked_gemm_supported",
    "mmfp4_fused_gate_up_marlin", "mmfp4_fused_qkv", "FP4_PER_UINT",
]

FP4_PER_UINT = 8


def _packed(t: torch.Tensor) -> torch.Tensor:
    if t.dtype not in (torch.int32, torch.uint32):
        raise TypeError(f"packed weights must be int32/uint32 words, got {t.dtype}")
    return t.contiguous()


def _half(t: torch.Tensor) -> torch.Tensor:
    return (t if t.dtype == torch.float16 else t.to(torch.float16)).contiguous()


def _check_groups(name: str, scales: torch.Tensor, K: int, N: int, group_size: int) -> None:
    if group_size <= 0 or K % group_size != 0:
        raise ValueError(f"{name}: K={K} must be divisible by group_size={group_size}")
    if tuple(scales.shape) != (K // group_size, N):
        raise ValueError(f"{name}: {name} shape {tuple(scales.shape)} != "
                         f"({K // group_size}, {N}) for K={K}, group_size={group_size}")


@functools.lru_cache(maxsize=4096)
def _ws_bytes(M: int, N: int, K: int) -> int:
    return int(_lib.load().mm_gemm_workspace_bytes(M, N, K))


def _gemm(kind: str, A: torch.Tensor, B_packed: torch.Tensor, scales: torch.Tensor,
          zeros: torch.Tensor | None, group_size: int) -> torch.Tensor:
    N = B_packed.shape[-1] if B_packed.dim() == 2 else 0
    if N % 4 != 0 and scales.dim() == 2 and scales.shape[-1] == N and \
            (zeros is None or (zeros.dim() == 2 and zeros.shape[-1] == N)):
        # The kernels store 4 adjacent columns per lane.  Other widths (an
        # lm_head over 32001 tokens, say) run on copies padded to a multiple
        # of 4 -- zero words, unit scales, zero points 0, so the extra columns
        # are exact zeros -- and return the first N columns.
        # The padded copies are cached on the operand tensors themselves
        # (rebuilt when a tensor is written in place or its storage changes),
        # so repeated calls with the same weights pay the copy once.
        pad = (0, -N % 4)
        F = torch.nn.functional
        zp = None if zeros is None else _lib.derived(zeros, "pad4", lambda t: F.pad(t, pad))
        words = _lib.derived(
            B_packed, "pad4",
            lambda t: F.pad(t.view(torch.int32) if t.dtype == torch.uint32 else t, pad))
        sp = _lib.derived(scales, "pad4", lambda t: F.pad(t, pad, value=1.0))
        out = _gemm(kind, A, words, sp, zp, group_size)
        return out[..., :N].contiguous()
    sz = None
    if kind == "u4" and A.shape[-1] and A.numel() // A.shape[-1] <= 32 and _sz_ok(scales, zeros):
        # decode sizes: scales and zero points interleaved once per (scales,
        # zeros) pair, so the kernels load one 16-byte piece per group
        sz = _lib.derived(scales, "sz", lambda t: _interleave_sz(t, zeros), also=zeros)
    fast = _BINDING if _BINDING is not None else _binding()
    if fast:
        # checks, output allocation and workspace in C++ (_mmfp4_torch.so)
        idx = A.get_device()
        try:
            return fast.gemm(A, B_packed, scales, zeros if kind == "u4" else None, sz, group_size,
                             _lib.raw_stream(idx) if idx >= 0 else 0)
        except RuntimeError as e:
            if type(e) is RuntimeError and "GPU only" not in str(e):
                raise _lib.MMError(str(e)) from None
            raise
    return _gemm_ctypes(kind, A, B_packed, scales, zeros, group_size, sz)


def _sz_ok(scales: torch.Tensor, zeros: torch.Tensor | None) -> bool:
    return (zeros is not None and scales.dim() == 2 and zeros.shape == scales.shape
            and scales.shape[-1] % 4 == 0 and scales.is_cuda and zeros.device == scales.device)


def _interleave_sz(scales: torch.Tensor, zeros: torch.Tensor) -> torch.Tensor:
    """[K/g, 2N] fp16: for each 4-column group its 4 scales then its 4 zero
    points (the interleaved operand of mm_u4_gemm_sz)."""
    R, N = scales.shape
    s4 = scales.to(torch.float16).reshape(R, N // 4, 4)
    z4 = zeros.to(torch.float16).reshape(R, N // 4, 4)
    return torch.stack((s4, z4), dim=2).reshape(R, 2 * N).contiguous()


_BINDING = None


def _binding():
    global _BINDING
    _BINDING = _lib.binding() or False
    return _BINDING


def _gemm_ctypes(kind: str, A: torch.Tensor, B_packed: torch.Tensor, scales: torch.Tensor,
                 zeros: torch.Tensor | None, group_size: int,
                 sz: torch.Tensor | None = None) -> torch.Tensor:
    # The per-call host path is kept short: one device check, the current
    # stream as a raw handle, a cached workspace, no copies of operands that
    # already have the right dtype and layout.
    idx = _lib.same_device_index(A, B_packed, scales, zeros)
    K = A.shape[-1]
    M = A.numel() // K if K else 0
    K_packed, N = B_packed.shape
    if K_packed * FP4_PER_UINT != K:
        raise ValueError(f"Packed K {K_packed * FP4_PER_UINT} does not match activations K {K}")
    if group_size <= 0 or K % group_size != 0 or scales.shape[0] * group_size != K \
            or scales.shape[1] != N:
        _check_groups("scales", scales, K, N, group_size)
    if zeros is not None:
        _check_groups("zeros", zeros, K, N, group_size)
    a = A if A.dtype == torch.float16 and A.is_contiguous() else _half(A)
    a = a.view(M, K)
    b = B_packed if B_packed.is_contiguous() else B_packed.contiguous()
    if b.dtype not in (torch.int32, torch.uint32):
        raise TypeError(f"packed weights must be int32/uint32 words, got {b.dtype}")
    s = scales if scales.dtype == torch.float16 and scales.is_contiguous() else _half(scales)
    out = torch.empty((M, N), dtype=torch.float16, device=a.device)
    st = _lib.raw_stream(idx)
    ws = _lib.workspace_on(idx, st, _ws_bytes(M, N, K))
    if _lib._lib is None:
        _lib.load()
    if kind == "fp4":
        rc = _lib.F.mm_fp4_gemm(a.data_ptr(), b.data_ptr(), s.data_ptr(), out.data_ptr(), M, N,
                                K, group_size, ws.data_ptr(), ws.numel(), st)
    elif sz is not None:
        z = _half(zeros)
        rc = _lib.F.mm_u4_gemm_sz(a.data_ptr(), b.data_ptr(), s.data_ptr(), z.data_ptr(),
                                  sz.data_ptr(), out.data_ptr(), M, N, K, group_size,
                                  ws.data_ptr(), ws.numel(), st)
    else:
        z = _half(zeros)
        rc = _lib.F.mm_u4_gemm(a.data_ptr(), b.data_ptr(), s.data_ptr(), z.data_ptr(),
                               out.data_ptr(), M, N, K, group_size, ws.data_ptr(), ws.numel(), st)
    if rc:
        _lib.check(rc)
    return out.view(*A.shape[:-1], N)


def marlin_gemm_fp4(A: torch.Tensor, B_packed: torch.Tensor, scales: torch.Tensor,
                    group_size: int = 32) -> torch.Tensor:
    """C = A @ dequant(B_packed, scales) -- kernels_core.py:1830-1937.

    A [*, K] (any float dtype, computed as fp16), B_packed [K/8, N] int32/uint32
    Marlin layout, scales [K/group_size, N].  Returns fp16 [*, N].  M <= 32 runs
    the decode kernel, larger M the MFMA prefill kernel (metal_dispatch.py:
    4083-4098 chooses by M the same way).
    """
    return _gemm("fp4", A, B_packed, scales, None, group_size)


def rowpacked_gemm_supported(M: int, N: int, K: int, group_size: int) -> bool:
    """Shapes mm_fp4_gemm_rowpacked takes (row-packed words read in place)."""
    return (M > 0 and group_size > 0 and group_size % (32 if M <= 32 else 64) == 0
            and K % group_size == 0 and N % (4 if M <= 32 else 8) == 0)


def _scales_layout(scales: torch.Tensor, N: int, n_groups: int, name: str = "scales") -> int:
    """0 for [n_groups, N] (the reference's canonical layout, read first when
    the tensor is square), 1 for [N, n_groups]; the same shape test as
    layers/mmfp4_linear.py:53-86 (_optimized_scale_load)."""
    shape = tuple(scales.shape)
    if shape == (n_groups, N):
        return 0
    if shape == (N, n_groups):
        return 1
    raise ValueError(f"{name} shape {shape} is neither ({n_groups}, {N}) nor ({N}, {n_groups})")


def mmfp4_gemm_rowpacked(A: torch.Tensor, B_rows: torch.Tensor, scales: torch.Tensor,
                         group_size: int = 128) -> torch.Tensor:
    """A [M, K] @ dequant(B_rows)^T with row-packed weights read in place:
    B_rows [N, K/8] words, scales [K/group_size, N] (the layer's canonical
    layout) or [N, K/group_size] (layers/mmfp4_linear.py:549-598).  M <= 32
    runs the decode kernels; larger M the pipelined prefill kernel, which
    reads the words in place too but takes [K/group_size, N] scales (the
    other layout is transposed here, K/group_size x N halves)."""
    dev = _lib.require_device(A, B_rows, scales)
    M, K = A.shape
    N, K_packed = B_rows.shape
    if K_packed * FP4_PER_UINT != K:
        raise ValueError(f"Packed K {K_packed * FP4_PER_UINT} does not match activations K {K}")
    if group_size <= 0 or K % group_size != 0:
        raise ValueError(f"K={K} must be divisible by group_size={group_size}")
    layout = _scales_layout(scales, N, K // group_size)
    a = _half(A)
    b = _packed(B_rows)
    s = _half(scales)
    if M > 32 and layout == 1:
        s, layout = s.t().contiguous(), 0
    out = torch.empty((M, N), dtype=torch.float16, device=dev)
    ws = _lib.workspace(dev, int(_lib.load().mm_gemm_workspace_bytes(M, N, K)))
    _lib.call("mm_fp4_gemm_rowpacked", _lib.ptr(a), _lib.ptr(b), _lib.ptr(s), _lib.ptr(out), M, N,
              K, group_size, layout, _lib.ptr(ws), ws.numel(), _lib.stream_of(a))
    return out


def marlin_gemm_fp4_tuned(A, B_packed, scales, group_size: int = 32):
    """Alias of marlin_gemm_fp4 (kernels_core.py:1939-1947)."""
    return marlin_gemm_fp4(A, B_packed, scales, group_size)


def marlin_gemm_fused_fp4(A, B_packed, scales, group_size: int = 32):
    """Alias of marlin_gemm_fp4 (kernels_core.py:1949-1957)."""
    return marlin_gemm_fp4(A, B_packed, scales, group_size)


def marlin_gemm_int4(A: torch.Tensor, B_packed: torch.Tensor, scales: torch.Tensor,
                     zeros: torch.Tensor, group_size: int = 32) -> torch.Tensor:
    """C = A @ ((q - zeros) * scales) -- kernels_core.py:1959-2066."""
    return _gemm("u4", A, B_packed, scales, zeros, group_size)


def marlin_gemm_fused_u4(A, B_packed, scales, zeros, group_size: int = 32):
    """Alias of marlin_gemm_int4 (kernels_core.py:2068-2077)."""
    return marlin_gemm_int4(A, B_packed, scales, zeros, group_size)


def _gate_up(x: torch.Tensor, gate_packed: torch.Tensor, gate_scales: torch.Tensor,
             up_packed: torch.Tensor, up_scales: torch.Tensor, group_size: int,
             act: int) -> torch.Tensor:
    """One launch over the gate and up matrices, both Marlin [K/8, N]:
    act=1 -> silu(x @ Wg) * (x @ Wu) [M, N]; act=0 -> [x @ Wg | x @ Wu] [M, 2N]."""
    dev = _lib.require_device(x, gate_packed, gate_scales, up_packed, up_scales)
    if x.dim() != 2:
        raise ValueError(f"x must be 2D [M, K], got shape={tuple(x.shape)}")
    M, K = x.shape
    K_packed, N = gate_packed.shape
    if tuple(up_packed.shape) != (K_packed, N):
        raise ValueError("up_packed must match gate_packed shape "
                         f"({K_packed}, {N}), got {tuple(up_packed.shape)}")
    if K != K_packed * FP4_PER_UINT:
        raise ValueError(f"K mismatch: x has K={K}, but packed tensors imply "
                         f"K={K_packed * FP4_PER_UINT}")
    _check_groups("gate_scales", gate_scales, K, N, group_size)
    _check_groups("up_scales", up_scales, K, N, group_size)
    if N % 8 != 0 or (M > 32 and K % 64 != 0):
        # The one-launch pair kernels take N % 8 == 0, and above 32 rows
        # stream 64-k chunks; other shapes take two GEMM launches (any N, and
        # the tile kernel for K % 64 tails), and SiLU then sees the fp16
        # products, as in the reference's kernel.
        g = marlin_gemm_fp4(x, gate_packed, gate_scales, group_size)
        u = marlin_gemm_fp4(x, up_packed, up_scales, group_size)
        if not act:
            return torch.cat([g, u], dim=1)
        return (torch.nn.functional.silu(g.float()) * u.float()).half()
    a = _half(x)
    out = torch.empty((M, N if act else 2 * N), dtype=torch.float16, device=dev)
    ws_bytes = int(_lib.load().mm_gemm_workspace_bytes(M, 2 * N, K))
    ws = _lib.workspace(dev, ws_bytes)
    gp, up = _packed(gate_packed), _packed(up_packed)
    gs, us = _half(gate_scales), _half(up_scales)
    _lib.call("mm_fp4_gate_up", _lib.ptr(a), _lib.ptr(gp), _lib.ptr(gs), _lib.ptr(up),
              _lib.ptr(us), _lib.ptr(out), M, N, K, group_size, act, _lib.ptr(ws), ws.numel(),
              _lib.stream_of(a))
    return out


def fused_gate_up_gemm(x: torch.Tensor, gate_packed: torch.Tensor, gate_scales: torch.Tensor,
                       up_packed: torch.Tensor, up_scales: torch.Tensor,
                       group_size: int = 128) -> torch.Tensor:
    """Gate and up projections in one launch (kernels_core.py:4749-4760 ->
    MetalKernels.fused_gate_up_gemm :4220-4267): packed [K/8, N] Marlin
    layout, scales [K/group_size, N]; returns [M, 2N] fp16 with the gate
    product in columns [0, N) and the up product in [N, 2N)."""
    return _gate_up(x, gate_packed, gate_scales, up_packed, up_scales, group_size, 0)


def mmfp4_fused_gate_up(x: torch.Tensor, gate_packed: torch.Tensor, gate_scales: torch.Tensor,
                        up_packed: torch.Tensor, up_scales: torch.Tensor,
                        group_size: int = 128) -> torch.Tensor:
    """silu(gate_proj(x)) * up_proj(x) (kernels_core.py:4762-4774 ->
    MetalKernels.mmfp4_fused_gate_up :4269-4408).  Layout as documented there:
    gate_packed / up_packed row-packed [N, K/8] uint32, scales [K/group_size, N].
    With N % 8 == 0 and a group size that is a multiple of 32 (up to 32 rows)
    or of 64 (above) the row-packed words are read in place at every M
    (mm_fp4_gate_up_rowpacked: the decode kernel up to 32 rows, the
    pipelined prefill kernel above); other shapes
    are transposed to the Marlin layout on the device for each call (as the
    reference's own M < 64 path does); callers that keep the Marlin layout
    call `mmfp4_fused_gate_up_marlin`.
    Rounding of the SiLU input depends on the path: the one-launch pair
    kernels (N % 8 == 0, and K % 64 == 0 above 32 rows) apply SiLU to the
    fp32 sums; the two-launch fallback for other shapes applies it to the
    fp16-rounded products, which is the reference's own rounding."""
    if x.dim() != 2:
        raise ValueError(f"x must be 2D [M, K], got shape={tuple(x.shape)}")
    M, K = x.shape
    N, K_packed = gate_packed.shape
    if tuple(up_packed.shape) != (N, K_packed):
        raise ValueError("up_packed must match gate_packed shape "
                         f"({N}, {K_packed}), got {tuple(up_packed.shape)}")
    if K != K_packed * FP4_PER_UINT:
        raise ValueError(f"K mismatch: x has K={K}, but packed tensors imply "
                         f"K={K_packed * FP4_PER_UINT}")
    if K % group_size != 0:
        raise ValueError(f"K ({K}) must be divisible by group_size ({group_size})")
    expected = (K // group_size, N)
    for name, sc in (("gate_scales", gate_scales), ("up_scales", up_scales)):
        if tuple(sc.shape) != expected:
            raise ValueError(f"{name} shape mismatch: expected {expected}, got {tuple(sc.shape)}")
    M = x.shape[0]
    if rowpacked_gemm_supported(M, N, K, group_size) and N % 8 == 0:
        # the row-packed words are read in place, no transpose
        dev = _lib.require_device(x, gate_packed, gate_scales, up_packed, up_scales)
        a = _half(x)
        out = torch.empty((M, N), dtype=torch.float16, device=dev)
        ws = _lib.workspace(dev, int(_lib.load().mm_gemm_workspace_bytes(M, 2 * N, K)))
        gp, upk = _packed(gate_packed), _packed(up_packed)
        gs, us = _half(gate_scales), _half(up_scales)
        _lib.call("mm_fp4_gate_up_rowpacked", _lib.ptr(a), _lib.ptr(gp), _lib.ptr(gs),
                  _lib.ptr(upk), _lib.ptr(us), _lib.ptr(out), M, N, K, group_size, 1,
                  _lib.ptr(ws), ws.numel(), _lib.stream_of(a))
        return out
    return _gate_up(x, _packed(gate_packed).t().contiguous(), gate_scales,
                    _packed(up_packed).t().contiguous(), up_scales, group_size, 1)


def mmfp4_fused_gate_up_marlin(x: torch.Tensor, gate_packed: torch.Tensor,
                               gate_scales: torch.Tensor, up_packed: torch.Tensor,
                               up_scales: torch.Tensor, group_size: int = 128) -> torch.Tensor:
    """mmfp4_fused_gate_up on Marlin-layout [K/8, N] weights (no transpose):
    silu(x @ Wg) * (x @ Wu) -> [M, N] fp16 in one launch."""
    return _gate_up(x, gate_packed, gate_scales, up_packed, up_scales, group_size, 1)


def mmfp4_fused_qkv(A: torch.Tensor, Q_packed: torch.Tensor, Q_scales: torch.Tensor,
                    K_packed: torch.Tensor, K_scales: torch.Tensor, V_packed: torch.Tensor,
                    V_scales: torch.Tensor, group_size: int = 128):
    """Q, K, V projections sharing A (kernels_core.py:4875-4948):
    Q = A @ dequant(Q_packed, Q_scales), and likewise K and V; packed
    [K/8, N*] Marlin layout, scales [K/group_size, N*].  Returns (Q, K, V)
    fp16 [M, Nq], [M, Nk], [M, Nv] (shaped like A's leading dims).  M <= 16
    runs one launch over all three matrices' column tiles; larger M runs one
    launch per matrix (the reference falls back to separate GEMMs for M > 1)."""
    dev = _lib.require_device(A, Q_packed, Q_scales, K_packed, K_scales, V_packed, V_scales)
    orig_shape = A.shape
    if A.dim() == 1:
        A = A.reshape(1, -1)
    Kdim = A.shape[-1]
    M = A.numel() // Kdim
    mats = []
    for name, p, sc in (("Q", Q_packed, Q_scales), ("K", K_packed, K_scales),
                        ("V", V_packed, V_scales)):
        if p.dim() != 2 or p.shape[0] * FP4_PER_UINT != Kdim:
            raise ValueError(f"{name} weights: K mismatch {Kdim} vs "
                             f"{p.shape[0] * FP4_PER_UINT if p.dim() == 2 else '?'}")
        _check_groups(f"{name}_scales", sc, Kdim, p.shape[1], group_size)
        mats.append((_packed(p), _half(sc)))
    a = _half(A.reshape(M, Kdim))
    Ns = [p.shape[1] for p, _ in mats]
    lead = tuple(orig_shape[:-1]) if len(orig_shape) > 1 else (1,)
    if any(n % 4 for n in Ns):
        # the one-launch form stores 4 adjacent columns per lane; other widths
        # take one (padded) GEMM per matrix
        return tuple(marlin_gemm_fp4(a, p, sc, group_size).reshape(*lead, n)
                     for (p, sc), n in zip(mats, Ns))
    outs = [torch.empty((M, n), dtype=torch.float16, device=dev) for n in Ns]
    lib = _lib.load()
    ws_bytes = max([int(lib.mm_gemm_workspace_bytes(M, sum(Ns), Kdim))] +
                   [int(lib.mm_gemm_workspace_bytes(M, n, Kdim)) for n in Ns])
    ws = _lib.workspace(dev, ws_bytes)
    import ctypes
    Bt = (ctypes.c_void_p * 3)(*[_lib.ptr(p) for p, _ in mats])
    St = (ctypes.c_void_p * 3)(*[_lib.ptr(sc) for _, sc in mats])
    Ct = (ctypes.c_void_p * 3)(*[_lib.ptr(o) for o in outs])
    Nt = (ctypes.c_int * 3)(*Ns)
    _lib.call("mm_fp4_gemm_multi", _lib.ptr(a), 3, Bt, St, Ct, Nt, M, Kdim, group_size,
              _lib.ptr(ws), ws.numel(), _lib.stream_of(a))
    return tuple(o.reshape(*lead, n) for o, n in zip(outs, Ns))


def dequant_fp4(B_packed: torch.Tensor, scales: torch.Tensor, K: int, N: int,
                group_size: int = 32) -> torch.Tensor:
    """[K/8, N] -> [K, N] fp16, bit-exact with the reference dequantizer
    (kernels_core.py:2079-2133)."""
    dev = _lib.require_device(B_packed, scales)
    if tuple(B_packed.shape) != (K // 8, N) or K % 8 != 0:
        raise ValueError(f"B_packed shape {tuple(B_packed.shape)} != ({K // 8}, {N})")
    _check_groups("scales", scales, K, N, group_size)
    b, s = _packed(B_packed), _half(scales)
    out = torch.empty((K, N), dtype=torch.float16, device=dev)
    _lib.call("mm_fp4_dequant", _lib.ptr(b), _lib.ptr(s), _lib.ptr(out), K, N, group_size,
              _lib.stream_of(out))
    return out


def dequant_int4(B_packed: torch.Tensor, scales: torch.Tensor, zeros: torch.Tensor, K: int,
                 N: int, group_size: int = 32) -> torch.Tensor:
    """INT4 bulk dequant [K/8, N] -> [K, N] fp16 (metal_marlin.py:615-678)."""
    dev = _lib.require_device(B_packed, scales, zeros)
    if tuple(B_packed.shape) != (K // 8, N) or K % 8 != 0:
        raise ValueError(f"B_packed shape {tuple(B_packed.shape)} != ({K // 8}, {N})")
    _check_groups("scales", scales, K, N, group_size)
    _check_groups("zeros", zeros, K, N, group_size)
    b, s, z = _packed(B_packed), _half(scales), _half(zeros)
    out = torch.empty((K, N), dtype=torch.float16, device=dev)
    _lib.call("mm_u4_dequant", _lib.ptr(b), _lib.ptr(s), _lib.ptr(z), _lib.ptr(out), K, N,
              group_size, _lib.stream_of(out))
    return out


def dequant_fp4_decode_gemv(A: torch.Tensor, B_packed: torch.Tensor, scales: torch.Tensor,
                            K: int, N: int, group_size: int = 128) -> torch.Tensor:
    """M=1 GEMV, A [K] -> [N] fp16 (kernels_core.py:2135-2200)."""
    if A.numel() != K:
        raise ValueError(f"A has {A.numel()} elements, expected K={K}")
    if B_packed.shape[1] != N:
        raise ValueError(f"B_packed has N={B_packed.shape[1]}, expected {N}")
    return marlin_gemm_fp4(A.reshape(1, K), B_packed, scales, group_size).reshape(N)


def decode_gemv_fp4(A: torch.Tensor, B_packed: torch.Tensor, B_scales: torch.Tensor,
                    group_size: int = 128) -> torch.Tensor:
    """Decode GEMV (kernels_core.py:3755-3831 / :4814): A [K] -> [N] or A [M, K]
    -> [M, N]; M > 1 is the same fused GEMM."""
    squeeze = A.ndim == 1
    A2 = A.reshape(1, -1) if squeeze else A
    K_packed = B_packed.shape[0]
    if A2.shape[-1] != K_packed * FP4_PER_UINT:
        raise ValueError(f"K mismatch: A has K={A2.shape[-1]}, B_packed implies "
                         f"K={K_packed * FP4_PER_UINT}")
    out = marlin_gemm_fp4(A2, B_packed, B_scales, group_size)
    return out.reshape(-1) if squeeze else out


def mmfp4_gemm(A: torch.Tensor, B_packed: torch.Tensor, B_scales: torch.Tensor,
               group_size: int = 128) -> torch.Tensor:
    """MMFP4 fused GEMM (kernels_core.py:4804-4812 -> MetalKernels.mmfp4_gemm
    :4550-4633): A [M, K], B_packed [K/8, N], B_scales [K/group_size, N] as the
    kernel reads them (shaders/mmfp4_gemm.metal:570-588, and the M=1
    decode_gemv_fp4_wide, decode_gemv.metal:4,40).  Scales given as
    [N, K/group_size] are accepted when the shape says so unambiguously (the
    layer's _optimized_scale_load, layers/mmfp4_linear.py:53-86, transposes
    them); at decode sizes they are read in place (mm_fp4_gemm_mmfp4), else
    transposed.  A square tensor is read as [K/group_size, N]."""
    K = B_packed.shape[0] * FP4_PER_UINT
    N = B_packed.shape[1]
    if group_size <= 0 or K % group_size != 0:
        raise ValueError(f"K={K} must be divisible by group_size={group_size}")
    if _scales_layout(B_scales, N, K // group_size, "B_scales") == 0:
        return marlin_gemm_fp4(A, B_packed, B_scales, group_size)
    M = 1
    for d in A.shape[:-1]:
        M *= d
    if 0 < M <= 16 and A.shape[-1] == K and N % 4 == 0 and group_size % 8 == 0:
        # decode sizes: the [N, K/g] scales are read in place (mm_fp4_gemm_mmfp4)
        dev = _lib.require_device(A, B_packed, B_scales)
        a = _half(A.reshape(M, K))
        b, s = _packed(B_packed), _half(B_scales)
        out = torch.empty((M, N), dtype=torch.float16, device=dev)
        ws = _lib.workspace(dev, int(_lib.load().mm_gemm_workspace_bytes(M, N, K)))
        _lib.call("mm_fp4_gemm_mmfp4", _lib.ptr(a), _lib.ptr(b), _lib.ptr(s), _lib.ptr(out), M, N,
                  K, group_size, _lib.ptr(ws), ws.numel(), _lib.stream_of(a))
        return out.reshape(*A.shape[:-1], N)
    return marlin_gemm_fp4(A, B_packed, B_scales.t().contiguous(), group_size)


def dequantize_mmfp4(packed: torch.Tensor, scales: torch.Tensor,
                     group_size: int = 128) -> torch.Tensor:
    """MMFP4 bulk dequant (kernels_core.py:4795-4802, 4699-4738) -> [K, N]
    fp16; scales [K/group_size, N] as shaders/mmfp4_dequant.metal reads them
    (scales[group_idx * N + n]); an unambiguous [N, K/group_size] tensor is
    transposed."""
    K = packed.shape[0] * FP4_PER_UINT
    N = packed.shape[1]
    if group_size <= 0 or K % group_size != 0:
        raise ValueError(f"K={K} must be divisible by group_size={group_size}")
    if _scales_layout(scales, N, K // group_size) == 1:
        scales = scales.t()
    return dequant_fp4(packed, scales, K, N, group_size)


def select_decode_kernel(M: int, N: int, K: int) -> str:
    """Kernel-family recommendation of kernels_core.py:3833-3852, same rule
    and names: "marlin_gemm_fp4" for M > 8, else "decode_gemv_fp4".  (The
    library chooses its own kernel inside mm_fp4_gemm: the skinny decode
    kernels up to M = 32, the MFMA tile kernel above.)"""
    del N, K
    return "marlin_gemm_fp4" if M > 8 else "decode_gemv_fp4"