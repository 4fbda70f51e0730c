"""GPU parity of the fused QKV projection (one launch over the Q, K and V
matrices' column tiles for M <= 16) against the fp32 reference built from
the bit-exact dequant, plus the oracle on a small ragged case."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from gpu_helpers import TOL, announce, max_abs_rel, to_dev, to_np
from oracle import fp4 as ofp4

pytestmark = pytest.mark.gpu


def _weights(gen, K, N, g):
    import mmfp4
    w = (torch.randn((N, K), generator=gen, device="cuda") * 0.02).half()
    p, s = mmfp4.quantize_fp4(w, group_size=g)
    return p, s, mmfp4.dequant_fp4(p, s, K, N, g).float()


@pytest.mark.parametrize("M,K,Ns,g", [(1, 4096, (4096, 1024, 1024), 128),
                                      (8, 4096, (4096, 1024, 1024), 128),
                                      (16, 14336, (512, 256, 256), 128),
                                      (17, 4096, (4096, 1024, 1024), 128),
                                      (64, 4096, (4096, 1024, 1024), 128),
                                      (3, 1024, (260, 132, 68), 32),
                                      (1, 512, (258, 130, 64), 64)])
def test_fused_qkv_vs_fp32_reference(M, K, Ns, g):
    import mmfp4
    gen = torch.Generator(device="cuda").manual_seed(M + K)
    mats = [_weights(gen, K, n, g) for n in Ns]
    x = torch.randn((M, K), generator=gen, device="cuda").half()
    announce(f"fused qkv M={M} K={K} Ns={Ns}")
    outs = mmfp4.mmfp4_fused_qkv(x, mats[0][0], mats[0][1], mats[1][0], mats[1][1], mats[2][0],
                                 mats[2][1], g)
    for o, (_, _, w), n in zip(outs, mats, Ns):
        assert tuple(o.shape) == (M, n)
        assert max_abs_rel(to_np(o), to_np(x.float() @ w)) <= TOL
    again = mmfp4.mmfp4_fused_qkv(x, mats[0][0], mats[0][1], mats[1][0], mats[1][1], mats[2][0],
                                  mats[2][1], g)
    for o, o2 in zip(outs, again):
        assert torch.equal(o, o2)


def test_fused_qkv_1d_input_vs_oracle(rng):
    import mmfp4
    K, Ns, g = 256, (64, 32, 32), 64
    ws = [ofp4.quantize_fp4(rng.normal(0, 0.02, (n, K)).astype(np.float16), g) for n in Ns]
    x = rng.normal(0, 1, (K,)).astype(np.float16)
    announce("fused qkv 1-D input vs oracle")
    outs = mmfp4.mmfp4_fused_qkv(to_dev(x), *[to_dev(t) for pair in ws for t in pair], g)
    for o, (p, s), n in zip(outs, ws, Ns):
        assert tuple(o.shape) == (1, n)
        ref = x.astype(np.float32)[None] @ ofp4.dequant_fp4_f32(p, s, g)
        assert max_abs_rel(to_np(o), ref) <= TOL


def test_fused_qkv_errors():
    import mmfp4
    x = torch.zeros((1, 64), dtype=torch.float16, device="cuda")
    p = torch.zeros((8, 16), dtype=torch.int32, device="cuda")
    s = torch.zeros((1, 16), dtype=torch.float16, device="cuda")
    with pytest.raises(ValueError, match="K weights: K mismatch"):
        mmfp4.mmfp4_fused_qkv(x, p, s, p[:4], s, p, s, 64)
