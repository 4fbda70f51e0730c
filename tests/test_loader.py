"""The on-disk FP4 checkpoint format (quantized_loader.py:30-220,
quantize_fp4.py:399-508): QuantizedModel.load on hand-built safetensors
files (CPU), and the converter's output against the oracle quantizer (GPU)."""

from __future__ import annotations

import json

import numpy as np
import pytest
import torch
from safetensors.numpy import save_file as save_np
from safetensors.torch import save_file as save_torch

from oracle import fp4 as ofp4


def test_quantized_model_load_metadata(tmp_path):
    import mmfp4
    rng = np.random.default_rng(0)
    K, N, g = 256, 64, 128
    packed, scales = ofp4.quantize_fp4(rng.normal(0, 0.02, (N, K)).astype(np.float16), g)
    pk = lambda: torch.from_numpy(np.ascontiguousarray(packed).view(np.int32)).clone()
    sc = lambda: torch.from_numpy(np.ascontiguousarray(scales)).clone()
    t = {
        "a.weight": pk(),
        "a.weight.scales": sc(),
        "b.weight_quantized": pk(),
        "b.weight_scales": sc(),
        "b.weight_group_size": torch.tensor([g], dtype=torch.int32),
        "b.weight.quant_type": torch.tensor(list(b"marlin_fp4_e2m1\x00\x00"), dtype=torch.uint8),
        "c.weight": pk(),
        "c.weight.scales": sc(),
        "c.weight.hadamard_block_size": torch.tensor([64], dtype=torch.int32),
        "router.weight": torch.randn(8, K).to(torch.bfloat16),
        "norm.weight": torch.ones(K),
        "rp.weight": pk().t().contiguous(),                  # row-packed [N, K/8]
        "rp.weight.scales": sc().t().contiguous(),           # [N, K/g]
    }
    save_torch(t, str(tmp_path / "model.safetensors"))
    (tmp_path / "quantization_config.json").write_text(json.dumps({"group_size": g,
                                                                   "format": "fp4"}))
    m = mmfp4.QuantizedModel.load(tmp_path)
    assert m.config["group_size"] == g
    a, b, c = m.weights["a.weight"], m.weights["b.weight"], m.weights["c.weight"]
    for q in (a, b, c):
        assert isinstance(q, mmfp4.QuantizedTensor)
        assert q.format == "fp4" and q.group_size == g
        # quantized_loader.py:198-215 infers the shape for row-packed data
        # ([N, K/8] with scales [N, K/g]); Marlin-layout data takes its
        # packing-factor branch: (rows, 8 * cols).
        assert q.original_shape == (K // 8, N * 8)
        assert torch.equal(q.data, t["a.weight"])
    assert m.weights["rp.weight"].original_shape == (N, K)
    assert not a.needs_hadamard and c.needs_hadamard
    assert set(m.bf16_weights) == {"router.weight"}
    assert torch.equal(m.weights["norm.weight"], t["norm.weight"])
    assert "a.weight.scales" not in m.weights


def test_quantized_model_load_errors(tmp_path):
    import mmfp4
    with pytest.raises(FileNotFoundError):
        mmfp4.QuantizedModel.load(tmp_path)
    save_torch({"w_quantized": torch.zeros(4, 4, dtype=torch.int32)},
               str(tmp_path / "model.safetensors"))
    with pytest.raises(ValueError, match="Missing scales"):
        mmfp4.QuantizedModel.load(tmp_path)


@pytest.mark.gpu
def test_convert_then_load_then_gemm(tmp_path):
    """convert_safetensors_to_fp4 writes the oracle's codes bit for bit;
    loading the result and running the GEMM matches the oracle GEMM."""
    import mmfp4
    from gpu_helpers import TOL, announce, max_abs_rel, to_dev, to_np
    rng = np.random.default_rng(1)
    K, N, g = 512, 256, 128
    w = rng.normal(0, 0.02, (N, K)).astype(np.float16)
    src = {"layers.0.q_proj.weight": w, "layers.0.input_norm.weight": np.ones(K, np.float16),
           "lm_head.weight": rng.normal(0, 0.02, (128, K)).astype(np.float16),
           "odd.weight": rng.normal(0, 0.02, (16, 100)).astype(np.float16)}
    save_np(src, str(tmp_path / "in.safetensors"))
    (tmp_path / "q").mkdir()
    announce("convert_safetensors_to_fp4")
    stats = mmfp4.convert_safetensors_to_fp4(tmp_path / "in.safetensors",
                                             tmp_path / "q" / "model.safetensors", g)
    assert stats["quantized_count"] == 1 and stats["skipped_count"] == 3
    assert stats["compression_ratio"] > 3.5 and len(stats["errors"]) == 1
    m = mmfp4.QuantizedModel.load(tmp_path / "q")
    q = m.weights["layers.0.q_proj.weight"]
    op, os_ = ofp4.quantize_fp4(w, g)
    assert np.array_equal(q.data.numpy().view(np.uint32), op)
    assert np.array_equal(q.scales.numpy().view(np.uint16), os_.view(np.uint16))
    x = rng.normal(0, 1, (3, K)).astype(np.float16)
    out = mmfp4.marlin_gemm_fp4(to_dev(x), q.data.cuda(), q.scales.cuda(), g)
    assert max_abs_rel(to_np(out), ofp4.gemm_fp4_ref(x, op, os_, g)) <= TOL
    assert np.array_equal(m.weights["odd.weight"].numpy(), src["odd.weight"])


def test_quantized_model_format_names_and_packing(tmp_path):
    """Format-name sidecars (NUL padding, marlin_ prefix, aliases, empty), the
    config defaults, and the codes-per-word rule of the unpacked shape."""
    import mmfp4
    words = torch.zeros((4, 6), dtype=torch.int32)
    name = lambda b: torch.tensor(list(b), dtype=torch.uint8)
    t = {
        "i2.weight": words.clone(), "i2.weight.scales": torch.ones((3, 5)).half(),
        "i2.weight.quant_type": name(b"int2\x00"),
        "s.weight": words.clone(), "s.weight_scales": torch.ones((3, 5)).half(),
        "s.weight_quant_type": name(b"MARLIN_INT4_SYM"),
        "d.weight": words.clone(), "d.weight.scales": torch.ones((3, 5)).half(),
        "e.weight": words.clone(), "e.weight.quant_type": name(b"\x00\x00"),
    }
    save_torch(t, str(tmp_path / "model.safetensors"))
    (tmp_path / "quantization_config.json").write_text(json.dumps({"group_size": 64,
                                                                   "format": "fp8_e4m3"}))
    m = mmfp4.QuantizedModel.load(tmp_path)
    assert m.weights["i2.weight"].format == "int2"
    assert m.weights["i2.weight"].original_shape == (4, 6 * 16)
    assert m.weights["s.weight"].format == "int4"
    assert m.weights["s.weight"].original_shape == (4, 6 * 8)
    assert m.weights["d.weight"].format == "fp8" and m.weights["d.weight"].group_size == 64
    # a format sidecar with no name marks nothing: e.weight is a plain tensor
    assert torch.equal(m.weights["e.weight"], t["e.weight"])
