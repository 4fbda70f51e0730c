"""On-disk format for FP4 checkpoints: safetensors with the packed weight
under `name` and its scales under `name.scales` (plus optional
`.group_size` / `.quant_type` / `.hadamard_block_size` metadata), and the
converter that writes it.

Reference: metal_marlin/quantized_loader.py:30-220 (QuantizedModel.load and
its helpers) and metal_marlin/quantize_fp4.py:399-508
(load_and_quantize_safetensors, convert_safetensors_to_fp4).  Files are read
with safetensors (no pickle).  Quantisation runs on the GPU
(`quantize_fp4`), so the converter needs a ROCm device; loading does not.
"""

from __future__ import annotations

import json
import logging
from collections.abc import Iterator
from dataclasses import dataclass, field
from pathlib import Path
from typing import Any

import numpy as np
import torch

from .quantize_fp4 import compute_quantization_error, quantize_fp4
from .quantized_linear import QuantizedTensor

__all__ = ["QuantizedModel", "load_and_quantize_safetensors", "convert_safetensors_to_fp4"]

logger = logging.getLogger(__name__)

_META_SUFFIXES = (".scales", "_scales", ".group_size", "_group_size", ".quant_type",
                  "_quant_type", ".hadamard_block_size", "_hadamard_block_size")


def _strip(name: str, suffix: str) -> str:
    return name[: -len(suffix)]


def _decode_quant_type(tensor: torch.Tensor) -> str | None:
    """A uint8/int8 tensor holding a UTF-8 format name (NUL padded)."""
    if tensor.numel() == 0 or tensor.dtype not in (torch.uint8, torch.int8):
        return None
    raw = bytes(tensor.flatten().to(torch.uint8).tolist()).strip(b"\x00")
    if not raw:
        return None
    try:
        return raw.decode("utf-8").strip()
    except UnicodeDecodeError:
        return raw.decode("latin-1", errors="ignore").strip()


def _get_group_size(tensor: torch.Tensor | None, config: dict[str, Any]) -> int:
    if tensor is not None and tensor.numel() > 0:
        return int(tensor.reshape(-1)[0].item())
    return int(config.get("group_size", 0))


def _normalize_format(fmt: str | None) -> str:
    if not fmt:
        return "fp4"
    fmt = fmt.lower()
    if fmt.startswith("marlin_"):
        fmt = fmt[len("marlin_"):]
    return {"fp4_e2m1": "fp4", "fp8_e4m3": "fp8", "int4_sym": "int4"}.get(fmt, fmt)


def _infer_original_shape(data: torch.Tensor, scales: torch.Tensor | None, group_size: int,
                          fmt: str) -> tuple[int, ...]:
    """Unpacked [rows, cols] of a packed weight, from its scales when they
    pin it, else from the packing factor (8 codes per word; 16 for int2)."""
    if scales is not None and scales.dim() == 2 and group_size > 0:
        if scales.shape[0] == data.shape[0]:
            return (int(scales.shape[0]), int(scales.shape[1]) * group_size)
        if scales.shape[0] * group_size == data.shape[0]:
            return (int(scales.shape[0]) * group_size, int(scales.shape[1]))
    pack = 16 if fmt == "int2" else 8
    if data.dim() >= 2:
        return (int(data.shape[0]), int(data.shape[1]) * pack)
    return (int(data.numel()) * pack,)


@dataclass
class QuantizedModel:
    """A quantized checkpoint: `weights` maps base names to QuantizedTensor
    (or plain tensors), `bf16_weights` holds bf16 tensors kept as they are
    (router gates and the like)."""

    config: dict[str, Any]
    weights: dict[str, QuantizedTensor | torch.Tensor]
    bf16_weights: dict[str, torch.Tensor] = field(default_factory=dict)

    @classmethod
    def load(cls, path: Path | str) -> "QuantizedModel":
        """Load `model.safetensors` (+ optional `quantization_config.json`)
        from the directory `path` (quantized_loader.py:38-138)."""
        from safetensors.torch import load_file

        path = Path(path)
        weights_path = path / "model.safetensors"
        if not weights_path.exists():
            raise FileNotFoundError(f"model.safetensors not found in {path}")
        config_path = path / "quantization_config.json"
        config = json.loads(config_path.read_text()) if config_path.exists() else {}
        tensors = load_file(str(weights_path))

        scales_map: dict[str, torch.Tensor] = {}
        group_map: dict[str, torch.Tensor] = {}
        qtype_map: dict[str, str] = {}
        hadamard_map: dict[str, torch.Tensor] = {}
        for name, t in tensors.items():
            for sep in (".", "_"):
                if name.endswith(f"{sep}scales"):
                    scales_map[_strip(name, f"{sep}scales")] = t
                elif name.endswith(f"{sep}group_size"):
                    group_map[_strip(name, f"{sep}group_size")] = t
                elif name.endswith(f"{sep}quant_type"):
                    q = _decode_quant_type(t)
                    if q is not None:
                        qtype_map[_strip(name, f"{sep}quant_type")] = q
                elif name.endswith(f"{sep}hadamard_block_size"):
                    hadamard_map[_strip(name, f"{sep}hadamard_block_size")] = t

        weights: dict[str, QuantizedTensor | torch.Tensor] = {}
        bf16: dict[str, torch.Tensor] = {}
        for name, t in tensors.items():
            if name.endswith(_META_SUFFIXES):
                continue
            base = name[:-len("_quantized")] if name.endswith("_quantized") else name
            quantized = (base in scales_map or base in group_map or base in qtype_map
                         or base in hadamard_map or name.endswith("_quantized"))
            if quantized:
                if base in weights or base in bf16:
                    continue
                scales = scales_map.get(base)
                if scales is None:
                    raise ValueError(f"Missing scales for quantized weight: {base}")
                gs = _get_group_size(group_map.get(base), config)
                fmt = _normalize_format(qtype_map.get(base) or config.get("format"))
                weights[base] = QuantizedTensor(
                    data=t, scales=scales, format=fmt, group_size=gs,
                    original_shape=_infer_original_shape(t, scales, gs, fmt),
                    needs_hadamard=base in hadamard_map, hadamard_matrix=None)
            elif t.dtype == torch.bfloat16:
                bf16[base] = t
            else:
                weights[base] = t
        return cls(config=config, weights=weights, bf16_weights=bf16)


def load_and_quantize_safetensors(path: str | Path, group_size: int = 128,
                                  skip_patterns: list[str] | None = None,
                                  ) -> Iterator[tuple[str, np.ndarray, np.ndarray | None]]:
    """Stream a safetensors file, quantizing 2-D weight matrices to FP4
    (quantize_fp4.py:399-440).  Yields (name, packed uint32 [K/8, N], scales
    fp16 [K/g, N]) for quantized tensors and (name, tensor, None) otherwise.
    Names containing any of `skip_patterns` (default embed / norm / bias /
    lm_head), non-2-D tensors, names without "weight" and shapes whose input
    dimension is not a multiple of 8 and of group_size are left as they are."""
    from safetensors import safe_open

    skip_patterns = skip_patterns or ["embed", "norm", "bias", "lm_head"]
    with safe_open(str(path), framework="numpy") as f:
        for name in f.keys():
            tensor = f.get_tensor(name)
            skip = any(p in name.lower() for p in skip_patterns)
            if (not skip and "weight" in name.lower() and tensor.ndim == 2
                    and tensor.shape[1] % 8 == 0 and tensor.shape[1] % group_size == 0):
                packed, scales = quantize_fp4(tensor, group_size)
                yield name, packed, scales
            else:
                yield name, tensor, None


def convert_safetensors_to_fp4(input_path: str | Path, output_path: str | Path,
                               group_size: int = 128, validate: bool = True) -> dict[str, Any]:
    """Write an FP4 checkpoint: packed weights under their own names, scales
    under `name.scales`, other tensors unchanged (quantize_fp4.py:445-508).
    Returns counts, sizes, the compression ratio and (validate=True) the
    per-tensor round-trip errors."""
    from safetensors import safe_open
    from safetensors.numpy import save_file

    out: dict[str, np.ndarray] = {}
    stats: dict[str, Any] = {"quantized_count": 0, "skipped_count": 0, "original_bytes": 0,
                             "quantized_bytes": 0, "errors": []}
    for name, tensor, scales in load_and_quantize_safetensors(input_path, group_size):
        if scales is None:
            out[name] = tensor
            stats["skipped_count"] += 1
            continue
        out[name] = tensor
        out[f"{name}.scales"] = scales
        stats["quantized_count"] += 1
        stats["original_bytes"] += tensor.shape[0] * tensor.shape[1] * 8 * 2
        stats["quantized_bytes"] += tensor.nbytes + scales.nbytes
        if validate:
            with safe_open(str(input_path), framework="numpy") as f:
                original = f.get_tensor(name)
            stats["errors"].append({"name": name, **compute_quantization_error(
                original, tensor, scales, group_size)})
    save_file(out, str(output_path))
    if stats["errors"]:
        stats["mean_rmse"] = float(np.mean([e["rmse"] for e in stats["errors"]]))
        stats["max_error"] = float(max(e["max_error"] for e in stats["errors"]))
    stats["compression_ratio"] = stats["original_bytes"] / max(stats["quantized_bytes"], 1)
    return stats
