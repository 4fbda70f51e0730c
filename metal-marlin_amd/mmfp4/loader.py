"""On-disk format for FP4 checkpoints and the converter that writes it.

Format (restated here from the reference's writer and reader,
metal_marlin/quantize_fp4.py:445-508 and metal_marlin/quantized_loader.py:
30-220):

* a directory holding `model.safetensors` and, optionally,
  `quantization_config.json` (a JSON object; `group_size` and `format` are
  the defaults for tensors that carry no sidecar of their own);
* a quantized matrix is a *record*: its data tensor, stored under the
  record's name `B` (or `B_quantized`), and sidecar tensors stored under
  `B<sep><field>` with `<sep>` either "." or "_":
    - `scales`              (required) fp16 group scales;
    - `group_size`          a 1-element integer tensor;
    - `quant_type`          the format name as NUL-padded UTF-8 bytes in a
                            uint8/int8 tensor (names are lower-cased and
                            reduced to a canonical form: a leading "marlin_"
                            is dropped, and fp4_e2m1 / fp8_e4m3 / int4_sym
                            are fp4 / fp8 / int4);
    - `hadamard_block_size` its presence marks the record as Hadamard-rotated;
* a key that names no record and has no sidecar is a plain tensor; bf16 plain
  tensors (router gates and the like) are reported apart.

The unpacked shape of a record follows from the data and scale shapes: data
rows equal to scale rows means the codes are packed along each row (row
packing, [N, K/8] with [N, K/g] scales: shape [N, groups * g]); data rows
equal to groups * g means unpacked rows; otherwise the last axis holds
`codes per word` codes (8, or 16 for int2).

Files are read with safetensors (no pickle).  Quantisation runs on the GPU
(`quantize_fp4`), so the converter needs a ROCm device; loading does not.
"""

from __future__ import annotations

import json
import logging
import re
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

# `<record><sep><field>` for every sidecar field of the format
_SIDECAR_KEY = re.compile(r"^(?P<record>.+)[._](?P<field>scales|group_size|quant_type|"
                          r"hadamard_block_size)$")
_DATA_MARK = "_quantized"
_CANONICAL_FORMAT = {"fp4_e2m1": "fp4", "fp8_e4m3": "fp8", "int4_sym": "int4"}
_CODES_PER_WORD = {"int2": 16}
_DEFAULT_CODES_PER_WORD = 8


@dataclass
class _Record:
    """Sidecars of one quantized matrix, gathered from the key scan."""
    scales: torch.Tensor | None = None
    group_size: torch.Tensor | None = None
    quant_type: str | None = None
    hadamard: bool = False
    data: torch.Tensor | None = None


def _format_name(t: torch.Tensor) -> str | None:
    """Text of a `quant_type` sidecar (None when it holds no name)."""
    if t.dtype not in (torch.uint8, torch.int8) or t.numel() == 0:
        return None
    text = t.reshape(-1).to(torch.uint8).numpy().tobytes().replace(b"\x00", b"")
    name = text.decode("utf-8", errors="ignore").strip()
    return name or None


def _canonical_format(name: str | None) -> str:
    name = (name or "fp4").lower()
    name = name.removeprefix("marlin_")
    return _CANONICAL_FORMAT.get(name, name)


def _unpacked_shape(data: torch.Tensor, scales: torch.Tensor, group_size: int,
                    fmt: str) -> tuple[int, ...]:
    if scales.dim() == 2 and group_size > 0:
        groups, cols = int(scales.shape[0]), int(scales.shape[1])
        if data.shape[0] == groups:              # row packing: [N, K/8], scales [N, K/g]
            return (groups, cols * group_size)
        if data.shape[0] == groups * group_size:  # unpacked rows
            return (groups * group_size, cols)
    per_word = _CODES_PER_WORD.get(fmt, _DEFAULT_CODES_PER_WORD)
    if data.dim() < 2:
        return (int(data.numel()) * per_word,)
    return (int(data.shape[0]), int(data.shape[1]) * per_word)


@dataclass
class QuantizedModel:
    """A quantized checkpoint: `weights` maps record names to QuantizedTensor
    (and plain tensors to themselves), `bf16_weights` holds bf16 plain
    tensors (router gates and the like)."""

    config: dict[str, Any]
    weights: dict[str, QuantizedTensor | torch.Tensor]
    bf16_weights: dict[str, torch.Tensor] = field(default_factory=dict)

    @classmethod
    def load(cls, path: Path | str) -> "QuantizedModel":
        """Read the checkpoint directory `path` (the format above; the
        reference reader is quantized_loader.py:38-138)."""
        from safetensors.torch import load_file

        path = Path(path)
        st_file = path / "model.safetensors"
        if not st_file.exists():
            raise FileNotFoundError(f"model.safetensors not found in {path}")
        cfg_file = path / "quantization_config.json"
        config = json.loads(cfg_file.read_text()) if cfg_file.exists() else {}
        tensors = load_file(str(st_file))

        # Pass 1: sidecars, keyed by record name.
        records: dict[str, _Record] = {}
        plain: list[str] = []
        for key, t in tensors.items():
            m = _SIDECAR_KEY.match(key)
            if m is None:
                plain.append(key)
                continue
            rec = records.setdefault(m["record"], _Record())
            fld = m["field"]
            if fld == "scales":
                rec.scales = t
            elif fld == "group_size":
                rec.group_size = t
            elif fld == "quant_type":
                rec.quant_type = _format_name(t)
            else:
                rec.hadamard = True

        # Pass 2: data tensors; a data key names a record when it carries the
        # `_quantized` mark or when sidecars were stored under its name.
        weights: dict[str, QuantizedTensor | torch.Tensor] = {}
        bf16: dict[str, torch.Tensor] = {}
        for key in plain:
            t = tensors[key]
            marked = key.endswith(_DATA_MARK)
            name = key[: -len(_DATA_MARK)] if marked else key
            rec = records.get(name)
            if rec is not None and rec.quant_type is None and rec.scales is None \
                    and rec.group_size is None and not rec.hadamard:
                rec = None   # a quant_type sidecar that held no name
            if rec is None and not marked:
                (bf16 if t.dtype == torch.bfloat16 else weights)[name] = t
                continue
            if name in weights or name in bf16:
                continue     # first data key of a record wins
            rec = rec or _Record()
            if rec.scales is None:
                raise ValueError(f"Missing scales for quantized weight: {name}")
            gs = (int(rec.group_size.reshape(-1)[0].item()) if rec.group_size is not None
                  and rec.group_size.numel() > 0 else int(config.get("group_size", 0)))
            fmt = _canonical_format(rec.quant_type or config.get("format"))
            weights[name] = QuantizedTensor(
                data=t, scales=rec.scales, format=fmt, group_size=gs,
                original_shape=_unpacked_shape(t, rec.scales, gs, fmt),
                needs_hadamard=rec.hadamard, hadamard_matrix=None)
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
