"""Helpers shared by the GPU parity tests."""

from __future__ import annotations

import sys

import numpy as np
import torch

DEV = "cuda"


def to_dev(x: np.ndarray) -> torch.Tensor:
    if x.dtype == np.uint32:
        x = x.view(np.int32)
    return torch.from_numpy(np.ascontiguousarray(x)).to(DEV)


def to_np(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().numpy()


def announce(msg: str) -> None:
    """Name the case on stdout before a GPU step, so a fault names its test."""
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


def max_abs_rel(out, ref) -> float:
    out = np.asarray(out, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    return float(np.max(np.abs(out - ref))) / max(float(np.max(np.abs(ref))), 1e-30)


# Parity bar of record (north star): max |out - ref| / max |ref| <= 1e-2.
TOL = 1e-2
