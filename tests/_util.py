"""Helpers shared by the tests: torch <-> numpy and error metrics."""

from __future__ import annotations

import numpy as np
import torch

DT = {torch.float16: "f16", torch.bfloat16: "bf16", torch.float32: "f32"}


def np32(t: torch.Tensor) -> np.ndarray:
    """Values of ``t`` as a float32 numpy array (exact for fp16/bf16/fp32)."""
    return t.detach().float().cpu().numpy()


def rel_l2(out, ref) -> float:
    out = np.asarray(out, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.linalg.norm(out - ref) / np.linalg.norm(ref))


def cosine(out, ref) -> float:
    a = np.asarray(out, np.float64).ravel()
    b = np.asarray(ref, np.float64).ravel()
    return float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b)))


def max_abs(out, ref) -> float:
    return float(np.abs(np.asarray(out, np.float64) - np.asarray(ref, np.float64)).max())
