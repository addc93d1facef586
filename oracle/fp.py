"""Exact float32 helpers for the oracle (test infrastructure only).

numpy has no float32 fused multiply-add and no bfloat16 type; the reference's
attention prep contracts ``k - ksum * inv_l`` into one FMA and its outputs are
rounded to bf16, so both are provided here exactly.
"""

from __future__ import annotations

import numpy as np


def fma_f32(a, b, c) -> np.ndarray:
    """Correctly rounded float32 ``a*b + c`` (one rounding), elementwise.

    The product of two float32 values is exact in float64. The sum with ``c``
    is formed in float64, its rounding error recovered exactly with TwoSum,
    and the float64 result turned into round-to-odd (a standard device: with
    53 >= 24 + 2 bits, rounding a round-to-odd value to float32 equals
    rounding the exact value once).
    """
    a64 = np.asarray(a, np.float32).astype(np.float64)
    b64 = np.asarray(b, np.float32).astype(np.float64)
    c64 = np.asarray(c, np.float32).astype(np.float64)
    p = a64 * b64                      # exact: 24 + 24 bits
    s = p + c64
    bb = s - p
    err = (p - (s - bb)) + (c64 - bb)  # TwoSum: p + c == s + err exactly
    s, err = np.broadcast_arrays(s, err)
    s = s.copy()
    bits = s.view(np.int64)
    inexact = err != 0
    even = (bits & 1) == 0
    fix = inexact & even & np.isfinite(s)
    # move to the neighbour toward the exact value; it has an odd last bit
    toward = np.where(err > 0, np.inf, -np.inf)
    s[fix] = np.nextafter(s[fix], toward[fix])
    return s.astype(np.float32)


def f32_to_bf16_bits(x) -> np.ndarray:
    """Round float32 to bfloat16 (round to nearest even), as uint16 bits."""
    x = np.ascontiguousarray(np.asarray(x, np.float32))
    u = x.view(np.uint32).astype(np.uint64)
    nan = np.isnan(x)
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    rounded[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return rounded


def bf16_bits_to_f32(b) -> np.ndarray:
    b = np.asarray(b, np.uint16).astype(np.uint32) << 16
    return b.view(np.float32)


def round_bf16(x) -> np.ndarray:
    """float32 -> nearest bfloat16 value, returned as float32."""
    return bf16_bits_to_f32(f32_to_bf16_bits(x))


def round_to(x, dtype: str) -> np.ndarray:
    """Round float32 values to ``dtype`` ("f16", "bf16", "f32"); float32 out."""
    x = np.asarray(x, np.float32)
    if dtype == "f32":
        return x.copy()
    if dtype == "f16":
        return x.astype(np.float16).astype(np.float32)
    if dtype == "bf16":
        return round_bf16(x)
    raise ValueError(dtype)
