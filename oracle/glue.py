"""Oracle: per-head QK RMSNorm + rotary embedding (test infrastructure only).

Follows the two producers of the attention's q and k in the reference:

* FLUX ``RMSNorm`` / ``QKNorm`` and ``apply_rope`` (``flux_dit.py:129-151,
  179-184``): ``x32 = float(x)``, ``rrms = rsqrt(mean(x32**2) + 1e-6)``,
  ``n = round(round(x32 * rrms) * scale)``, then pairs ``(2i, 2i+1)``;
* Anima ``_qk_norm_rope_kernel`` (``_fused.py:114-139``):
  ``n = round(w * (x32 * rrms))``, then pairs ``(i, i + D/2)``.

Rotary step for a pair ``(a, b)`` with a position's 2x2 matrix ``f``:
``(round(f00*a + f01*b), round(f10*a + f11*b))``, each float32 product and sum
rounded on its own (numpy float32 arithmetic rounds every operation, and
neither reference contracts them). ``round`` is to the activation dtype.

The sum of squares is formed in float64 and rounded once, and ``rrms`` is the
correctly rounded float32 of ``1/sqrt(mean + eps)``: the reference's float32
reduction order and its hardware ``rsqrt`` are not fixed by its source, so
parity with either is a tolerance (one float32 ulp of ``rrms``), stated in
the tests.
"""

from __future__ import annotations

import numpy as np

from .fp import round_to


def rrms(x32: np.ndarray, eps: float) -> np.ndarray:
    """float32 ``1/sqrt(mean(x^2) + eps)`` over the last axis, [..., 1]."""
    sq = (x32 * x32).astype(np.float64)            # each x^2 rounded to float32 first
    mean = np.float32(sq.sum(-1, keepdims=True)) / np.float32(x32.shape[-1])
    mean = np.asarray(mean, np.float32)
    return (1.0 / np.sqrt((mean + np.float32(eps)).astype(np.float64))).astype(np.float32)


def qk_norm(x, w, eps: float, dtype: str, weight_f32: bool) -> np.ndarray:
    """The normalized, rounded values ``n`` of ``x`` [..., D] (float32 array
    holding ``dtype`` values)."""
    x32 = np.asarray(x, np.float32)
    w32 = np.asarray(w, np.float32)
    r = rrms(x32, eps)
    if weight_f32:
        return round_to(w32 * (x32 * r), dtype)
    return round_to(round_to(x32 * r, dtype) * w32, dtype)


def rope(n, freqs, dtype: str, half_pairs: bool) -> np.ndarray:
    """Rotary step on ``n`` [..., L, H, D] with ``freqs`` [.., L, D/2, 2, 2]
    (broadcast over the heads)."""
    n = np.asarray(n, np.float32)
    D = n.shape[-1]
    if half_pairs:
        a, b = n[..., : D // 2], n[..., D // 2:]
    else:
        a, b = n[..., 0::2], n[..., 1::2]
    f = np.asarray(freqs, np.float32)[..., :, None, :, :, :]     # [.., L, 1, D/2, 2, 2]
    oa = round_to(f[..., 0, 0] * a + f[..., 0, 1] * b, dtype)
    ob = round_to(f[..., 1, 0] * a + f[..., 1, 1] * b, dtype)
    out = np.empty(np.broadcast_shapes(oa.shape, n.shape[:-1] + (D // 2,))[:-1] + (D,), np.float32)
    if half_pairs:
        out[..., : D // 2], out[..., D // 2:] = oa, ob
    else:
        out[..., 0::2], out[..., 1::2] = oa, ob
    return out


def qk_norm_rope(x, w, freqs, eps: float, dtype: str, half_pairs: bool = False,
                 weight_f32: bool = False) -> np.ndarray:
    """``x`` [B, L, H, D] -> normalized (and rotated, if ``freqs``) values."""
    n = qk_norm(x, w, eps, dtype, weight_f32)
    return n if freqs is None else rope(n, freqs, dtype, half_pairs)
