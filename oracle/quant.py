"""Oracle: per-row int8 quantizer and ConvRot rotation (test infrastructure only).

Follows reference ``src/diffucore/models/_int8.py``:

* ``quantize_rows``  <- ``_quantize_rows`` (``_int8.py:87-97``) and the Triton
  ``_store_quantized`` (``_int8.py:392-397``): ``scale = max(amax/127, 1e-30)``,
  ``q = clamp(rint(x / scale), -128, 127)``, all in float32 with an IEEE
  division.
* ``hadamard``       <- ``_hadamard`` (``_int8.py:64-76``).
* ``rotate_matmul``  <- ``_rotate`` (``_int8.py:79-84``): ``t @ H`` per group.
* ``rotate_butterfly`` <- ``_hadamard_rows`` (``_int8.py:363-372``), with the
  summation order this build fixes (see its docstring).
* ``ln_mod_quantize`` <- the LayerNorm-modulate glue ``_ln_mod_kernel``
  (``_fused.py:73-85``) followed by ``quantize_activation``.
* ``gelu`` / ``act_quantize`` <- the fused MLP middle ``_gelu`` and
  ``_gelu_f16_rot_quant_kernel`` (``_int8.py:433-443``, ``_gelu_quantize``
  ``:348-358``); the tanh form is torch's ``gelu(approximate="tanh")`` that
  FLUX's MLPs use (``flux_dit.py:228-239, 335``).
* ``geglu`` <- the UNet's ``GEGLU.forward`` (``unet.py:148-155``):
  ``x * F.gelu(gate)`` on the two chunks of the projection output.
"""

from __future__ import annotations

import numpy as np
from scipy.special import erf as _erf64

from .fp import round_to

_H4 = np.array([[1, 1, 1, -1], [1, 1, -1, 1], [1, -1, 1, 1], [-1, 1, 1, 1]], np.float32)
SCALE_FLOOR = np.float32(1e-30)


def quantize_rows(t) -> tuple[np.ndarray, np.ndarray]:
    """(int8 [M, K], float32 scale [M]) for float32 rows ``t`` [M, K]."""
    t = np.asarray(t, np.float32)
    amax = np.abs(t).max(axis=-1) if t.shape[-1] else np.zeros(t.shape[:-1], np.float32)
    scale = np.maximum(amax / np.float32(127.0), SCALE_FLOOR).astype(np.float32)
    x = (t / scale[..., None]).astype(np.float32)
    q = np.clip(np.rint(x), -128, 127).astype(np.int8)
    return q, scale


def hadamard(n: int) -> np.ndarray:
    """Normalized regular Hadamard of order ``n`` (a power of 4), float32."""
    h = _H4
    while h.shape[0] < n:
        h = np.kron(h, _H4)
    if h.shape[0] != n:
        raise ValueError(f"ConvRot group must be a power of 4, got {n}")
    return (h / np.float32(n ** 0.5)).astype(np.float32)


def rotate_matmul(t, group: int) -> np.ndarray:
    """``t @ H`` per ``group``-wide slice of the last dim (float32 matmul)."""
    t = np.asarray(t, np.float32)
    if not group:
        return t
    shape = t.shape
    out = t.reshape(-1, shape[-1] // group, group) @ hadamard(group)
    return out.reshape(shape).astype(np.float32)


def _h4_along(y: np.ndarray, axis: int) -> np.ndarray:
    """``y @ H4`` along ``axis`` (length 4): ``S - 2 * y[3 - j]`` with the sum
    formed pairwise, ``S = (y0 + y1) + (y2 + y3)``."""
    y0, y1, y2, y3 = (np.take(y, i, axis=axis) for i in range(4))
    s = (y0 + y1) + (y2 + y3)
    out = [s - np.float32(2.0) * yy for yy in (y3, y2, y1, y0)]
    return np.stack(out, axis=axis).astype(np.float32)


def rotate_butterfly(t, group: int = 256) -> np.ndarray:
    """ConvRot rotation as the in-register butterfly the HIP kernel runs.

    The in-group index ``i`` (0..255) is read as four base-4 digits
    ``i = 64*d1 + 16*d2 + 4*d3 + d4``; ``H4`` is applied along ``d1``, then
    ``d2``, ``d3``, ``d4`` (the reference's Triton order, ``_int8.py:367-371``),
    each as ``sum - 2 * reversed`` with the four-term sum taken pairwise
    ``(y0 + y1) + (y2 + y3)``; the result is scaled by 1/16 last (exact).
    The reference's Triton ``tl.sum`` order is implementation-defined, so this
    pairwise order is the one this build documents and pins.
    """
    t = np.asarray(t, np.float32)
    if not group:
        return t
    if group != 256:
        raise ValueError("the butterfly is defined for group 256")
    shape = t.shape
    y = t.reshape(-1, shape[-1] // 256, 4, 4, 4, 4)
    for axis in (2, 3, 4, 5):
        y = _h4_along(y, axis)
    return (y.reshape(shape) * np.float32(0.0625)).astype(np.float32)


def quantize_activation(x, group: int) -> tuple[np.ndarray, np.ndarray]:
    """What the HIP quantize kernel computes: butterfly rotation (group 256)
    or none (group 0), then ``quantize_rows``."""
    x = np.asarray(x, np.float32)
    return quantize_rows(rotate_butterfly(x, group) if group else x)


def quantize_weight(w, group: int) -> tuple[np.ndarray, np.ndarray]:
    """``quantize_weight`` (``_int8.py:100-102``): matmul-form rotation."""
    return quantize_rows(rotate_matmul(np.asarray(w, np.float32), group))


def dequantize_weight(q, scale, group: int) -> np.ndarray:
    """``dequantize_weight`` (``_int8.py:105-107``)."""
    return rotate_matmul(np.asarray(q, np.float32) * np.asarray(scale, np.float32)[:, None], group)


def gelu(x, approximate: str = "none", dtype: str = "bf16") -> np.ndarray:
    """GELU of float32 ``x`` rounded to the 16-bit ``dtype`` ("bf16"/"f16"), as
    the reference's ``_gelu`` rounds it (``_int8.py:433-435``):
    ``(0.5 * h) * (1 + erf(h * 0.7071067811865476))``, float32 operations in
    that order; ``approximate="tanh"``: ``(0.5 * x) * (1 + tanh(0.7978845608028654
    * (x + 0.044715 * ((x * x) * x))))``. erf and tanh are evaluated in float64
    and rounded once to float32. A device's float32 erf / tanh may differ from
    that by an ulp or two; the rounding to 16 bits hides it except next to a
    rounding boundary, so for the transcendental itself parity is within
    tolerance, and everything after it (rotation, codes) is exact."""
    x = np.asarray(x, np.float32)
    if approximate == "none":
        t = (x * np.float32(0.7071067811865476)).astype(np.float32)
        e = _erf64(t.astype(np.float64)).astype(np.float32)
    elif approximate == "tanh":
        inner = (np.float32(0.7978845608028654) * (x + np.float32(0.044715) * ((x * x) * x))).astype(np.float32)
        e = np.tanh(inner.astype(np.float64)).astype(np.float32)
    else:
        raise ValueError(f"unknown approximate={approximate!r}")
    y = ((np.float32(0.5) * x) * (np.float32(1.0) + e)).astype(np.float32)
    return round_to(y, dtype)


def geglu(x2, dtype: str = "f16") -> np.ndarray:
    """``x * gelu(gate)`` for ``x, gate = x2.chunk(2, -1)`` (``unet.py:148-155``):
    the erf GELU of ``gate`` rounded to ``dtype`` (torch's half-precision
    ``F.gelu``), then the product of two 16-bit values (exact in float32)
    rounded to ``dtype`` once (torch's half-precision multiply)."""
    x2 = np.asarray(x2, np.float32)
    n = x2.shape[-1] // 2
    x, gate = x2[..., :n], x2[..., n:]
    return round_to((x * gelu(gate, "none", dtype)).astype(np.float32), dtype)


def act_quantize(x2, group: int, approximate: str = "none", dtype: str = "bf16", prefix=None):
    """``quantize_activation`` of the rows of ``cat(prefix, act(x2))``: what
    the fused HIP kernel computes (prefix columns taken as they are);
    ``approximate`` is "none" / "tanh" (GELU forms) or "geglu"."""
    h = geglu(x2, dtype) if approximate == "geglu" else gelu(x2, approximate, dtype)
    if prefix is not None:
        h = np.concatenate([np.asarray(prefix, np.float32), h], axis=-1)
    return quantize_activation(h, group)


def ln_mod_quantize(x, sc1, shift, rows_per_mod: int, eps: float, group: int, dtype: str = "bf16"):
    """``quantize_activation`` of ``round(LayerNorm(x) * sc1 + shift)``: the
    reference's ``_ln_mod_kernel`` (``_fused.py:73-85``) in float32 - mean =
    sum / K, centered variance, rstd = 1 / sqrt(var + eps), y = ((x - mean) *
    rstd) * sc1 + shift with separate roundings - rounded to ``dtype``. The
    row sums are float32 in numpy's order; the kernel's order differs, so
    parity is within the last bits of the mean and rstd."""
    x = np.asarray(x, np.float32)
    sc1 = np.asarray(sc1, np.float32)
    shift = np.asarray(shift, np.float32)
    K = x.shape[1]
    m = np.arange(x.shape[0]) // rows_per_mod
    mean = (x.sum(axis=1, dtype=np.float32) / np.float32(K)).astype(np.float32)
    xc = (x - mean[:, None]).astype(np.float32)
    var = ((xc * xc).sum(axis=1, dtype=np.float32) / np.float32(K)).astype(np.float32)
    rstd = (np.float32(1.0) / np.sqrt(var + np.float32(eps))).astype(np.float32)
    y = (((xc * rstd[:, None]).astype(np.float32) * sc1[m]).astype(np.float32) + shift[m]).astype(np.float32)
    return quantize_activation(round_to(y, dtype), group)
