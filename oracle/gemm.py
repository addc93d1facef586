"""Oracle: exact int8 GEMM and the W8A8 epilogue (test infrastructure only).

* ``int_mm``  <- ``int_mm`` (``_int8.py:200-207``): ``q @ w.T`` in int32.
* ``rescale`` <- ``rescale`` torch path (``_int8.py:322-323``) and the Triton
  ``_rescale_kernel`` (``_int8.py:408-417``); the fused GEMM epilogue of
  ``kernels/int8_gemm_sm75.cu:31-38`` rounds identically
  (``tests/test_int8.py:174-183``).
"""

from __future__ import annotations

import numpy as np

from .fp import round_to


def int_mm(q, w) -> np.ndarray:
    """int32 ``q @ w.T`` for int8 ``q`` [M, K] and ``w`` [N, K] (exact)."""
    q = np.asarray(q, np.int8)
    w = np.asarray(w, np.int8)
    if q.shape[1] * 128 * 128 >= 2**53:
        raise OverflowError("K too large for an exact float64 product")
    # every partial sum is an integer below 2**53, so float64 BLAS is exact
    acc = q.astype(np.float64) @ w.astype(np.float64).T
    if acc.size and (acc.max() > 2**31 - 1 or acc.min() < -2**31):
        raise OverflowError("int32 accumulator overflow")
    return acc.astype(np.int64).astype(np.int32)


def rescale(acc, sx, sw, bias, dtype: str) -> np.ndarray:
    """``cast(float(acc) * (sx[:, None] * sw))`` then ``+ cast(bias)`` in
    ``dtype`` ("f16", "bf16" or "f32"); returns the values as float32.

    Order (``_int8.py:322-323``): the int32 accumulator becomes float32 (round
    to nearest even), ``sx * sw`` is formed first, the product is rounded to the
    output dtype, and the bias, already rounded to the output dtype, is added
    with one more rounding to the output dtype.
    """
    a = np.asarray(acc, np.int32).astype(np.float32)
    s = (np.asarray(sx, np.float32)[:, None] * np.asarray(sw, np.float32)[None, :]).astype(np.float32)
    y = round_to((a * s).astype(np.float32), dtype)
    if bias is not None:
        b = round_to(np.asarray(bias, np.float32), dtype)
        y = round_to((y + b[None, :]).astype(np.float32), dtype)
    return y


def w8a8_linear(q, sx, w, sw, bias, dtype: str) -> np.ndarray:
    """``Int8Linear.matmul_quantized`` (``_int8.py:163-167``) on quantized rows."""
    return rescale(int_mm(q, w), sx, sw, bias, dtype)
