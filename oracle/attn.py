"""Oracle: INT8-QK / 16-bit-PV attention (test infrastructure only).

Restates reference ``src/diffucore/kernels/int8_attn_sm80.cu`` (the sm75 file
has the same math) for any head dim ``D`` and for fp16 or bf16 inputs:

* ``k_colsum``   <- ``kv_stats_kernel`` + ``k_sum_kernel`` (``:92-142``): the
  per-channel key sum in the kernel's fixed float32 order: within each
  128-key window, 16 partial sums over keys ``r0+rg, r0+rg+16, ...``
  (``:101-115``), combined sequentially over ``rg`` (``:124-129``), then summed
  sequentially over windows (``:137-142``).
* ``k_quantize`` <- ``k_quant_kernel`` (``:38-90``): ``val = k - ksum * (1/L)``
  contracted into one fused multiply-add (the file is built without
  ``-fmad=false``, ``_attention.py:101``); per 64-key block
  ``ks = amax / 127`` and ``ki = rint(val * (127 / amax))`` (no clamp; 0 when
  ``amax == 0``); keys at and past ``L`` are zero.
* ``q_quantize`` <- the Q prologue of ``attn_kernel`` (``:341-388``): per token
  ``q8 = rint(q * (127 / amax))``; the logit scale is
  ``(amax / 127) * (float(sm_scale) * log2(e))`` (``:384``, ``:490``).
* ``int8_attention`` <- ``attn_kernel`` (``:196-448``): exact int32 scores, the
  base-2 softmax of ``S * (cq * ks_block)``, probabilities rounded to the
  16-bit PV operand type, and ``P V / sum(P)``. The softmax is evaluated in
  float64 against the global row max (the kernel's online rescaling is the
  same quantity up to float32 rounding).
"""

from __future__ import annotations

import numpy as np

from .fp import fma_f32, round_to

BC = 64          # keys per K-scale block (int8_attn_sm80.cu:25)
WIN = 128        # keys per column-sum window (FLUSH_EVERY * BC, :95)
LOG2E = np.float32(1.4426950408889634)


def _f32(x) -> np.ndarray:
    return np.asarray(x, np.float32)


def k_colsum(k) -> np.ndarray:
    """ksum float32 [B, H, D] from keys ``k`` [B, L, H, D] (fp16/bf16 values)."""
    k = _f32(k)
    B, L, H, D = k.shape
    nwin = -(-L // WIN)
    kp = np.zeros((B, H, nwin * WIN, D), np.float32)
    kp[:, :, :L, :] = k.transpose(0, 2, 1, 3)
    kp = kp.reshape(B, H, nwin, 8, 16, D)          # key = r0 + 16*i + rg
    part = np.zeros((B, H, nwin, 16, D), np.float32)
    for i in range(8):
        part = part + kp[:, :, :, i]
    kpart = np.zeros((B, H, nwin, D), np.float32)
    for rg in range(16):
        kpart = kpart + part[:, :, :, rg]
    ksum = np.zeros((B, H, D), np.float32)
    for w in range(nwin):
        ksum = ksum + kpart[:, :, w]
    return ksum


def k_smooth(k, ksum) -> np.ndarray:
    """``k - ksum * (1/L)`` as one float32 FMA; [B, H, L, D]."""
    k = _f32(k)
    L = k.shape[1]
    inv_l = np.float32(1.0) / np.float32(L)
    return fma_f32(-_f32(ksum)[:, :, None, :], inv_l, k.transpose(0, 2, 1, 3))


def k_quantize(k, ksum=None) -> tuple[np.ndarray, np.ndarray]:
    """(ki int8 [B, H, Lpad, D], ks float32 [B, H, Lpad/64]); ``Lpad`` is ``L``
    rounded up to 64 and the padded keys are zero."""
    k = _f32(k)
    B, L, H, D = k.shape
    if ksum is None:
        ksum = k_colsum(k)
    nblk = -(-L // BC)
    val = np.zeros((B, H, nblk * BC, D), np.float32)
    val[:, :, :L] = k_smooth(k, ksum)
    vb = val.reshape(B, H, nblk, BC * D)
    amax = np.abs(vb).max(axis=-1)
    with np.errstate(divide="ignore"):
        inv = np.where(amax > 0, np.float32(127.0) / amax, np.float32(0.0)).astype(np.float32)
    ks = (amax / np.float32(127.0)).astype(np.float32)
    ki = np.rint((vb * inv[..., None]).astype(np.float32)).astype(np.int8)
    return ki.reshape(B, H, nblk * BC, D), ks


def q_quantize(q) -> tuple[np.ndarray, np.ndarray]:
    """(q8 int8 [B, H, L, D], qs float32 [B, H, L]) with ``qs = amax / 127``."""
    q = _f32(q).transpose(0, 2, 1, 3)
    amax = np.abs(q).max(axis=-1)
    with np.errstate(divide="ignore"):
        inv = np.where(amax > 0, np.float32(127.0) / amax, np.float32(0.0)).astype(np.float32)
    q8 = np.rint((q * inv[..., None]).astype(np.float32)).astype(np.int8)
    return q8, (amax / np.float32(127.0)).astype(np.float32)


def logit_scale(qs, sm_scale: float) -> np.ndarray:
    """cq = qs * (float32(sm_scale) * log2 e), all float32 (``:384, :490``)."""
    return (_f32(qs) * (np.float32(sm_scale) * LOG2E)).astype(np.float32)


def int8_attention(q, k, v, sm_scale: float | None = None, p_dtype: str = "bf16",
                   out_dtype: str = "bf16") -> np.ndarray:
    """Attention over ``(B, L, H, D)`` q/k/v -> ``(B, Lq, H, D)`` float32 values
    rounded to ``out_dtype``; ``p_dtype`` is the PV operand type (the input type)."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    B, Lq, H, D = q.shape
    Lk = k.shape[1]
    if sm_scale is None:
        sm_scale = D ** -0.5
    q8, qs = q_quantize(q)
    ki, ks = k_quantize(k)
    cq = logit_scale(qs, sm_scale)                                   # [B,H,Lq]
    # integer scores, exact in float64 (|S| <= D * 128 * 128 < 2**53)
    s = q8.astype(np.float64) @ ki[:, :, :Lk].astype(np.float64).transpose(0, 1, 3, 2)
    ksk = np.repeat(ks, BC, axis=-1)[:, :, :Lk]                      # [B,H,Lk]
    c = (cq[..., :, None] * ksk[..., None, :]).astype(np.float32)    # float32 product
    t = s * c.astype(np.float64)
    t = t - t.max(axis=-1, keepdims=True)
    p = round_to(np.exp2(t).astype(np.float32), p_dtype).astype(np.float64)
    num = p @ v.transpose(0, 2, 1, 3).astype(np.float64)
    o = num / p.sum(axis=-1)[..., None]
    return round_to(o.astype(np.float32), out_dtype).transpose(0, 2, 1, 3)
