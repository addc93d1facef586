"""Per-head QK RMSNorm + rotary embedding on the gfx950 kernel
``dc_qk_norm_rope``: the producer side of the INT8 attention.

Two formulations, both with float32 statistics and the reference's rounding
points (each float32 product and sum rounded on its own):

* FLUX (``flux_dit.py:129-151, 179-184``; eager torch in the reference):
  ``n = round(round(x * rrms) * scale)``, then rotary pairs ``(2i, 2i+1)``;
* Anima (``_fused.py:114-139, 174-185``, a Triton kernel there):
  ``n = round(w * (x * rrms))``, then rotary pairs ``(i, i + D/2)``;

with ``rrms = rsqrt(mean(x^2) + eps)`` and the frequency table in the
reference's ``[.., L, D/2, 2, 2]`` float32 layout. One launch covers q, k and
an optional copy of v, writing into any (B, L, H, D) views, so a caller can
gather several streams straight into the attention's input buffers.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib

ROPE_HALF, WEIGHT_F32 = 1, 2            # DC_QK_ROPE_HALF, DC_QK_WEIGHT_F32
_DTYPES = (torch.float16, torch.bfloat16)
_HEAD_DIMS = (32, 64, 128, 256)


def _blhd(t: torch.Tensor, shape, what: str) -> torch.Tensor:
    if t.dim() != 4 or tuple(t.shape) != tuple(shape):
        raise RuntimeError(f"{what}: expected shape {tuple(shape)}, got {tuple(t.shape)}")
    if t.stride(-1) != 1:
        raise RuntimeError(f"{what}: the head dim must be contiguous")
    return t


def _freq_strides(freqs: torch.Tensor, B: int, L: int, D: int):
    """(batch stride, position stride) in floats of a ``[.., L, D/2, 2, 2]``
    table whose leading dims are 1 or B."""
    if freqs.dtype != torch.float32 or freqs.dim() < 4 or tuple(freqs.shape[-4:]) != (L, D // 2, 2, 2):
        raise RuntimeError(f"freqs: expected float32 [.., {L}, {D // 2}, 2, 2], got {freqs.dtype} "
                           f"{tuple(freqs.shape)}")
    if freqs.stride(-1) != 1 or freqs.stride(-2) != 2 or freqs.stride(-3) != 4:
        raise RuntimeError("freqs: the [D/2, 2, 2] block of a position must be contiguous")
    lead = [(n, s) for n, s in zip(freqs.shape[:-4], freqs.stride()[:-4]) if n != 1]
    if not lead:
        return 0, freqs.stride(-4)
    if len(lead) != 1 or lead[0][0] != B:
        raise RuntimeError(f"freqs: leading dims {tuple(freqs.shape[:-4])} are neither 1 nor the batch {B}")
    return lead[0][1], freqs.stride(-4)


def norm_rope(q: torch.Tensor, q_weight: torch.Tensor, eps: float, freqs: torch.Tensor | None = None, *,
              k: torch.Tensor | None = None, k_weight: torch.Tensor | None = None, v: torch.Tensor | None = None,
              half_pairs: bool = False, weight_f32: bool = False, out_q: torch.Tensor | None = None,
              out_k: torch.Tensor | None = None, out_v: torch.Tensor | None = None):
    """RMSNorm (weights ``q_weight`` / ``k_weight``, ``[D]``) and rotary
    embedding of ``q`` (and ``k``), plus a copy of ``v``, for ``(B, L, H, D)``
    views with D contiguous; returns ``(q_out, k_out, v_out)`` (None where no
    input). ``freqs`` is ``[.., L, D/2, 2, 2]`` float32 for these L positions
    (None: norm only). ``half_pairs`` / ``weight_f32`` select the Anima
    formulation; the defaults are FLUX's. Outputs may be given (any
    (B, L, H, D) views, e.g. slices of a larger buffer) or are allocated."""
    so = _lib.require()
    if not q.is_cuda:
        raise RuntimeError("norm_rope: GPU only (no CPU path)")
    if q.dtype not in _DTYPES:
        raise RuntimeError(f"norm_rope: dtype must be float16 or bfloat16, got {q.dtype}")
    B, L, H, D = q.shape
    shape = (B, L, H, D)
    _blhd(q, shape, "q")
    if k is not None:
        _blhd(k, shape, "k")
        if k.dtype != q.dtype or k_weight is None:
            raise RuntimeError("norm_rope: k needs q's dtype and a k_weight")
    if v is not None:
        _blhd(v, shape, "v")
        if v.dtype != q.dtype:
            raise RuntimeError("norm_rope: v needs q's dtype")
    wdt = q_weight.dtype
    for w in (q_weight, k_weight):
        if w is not None and (w.dtype != wdt or w.dtype not in (q.dtype, torch.float32) or tuple(w.shape) != (D,)
                              or not w.is_contiguous()):
            raise RuntimeError(f"norm_rope: weights must be contiguous [{D}] of the activation dtype or float32")

    def out_for(x, given, what):
        if x is None:
            return None
        if given is None:
            return torch.empty(shape, device=q.device, dtype=q.dtype)
        if given.dtype != q.dtype:
            raise RuntimeError(f"{what}: dtype {given.dtype} != {q.dtype}")
        return _blhd(given, shape, what)

    oq, ok_, ov = out_for(q, out_q, "out_q"), out_for(k, out_k, "out_k"), out_for(v, out_v, "out_v")
    fb, fl = _freq_strides(freqs, B, L, D) if freqs is not None else (0, 0)
    flags = (ROPE_HALF if half_pairs else 0) | (WEIGHT_F32 if weight_f32 else 0)

    def ptr(t):
        return t.data_ptr() if t is not None else None

    def st(t):
        return _lib.strides3(t) if t is not None else None

    with _lib.device_ctx(q.device):
        rc = so.dc_qk_norm_rope(_lib.dtype_code(q.dtype), B, L, H, D, flags, ctypes.c_float(eps),
                                ptr(q), st(q), ptr(q_weight), ptr(k), st(k), ptr(k_weight), _lib.dtype_code(wdt),
                                ptr(freqs), fb, fl, ptr(oq), st(oq), ptr(ok_), st(ok_), ptr(v), st(v), ptr(ov),
                                st(ov), _lib.stream_ptr(q.device))
    _lib.check(rc, "dc_qk_norm_rope")
    return oq, ok_, ov


def qk_ok(x: torch.Tensor, n_heads: int, head_dim: int) -> bool:
    """Whether :func:`qk_norm_rope` takes ``x`` (``_fused.py:167-170``, here for
    fp16 and bf16 and head dims 32 to 256)."""
    return (x.is_cuda and x.dtype in _DTYPES and x.dim() == 3 and x.stride(2) == 1 and head_dim in _HEAD_DIMS
            and x.shape[2] == n_heads * head_dim and x.stride(1) % 8 == 0 and x.stride(0) % 8 == 0
            and x.data_ptr() % 16 == 0)


def qk_norm_rope(x: torch.Tensor, weight: torch.Tensor, eps: float, n_heads: int, head_dim: int,
                 freqs: torch.Tensor | None = None) -> torch.Tensor:
    """Anima's fused q/k glue (``_fused.py:174-185``): RMSNorm per head with the
    weight applied in float32, then RoPE on pairs ``(i, i + head_dim/2)`` with
    ``freqs`` ``(L, head_dim/2, 2, 2)``, of ``x`` ``(B, S, H*HD)`` ->
    ``(B, S, H, HD)``."""
    B, S, _ = x.shape
    xv = x.view(B, S, n_heads, head_dim) if x.is_contiguous() else x.unflatten(2, (n_heads, head_dim))
    f = None
    if freqs is not None:
        f = freqs[:S] if freqs.shape[-4] != S else freqs
    out, _, _ = norm_rope(xv, weight, eps, f, half_pairs=True, weight_f32=True)
    return out


def flux_qk_norm_rope(q: torch.Tensor, k: torch.Tensor, q_scale: torch.Tensor, k_scale: torch.Tensor,
                      pe: torch.Tensor, v: torch.Tensor | None = None, out=(None, None, None)):
    """FLUX's ``QKNorm`` then ``apply_rope`` (``flux_dit.py:129-151, 179-184``)
    for ``(B, L, H, D)`` views, ``pe`` ``[.., L, D/2, 2, 2]``: one launch, with
    an optional copy of ``v`` alongside."""
    return norm_rope(q, q_scale, 1e-6, pe, k=k, k_weight=k_scale, v=v, out_q=out[0], out_k=out[1], out_v=out[2])


def set_fused_glue(module: torch.nn.Module, on: bool) -> int:
    """Set ``fused_glue`` on every submodule that has the slot and return how
    many (``_fused.py:40-48``): blocks with it on run their q/k norm + rotary
    glue through :func:`norm_rope`."""
    slots = [m for m in module.modules() if hasattr(m, "fused_glue")]
    for m in slots:
        m.fused_glue = bool(on)
    return len(slots)
