"""dc_qk_norm_rope on the GPU: FLUX's QKNorm + apply_rope (reference
``flux_dit.py:129-151, 179-184``) and Anima's fused q/k glue
(``_fused.py:114-139, 174-185``) against torch's eager ops of the same
formulas on the same GPU and against the oracle (``oracle/glue.py``).

Tolerance (the reductions' order and rsqrt are not fixed by the reference):
at least 99% of the outputs are bit-equal and every one is within one dtype
ulp of the row's size, ``|d| <= u * (|out| + 2 max|row|)``. Rows whose sum of
squares is exact in any order (small integers) and the plain v copy are
bit-exact.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from diffucore_amd import _qknorm as QK
from oracle import glue as OGL
from tests._util import DT, np32

pytestmark = pytest.mark.gpu

ULP = {torch.bfloat16: 2.0 ** -7, torch.float16: 2.0 ** -10}


def _table(L, half, device, seed=0):
    """FLUX rotary matrices [1, 1, L, D/2, 2, 2] (float32) from random angles."""
    g = torch.Generator().manual_seed(seed)
    ang = (torch.rand(L, half, generator=g, dtype=torch.float64) * 2 - 1) * math.pi
    c, s = ang.cos(), ang.sin()
    return torch.stack((c, -s, s, c), -1).unflatten(-1, (2, 2)).float()[None, None].to(device)


def _eager_flux(q, scale, pe):
    """The reference's QKNorm (RMSNorm) + apply_rope as eager torch ops on
    (B, L, H, D) -> same layout."""
    xf = q.float()
    n = (xf * torch.rsqrt(torch.mean(xf ** 2, dim=-1, keepdim=True) + 1e-6)).to(q.dtype) * scale
    n = n.to(q.dtype)
    if pe is None:
        return n
    f = pe[0, 0][:, None]                                            # [L, 1, D/2, 2, 2]
    n_ = n.float().reshape(*n.shape[:-1], -1, 1, 2)
    out = f[..., 0] * n_[..., 0] + f[..., 1] * n_[..., 1]
    return out.reshape(*n.shape).to(q.dtype)


def _eager_anima(x, w, f, eps):
    half = x.shape[-1] // 2
    xf = x.float()
    xa, xb = xf[..., :half], xf[..., half:]
    r = torch.rsqrt(((xa * xa).sum(-1) + (xb * xb).sum(-1)) / x.shape[-1] + eps)[..., None]
    wf = w.float()
    na = (wf[:half] * (xa * r)).to(x.dtype).float()
    nb = (wf[half:] * (xb * r)).to(x.dtype).float()
    if f is None:
        return torch.cat((na, nb), -1).to(x.dtype)
    ft = f[:, None]
    oa = (ft[..., 0, 0] * na + ft[..., 0, 1] * nb).to(x.dtype)
    ob = (ft[..., 1, 0] * na + ft[..., 1, 1] * nb).to(x.dtype)
    return torch.cat((oa, ob), -1)


def _close(got, want, dtype, frac=0.99):
    g, w = np32(got), np32(want)
    d = np.abs(g - w)
    assert (d == 0).mean() >= frac, (d == 0).mean()
    bound = ULP[dtype] * (np.abs(w) + 2.0 * np.abs(w).max(-1, keepdims=True)) + 1e-30
    assert np.all(d <= bound), float((d / bound).max())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("B,L,H,D", [(1, 600, 24, 128), (2, 77, 3, 64), (1, 33, 5, 32), (1, 40, 2, 256)])
def test_flux_form_matches_eager_and_oracle(gpu, dtype, B, L, H, D):
    g = torch.Generator(device=gpu).manual_seed(B * L + D)
    q = (torch.randn(B, L, H, D, device=gpu, generator=g) * 2).to(dtype)
    k = (torch.randn(B, L, H, D, device=gpu, generator=g) * 0.5).to(dtype)
    qs = torch.rand(D, device=gpu, generator=g).add(0.5).to(dtype)
    ks = torch.rand(D, device=gpu, generator=g).add(0.5).to(dtype)
    pe = _table(L, D // 2, gpu)
    oq, ok, ov = QK.flux_qk_norm_rope(q, k, qs, ks, pe)
    assert ov is None and oq.shape == q.shape and oq.dtype == dtype
    _close(oq, _eager_flux(q, qs, pe), dtype)
    _close(ok, _eager_flux(k, ks, pe), dtype)
    want = OGL.qk_norm_rope(np32(q), np32(qs), np32(pe[0, 0]), 1e-6, DT[dtype])
    _close(oq, torch.from_numpy(want), dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("D", [128, 32, 64, 256])   # each lane count's partner exchange
def test_anima_form_matches_eager_and_oracle(gpu, dtype, D):
    B, S, H = 2, 300, 16
    g = torch.Generator(device=gpu).manual_seed(11)
    x = torch.randn(B, S, H * D, device=gpu, generator=g).to(dtype)
    w = torch.rand(D, device=gpu, generator=g).add(0.5).to(dtype)
    f = _table(S, D // 2, gpu, seed=3)[0, 0]
    assert QK.qk_ok(x, H, D)
    out = QK.qk_norm_rope(x, w, 1e-5, H, D, f)
    assert out.shape == (B, S, H, D)
    want = _eager_anima(x.view(B, S, H, D), w, f, 1e-5)
    _close(out, want, dtype)
    ref = OGL.qk_norm_rope(np32(x).reshape(B, S, H, D), np32(w), np32(f), 1e-5, DT[dtype], True, True)
    _close(out, torch.from_numpy(ref), dtype)
    # no table: the norm alone
    _close(QK.qk_norm_rope(x, w, 1e-5, H, D), _eager_anima(x.view(B, S, H, D), w, None, 1e-5), dtype)


def test_exact_when_the_sum_of_squares_is_exact(gpu):
    """Small-integer rows: every order of the float32 sum gives the same mean,
    so the kernel equals the eager ops bit for bit (both take rsqrt of the
    same float; the hardware rsqrt agrees on these rows)."""
    g = torch.Generator(device=gpu).manual_seed(5)
    q = torch.randint(-8, 9, (1, 256, 8, 128), device=gpu, generator=g).to(torch.bfloat16)
    s = torch.rand(128, device=gpu, generator=g).add(0.5).to(torch.bfloat16)
    pe = _table(256, 64, gpu, seed=4)
    oq, _, _ = QK.flux_qk_norm_rope(q, q, s, s, pe)
    want = _eager_flux(q, s, pe)
    assert torch.equal(oq, want), (oq != want).float().mean().item()


def test_strided_views_v_copy_and_gathered_outputs(gpu):
    """FLUX double block: txt and img q/k/v come as strided views of two qkv
    projections and land in one (B, Ltxt + Limg, H, D) buffer each."""
    H, D, Lt, Li = 6, 128, 40, 200
    g = torch.Generator(device=gpu).manual_seed(6)
    tqkv = torch.randn(1, Lt, 3 * H * D, device=gpu, generator=g).to(torch.bfloat16).view(1, Lt, 3, H, D)
    iqkv = torch.randn(1, Li, 3 * H * D, device=gpu, generator=g).to(torch.bfloat16).view(1, Li, 3, H, D)
    ts, ts2, is_, is2 = (torch.rand(D, device=gpu, generator=g).add(0.5).to(torch.bfloat16) for _ in range(4))
    pe = _table(Lt + Li, D // 2, gpu, seed=5)
    qb, kb, vb = (torch.empty(1, Lt + Li, H, D, device=gpu, dtype=torch.bfloat16) for _ in range(3))
    QK.flux_qk_norm_rope(tqkv[:, :, 0], tqkv[:, :, 1], ts, ts2, pe[:, :, :Lt], v=tqkv[:, :, 2],
                         out=(qb[:, :Lt], kb[:, :Lt], vb[:, :Lt]))
    QK.flux_qk_norm_rope(iqkv[:, :, 0], iqkv[:, :, 1], is_, is2, pe[:, :, Lt:], v=iqkv[:, :, 2],
                         out=(qb[:, Lt:], kb[:, Lt:], vb[:, Lt:]))
    assert torch.equal(vb, torch.cat((tqkv[:, :, 2], iqkv[:, :, 2]), 1))
    _close(qb, torch.cat((_eager_flux(tqkv[:, :, 0], ts, pe[:, :, :Lt]),
                          _eager_flux(iqkv[:, :, 0], is_, pe[:, :, Lt:])), 1), torch.bfloat16)
    _close(kb, torch.cat((_eager_flux(tqkv[:, :, 1], ts2, pe[:, :, :Lt]),
                          _eager_flux(iqkv[:, :, 1], is2, pe[:, :, Lt:])), 1), torch.bfloat16)


def test_float32_weights_batch_table_and_in_place(gpu):
    g = torch.Generator(device=gpu).manual_seed(7)
    B, L, H, D = 2, 64, 4, 64
    x = torch.randn(B, L, H, D, device=gpu, generator=g).to(torch.float16)
    w = torch.rand(D, device=gpu, generator=g).add(0.5)                  # float32 weight
    f = torch.cat([_table(L, D // 2, gpu, seed=s) for s in (8, 9)], 0)   # one table per sample
    out, _, _ = QK.norm_rope(x, w, 1e-6, f[:, 0])
    want = torch.stack([_eager_flux(x[b:b + 1], w, f[b:b + 1])[0] for b in range(B)])
    _close(out, want, torch.float16)
    y = x.clone()
    QK.norm_rope(y, w, 1e-6, f[:, 0], out_q=y)                          # in place
    assert torch.equal(y, out)


def test_rejects_what_it_cannot_take(gpu):
    x = torch.randn(1, 8, 2, 96, device=gpu, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="D must be"):
        QK.norm_rope(x, torch.ones(96, device=gpu, dtype=torch.bfloat16), 1e-6)
    x = torch.randn(1, 8, 2, 64, device=gpu, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="freqs"):
        QK.norm_rope(x, torch.ones(64, device=gpu, dtype=torch.bfloat16), 1e-6, _table(7, 32, gpu))
    with pytest.raises(RuntimeError, match="aligned"):
        QK.norm_rope(torch.randn(1, 8, 2, 68, device=gpu, dtype=torch.bfloat16)[..., :64],
                     torch.ones(64, device=gpu, dtype=torch.bfloat16), 1e-6)
