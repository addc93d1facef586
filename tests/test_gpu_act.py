"""dc_act_quantize_rows on the GPU: the fused MLP middle (GELU, then ConvRot
and per-row int8 quantization, reference ``_int8.py:326-358, 433-443``) and
FLUX's single-block ``cat(attention, gelu_tanh(mlp))`` input (``flux_dit.py:335``).

Everything after the GELU is exact; the GELU's erf / tanh is a float32 library
function, so the checks allow the rare element where the device's float32
value rounds to the other neighbouring 16-bit value (parity within tolerance,
stated in each test)."""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

from diffucore_amd import _int8
from oracle import quant as OQ
from tests._util import DT, cosine, np32, rel_l2

pytestmark = pytest.mark.gpu

APPROX = {"gelu": "none", "gelu_tanh": "tanh"}


def _agree(q, s, q_ref, s_ref, code_frac=0.999):
    """A GELU value one 16-bit ulp off (the library erf / tanh differing in the
    last float32 bit next to a rounding boundary) moves its rotated group by
    under one code step and the row maximum by at most that ulp: every scale
    within 2^-8 relative, every code within 1, and at least ``code_frac`` of
    the codes equal."""
    q = q.cpu().numpy().astype(np.int32) if hasattr(q, "cpu") else np.asarray(q, np.int32)
    s = s.cpu().numpy() if hasattr(s, "cpu") else np.asarray(s, np.float32)
    q_ref, s_ref = np.asarray(q_ref, np.int32), np.asarray(s_ref, np.float32)
    assert np.all(np.abs(s - s_ref) <= s_ref * 2 ** -8)
    d = np.abs(q - q_ref)
    assert d.max(initial=0) <= 1
    assert (d == 0).mean() >= code_frac, (d == 0).mean()


@pytest.mark.parametrize("act", ["gelu", "gelu_tanh"])
@pytest.mark.parametrize("M,K,group,dtype", [
    (512, 12288, 256, torch.bfloat16),    # FLUX MLP middle (text rows)
    (300, 3072, 256, torch.float16),
    (129, 2048, 0, torch.bfloat16),
    (64, 8192, 256, torch.float16),
    (97, 9216, 256, torch.bfloat16),      # 36 groups: one row per 320-thread workgroup
])
def test_gelu_quantize_matches_unfused(gpu, act, M, K, group, dtype):
    g = torch.Generator().manual_seed(M + K)
    h = (torch.randn(M, K, generator=g) * 2).to(dtype).to(gpu)
    q, s = _int8.act_quantize(h, group, act)
    # the reference's unfused form: GELU on the GPU in float32, rounded to the dtype, then quantized
    q_u, s_u = _int8.quantize_activation(F.gelu(h.float(), approximate=APPROX[act]).to(dtype), group)
    _agree(q, s, q_u.cpu().numpy(), s_u.cpu().numpy())
    # and the oracle's restatement (float64 erf / tanh rounded once to float32)
    q_o, s_o = OQ.act_quantize(np32(h), group, APPROX[act], DT[dtype])
    _agree(q, s, q_o, s_o)


@pytest.mark.parametrize("M,K1,K2,dtype", [(4608, 3072, 12288, torch.bfloat16), (77, 256, 512, torch.float16)])
def test_concat_prefix_and_gelu_tanh(gpu, M, K1, K2, dtype):
    """FLUX single block: linear2's input is cat(attention, gelu_tanh(mlp)),
    the mlp half a column slice of linear1's output (row stride > width)."""
    g = torch.Generator().manual_seed(K1 + K2)
    attn = torch.randn(M, K1, generator=g).to(dtype).to(gpu)
    lin1 = (torch.randn(M, 3 * K1 + K2, generator=g) * 2).to(dtype).to(gpu)
    mlp = lin1[:, 3 * K1:]
    q, s = _int8.act_quantize(mlp, 256, "gelu_tanh", prefix=attn)
    cat = torch.cat((attn, F.gelu(mlp.float(), approximate="tanh").to(dtype)), 1)
    q_u, s_u = _int8.quantize_activation(cat, 256)
    _agree(q, s, q_u.cpu().numpy(), s_u.cpu().numpy())
    # act "none" with a prefix is an exact concatenation
    q0, s0 = _int8.act_quantize(mlp, 256, "none", prefix=attn)
    q0_u, s0_u = _int8.quantize_activation(torch.cat((attn, mlp), 1), 256)
    assert torch.equal(q0, q0_u) and torch.equal(s0, s0_u)


def test_act_quantize_rejects_unaligned_widths(gpu):
    h = torch.randn(4, 300, device=gpu, dtype=torch.bfloat16)
    assert not _int8.act_fusable(h)
    with pytest.raises(RuntimeError, match="multiples of 256"):
        _int8.act_quantize(h, 0, "gelu")
    # gelu_quantize falls back to the unfused ops for such rows
    q, s = _int8.gelu_quantize(h, 0)
    q_u, s_u = _int8.quantize_activation(F.gelu(h.float()).to(h.dtype), 0)
    assert torch.equal(q, q_u) and torch.equal(s, s_u)


@pytest.mark.parametrize("approximate,bias", [("none", False), ("tanh", True)])
def test_int8_mlp_matches_eager(gpu, approximate, bias):
    """int8_mlp (fused middle) against the same two Int8Linear layers run
    eagerly, l2(gelu(l1(x))), and against the float MLP."""
    torch.manual_seed(5)
    d, m = 1024, 4096
    fc1, fc2 = nn.Linear(d, m, bias=bias).to(gpu).bfloat16(), nn.Linear(m, d, bias=bias).to(gpu).bfloat16()
    l1, l2 = _int8.Int8Linear.from_linear(fc1, 256), _int8.Int8Linear.from_linear(fc2, 256)
    x = torch.randn(2, 333, d, device=gpu, dtype=torch.bfloat16)
    y = _int8.int8_mlp(x, l1, l2, approximate)
    y_eager = l2(F.gelu(l1(x), approximate=approximate))
    assert y.shape == y_eager.shape and y.dtype == torch.bfloat16
    assert rel_l2(np32(y), np32(y_eager)) < 2e-3
    y_float = fc2(F.gelu(fc1(x).float(), approximate=approximate).bfloat16())
    assert rel_l2(np32(y), np32(y_float)) < 3e-2 and cosine(np32(y), np32(y_float)) > 0.999


@pytest.mark.parametrize("M,K,rpm,group,xdt,mdt", [
    (4096, 3072, 4096, 256, torch.bfloat16, torch.bfloat16),   # FLUX image stream, one sample
    (2 * 512, 3072, 512, 256, torch.bfloat16, torch.bfloat16), # two samples of text rows
    (333, 2048, 111, 0, torch.float32, torch.float16),          # fp32 residual stream (reference ln_mod)
    (65, 11264, 65, 256, torch.bfloat16, torch.bfloat16),       # 44 groups: one row per 384-thread workgroup
])
def test_ln_mod_quantize_matches_unfused(gpu, M, K, rpm, group, xdt, mdt):
    """One pass of LayerNorm-modulate + quantize against the reference's
    ln_mod formulation computed with torch float32 ops on the GPU, rounded to
    the modulation dtype and then quantized (and against the oracle): the row
    statistics are sums in different orders, so parity is within the last
    bits (the _agree bound)."""
    g = torch.Generator().manual_seed(M + K)
    x = (torch.randn(M, K, generator=g) * 3 + 0.5).to(xdt).to(gpu)
    n = M // rpm
    sc1 = (1 + torch.randn(n, K, generator=g) * 0.1).to(mdt).to(gpu)
    sh = (torch.randn(n, K, generator=g) * 0.1).to(mdt).to(gpu)
    q, s = _int8.ln_mod_quantize(x, sc1, sh, rpm, 1e-6, group)
    xf = x.float()
    mean = xf.mean(1, keepdim=True)
    xc = xf - mean
    y = xc * torch.rsqrt((xc * xc).mean(1, keepdim=True) + 1e-6)
    idx = torch.arange(M, device=gpu) // rpm
    y = (y * sc1.float()[idx] + sh.float()[idx]).to(mdt)
    q_u, s_u = _int8.quantize_activation(y, group)
    _agree(q, s, q_u.cpu().numpy(), s_u.cpu().numpy())
    q_o, s_o = OQ.ln_mod_quantize(np32(x), np32(sc1), np32(sh), rpm, 1e-6, group, DT[mdt])
    _agree(q, s, q_o, s_o)


def test_ln_mod_quantize_strided_modulation(gpu):
    """Modulation rows as FLUX's Modulation produces them: chunks of one
    [B, 6K] projection (row stride 6K)."""
    B, L, K = 2, 256, 3072
    g = torch.Generator().manual_seed(9)
    x = torch.randn(B * L, K, generator=g).to(torch.bfloat16).to(gpu)
    mod = (torch.randn(B, 6 * K, generator=g) * 0.1).to(torch.bfloat16).to(gpu)
    shift, scale = mod[:, :K], mod[:, K:2 * K]
    sc1 = (1 + scale).contiguous()
    q, s = _int8.ln_mod_quantize(x, sc1, shift.contiguous(), L, 1e-6, 256)
    # the strided shift view gives the same result as its contiguous copy
    sc1_s = torch.empty(B, 6 * K, device=gpu, dtype=torch.bfloat16)[:, :K]
    sc1_s.copy_(sc1)
    q2, s2 = _int8.ln_mod_quantize(x, sc1_s, shift, L, 1e-6, 256)
    assert torch.equal(q, q2) and torch.equal(s, s2)


# ---------------------------------------------------------------- GEGLU (SD1.5 / SDXL UNet feed-forward)

@pytest.mark.parametrize("M,N,group,dtype", [
    (8192, 5120, 256, torch.float16),     # SDXL 1024^2 level-1 blocks: GEGLU proj 640 -> 2 x 5120
    (2048, 10240, 256, torch.float16),    # SDXL level-2 blocks: GEGLU proj 1280 -> 2 x 10240
    (300, 1280, 0, torch.bfloat16),
])
def test_geglu_quantize_matches_unfused(gpu, M, N, group, dtype):
    """The fused GEGLU middle (value * gelu(gate), each op rounded to the
    dtype, then ConvRot + int8) against the reference's unfused torch ops on
    the GPU and against the oracle, to the _agree bound."""
    g = torch.Generator().manual_seed(M + N)
    h = (torch.randn(M, 2 * N, generator=g) * 2).to(dtype).to(gpu)
    q, s = _int8.act_quantize(h, group, "geglu")
    assert q.shape == (M, N)
    a, gate = h.chunk(2, dim=-1)
    q_u, s_u = _int8.quantize_activation(a * F.gelu(gate), group)
    _agree(q, s, q_u.cpu().numpy(), s_u.cpu().numpy())
    q_o, s_o = OQ.act_quantize(np32(h), group, "geglu", DT[dtype])
    _agree(q, s, q_o, s_o)
    # geglu_quantize takes the fused path for these rows and gives the same
    q2, s2 = _int8.geglu_quantize(h, group)
    assert torch.equal(q, q2) and torch.equal(s, s2)


def test_geglu_strided_projection_rows(gpu):
    """The projection output as a column slice of a wider buffer (row stride >
    2N), and a prefix: same codes as the contiguous copy."""
    g = torch.Generator().manual_seed(31)
    buf = torch.randn(129, 3 * 1024, generator=g).half().to(gpu)
    h = buf[:, 512:512 + 2 * 1024]
    pre = torch.randn(129, 256, generator=g).half().to(gpu)
    q, s = _int8.act_quantize(h, 256, "geglu", prefix=pre)
    q2, s2 = _int8.act_quantize(h.contiguous(), 256, "geglu", prefix=pre)
    assert torch.equal(q, q2) and torch.equal(s, s2)
    a, gate = h.chunk(2, dim=-1)
    q_u, s_u = _int8.quantize_activation(torch.cat((pre, a * F.gelu(gate)), 1), 256)
    _agree(q, s, q_u.cpu().numpy(), s_u.cpu().numpy())


@pytest.mark.parametrize("act", ["gelu", "gelu_tanh"])
def test_gelu_negative_tail(gpu, act):
    """Rows that lie wholly in the negative tail (x in [-8, -3]), where the
    reference's forms 0.5 x (1 + erf) / 0.5 x (1 + tanh) cancel: the kernel's
    cancellation-free forms keep a small relative error, so its codes follow
    the float64 GELU (rounded to the dtype, then quantized) within one step on
    every element and exactly on at least 99% of them."""
    from scipy.special import erfc
    g = torch.Generator().manual_seed(41)
    x = (torch.rand(64, 1024, generator=g) * -5 - 3).half().to(gpu)
    q, s = _int8.act_quantize(x, 256, act)
    xd = np32(x).astype(np.float64)
    if act == "gelu":
        y = 0.5 * xd * erfc(-xd / np.sqrt(2))          # 1 + erf(z) = erfc(-z), no cancellation
    else:
        u = np.sqrt(2 / np.pi) * (xd + 0.044715 * xd ** 3)
        y = xd / (1 + np.exp(-2 * u))
    q_ref, s_ref = OQ.quantize_activation(y.astype(np.float32).astype(np.float16).astype(np.float32), 256)
    qn, sn = q.cpu().numpy().astype(np.int32), s.cpu().numpy()
    assert np.all(np.abs(sn - s_ref) <= s_ref * 2 ** -8)
    d = np.abs(qn - q_ref.astype(np.int32))
    assert d.max() <= 1 and (d == 0).mean() >= 0.99, (d == 0).mean()


@pytest.mark.parametrize("dim,bias", [(640, True), (1280, False)])
def test_int8_geglu_ff_matches_eager(gpu, dim, bias):
    """int8_geglu_ff (fused middle) against the same two Int8Linear layers run
    eagerly, out(x * gelu(gate)), and against the float feed-forward."""
    torch.manual_seed(dim)
    inner = 4 * dim
    proj = nn.Linear(dim, 2 * inner, bias=bias).to(gpu).half()
    out = nn.Linear(inner, dim, bias=bias).to(gpu).half()
    # ConvRot group 256 where the input width allows it, else none (SDXL's 640-wide blocks)
    lp = _int8.Int8Linear.from_linear(proj, 256 if dim % 256 == 0 else 0)
    lo = _int8.Int8Linear.from_linear(out, 256)
    x = torch.randn(2, 1024, dim, device=gpu, dtype=torch.float16)
    y = _int8.int8_geglu_ff(x, lp, lo)
    a, gate = lp(x).chunk(2, dim=-1)
    y_eager = lo(a * F.gelu(gate))
    assert y.shape == y_eager.shape == (2, 1024, dim) and y.dtype == torch.float16
    assert rel_l2(np32(y), np32(y_eager)) < 2e-3
    af, gf = proj(x).chunk(2, dim=-1)
    y_float = out(af * F.gelu(gf))
    assert rel_l2(np32(y), np32(y_float)) < 3e-2 and cosine(np32(y), np32(y_float)) > 0.999
