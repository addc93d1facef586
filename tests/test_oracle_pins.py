"""Pins of the CPU oracle (no GPU): each oracle function is checked against an
independent computation - exact rational arithmetic, float64 with a single
final rounding, explicit matrices, brute-force loops over the reference's
literal loop structure, textbook special cases - and a planted mistake shows
the check would catch the plausible bug. The reference ships no numeric golden
vectors for this path (its only bit-exact contract is
``tests/test_int8.py:174-183``), so these pins are the oracle's anchor.
"""

from __future__ import annotations

from fractions import Fraction

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import attn as OA
from oracle import cpu_path as OC
from oracle import fp as OF
from oracle import gemm as OG
from oracle import quant as OQ

RNG = np.random.default_rng(1234)


def _f32(x):
    return np.asarray(x, np.float32)


def _round_exact_to_f32(q: Fraction) -> np.float32:
    """Nearest float32 to an exact rational (ties to even), by comparing the
    two float32 neighbours exactly."""
    f = np.float32(float(q))           # within one ulp of the answer
    cands = {f, np.nextafter(f, np.float32(np.inf)), np.nextafter(f, np.float32(-np.inf))}
    best = min(cands, key=lambda c: (abs(Fraction(float(c)) - q), int(np.array(c).view(np.int32)) & 1))
    return np.float32(best)


# ---------------------------------------------------------------- float helpers

def test_fma_f32_matches_exact_rational_rounding():
    a = _f32(RNG.standard_normal(400) * 3)
    b = _f32(RNG.standard_normal(400) / 7)
    c = _f32(RNG.standard_normal(400))
    # hard cases: c ~= -a*b so the result is dominated by the product's low bits
    c[:100] = -(a[:100].astype(np.float64) * b[:100]).astype(np.float32)
    got = OF.fma_f32(a, b, c)
    for i in range(400):
        exact = Fraction(float(a[i])) * Fraction(float(b[i])) + Fraction(float(c[i]))
        assert got[i] == _round_exact_to_f32(exact), i
    # a separate multiply and add (two roundings) differs somewhere on these inputs
    two = (a * b).astype(np.float32) + c
    assert (two != got).any()


def test_bf16_rounding_ties_to_even_and_specials():
    x = np.array([1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, 1.0 + 2 ** -8 + 2 ** -20, -2.5, 0.0, -0.0, np.inf, 3e38],
                 np.float32)
    got = OF.round_bf16(x)
    assert got[0] == 1.0                       # tie -> even mantissa
    assert got[1] == 1.0 + 4 * 2 ** -8         # tie -> even (up)
    assert got[2] == 1.0 + 2 * 2 ** -8         # above the tie -> up
    assert got[3] == -2.5 and got[4] == 0 and np.isinf(got[6])
    assert np.isnan(OF.round_bf16(np.array([np.nan], np.float32)))[0]
    # agrees with torch's bfloat16 conversion on random values
    r = _f32(RNG.standard_normal(10000) * 100)
    assert np.array_equal(OF.round_bf16(r), torch.tensor(r).bfloat16().float().numpy())


# ---------------------------------------------------------------- quantizer

def test_quantize_rows_against_float64_and_properties():
    x = _f32(RNG.standard_normal((64, 320)))
    x[:, RNG.permutation(320)[:2]] *= 20        # outlier channels
    x[5] = 0
    q, s = OQ.quantize_rows(x)
    amax = np.abs(x.astype(np.float64)).max(1)
    s_ref = np.maximum((amax / 127.0).astype(np.float32), np.float32(1e-30))   # one rounding of the exact quotient
    assert np.array_equal(s, s_ref)
    quot = (x.astype(np.float64) / s_ref.astype(np.float64)[:, None]).astype(np.float32)   # correctly rounded x/s
    assert np.array_equal(q, np.clip(np.rint(quot), -128, 127).astype(np.int8))
    assert np.abs(q.astype(np.int32)).max() <= 127
    nz = amax > 0
    assert (np.abs(q[nz].astype(np.int32)).max(1) == 127).all()
    assert s[5] == np.float32(1e-30) and not q[5].any()


def test_quantize_rows_ties_round_to_even():
    # x / scale lands exactly on k + 0.5 for these values: scale = 1 (amax 127)
    x = _f32([[127.0, 2.5, 3.5, -2.5, -0.5, 0.5, 1.5, 0.0]])
    q, s = OQ.quantize_rows(x)
    assert s[0] == 1.0
    assert q.tolist() == [[127, 2, 4, -2, 0, 0, 2, 0]]
    # planted mistake: round-half-away-from-zero would give 3, 4, -3, -1, 1, 2
    away = np.sign(x) * np.floor(np.abs(x) + 0.5)
    assert not np.array_equal(away.astype(np.int8), q)


def test_torch_cpu_path_and_numpy_oracle_agree():
    """Two independent statements of ``_quantize_rows`` (torch ops as the
    reference writes them, numpy ops in the oracle) are bit-identical."""
    x = torch.randn(200, 768) * 3
    q_t, s_t = OC.quantize_rows(x)
    q_n, s_n = OQ.quantize_rows(x.numpy())
    assert np.array_equal(q_t.numpy(), q_n) and np.array_equal(s_t.numpy(), s_n)


def test_hadamard_symmetric_self_inverse():
    h = OQ.hadamard(256)
    assert np.array_equal(h, h.T)
    np.testing.assert_allclose(h.astype(np.float64) @ h, np.eye(256), atol=1e-6)
    assert np.array_equal(OQ.hadamard(256), OC.hadamard(256).numpy())


def test_butterfly_equals_explicit_hadamard():
    # exact on basis vectors: e_i @ H is row i of H (every entry +-1/16)
    e = np.eye(256, dtype=np.float32)
    assert np.array_equal(OQ.rotate_butterfly(e, 256), OQ.hadamard(256))
    # close to the float64 product on random rows, and linear
    x = _f32(RNG.standard_normal((16, 512)))
    ref = (x.astype(np.float64).reshape(16, 2, 256) @ OQ.hadamard(256).astype(np.float64)).reshape(16, 512)
    np.testing.assert_allclose(OQ.rotate_butterfly(x, 256), ref, rtol=0, atol=2e-6)
    # planted mistake: H4 applied with the wrong sign pattern (S - 2 x[j] instead of S - 2 x[3-j])
    y = x.reshape(16, 2, 4, 64)
    s = (y[:, :, 0] + y[:, :, 1]) + (y[:, :, 2] + y[:, :, 3])
    wrong = np.stack([s - 2 * y[:, :, j] for j in range(4)], 2).reshape(16, 512)
    right_first_axis = np.stack([s - 2 * y[:, :, 3 - j] for j in range(4)], 2).reshape(16, 512)
    assert not np.allclose(wrong, right_first_axis)


def test_convrot_codes_match_matmul_form_closely():
    x = _f32(RNG.standard_normal((256, 3072)))
    q_b, s_b = OQ.quantize_activation(x, 256)
    q_m, s_m = OQ.quantize_rows(OQ.rotate_matmul(x, 256))
    d = np.abs(q_b.astype(np.int32) - q_m.astype(np.int32))
    assert d.max() <= 1 and (d != 0).mean() < 1e-2
    np.testing.assert_allclose(s_b, s_m, rtol=1e-5)


# ---------------------------------------------------------------- GEMM epilogue

def test_int_mm_exact_against_python_ints():
    q = RNG.integers(-127, 128, (7, 48), dtype=np.int8)
    w = RNG.integers(-127, 128, (5, 48), dtype=np.int8)
    ref = [[sum(int(a) * int(b) for a, b in zip(q[i], w[j])) for j in range(5)] for i in range(7)]
    assert OG.int_mm(q, w).tolist() == ref
    big = np.full((1, 4096), 127, np.int8)
    assert OG.int_mm(big, big)[0, 0] == 4096 * 127 * 127


def test_rescale_closed_forms():
    # int32 -> float32 is round-to-nearest-even above 2^24
    acc = np.array([[2 ** 24 + 1, 2 ** 24 + 3, -(2 ** 24 + 1), 7]], np.int32)
    y = OG.rescale(acc, _f32([1.0]), _f32([1.0, 1.0, 1.0, 0.25]), None, "f32")
    assert y.tolist() == [[2 ** 24, 2 ** 24 + 4, -(2 ** 24), 1.75]]
    # the fp16 tie the GPU epilogue once got wrong: float32 -0.2623291 is the
    # midpoint of two fp16 values and rounds to the even one
    acc = np.array([[1]], np.int32)
    yy = OG.rescale(acc, _f32([-0.2623291015625]), _f32([1.0]), None, "f16")
    assert np.float16(yy[0, 0]).view(np.uint16) == 0xB432
    # bias double rounding: round(round(y) + round(b)) differs from round(y + b)
    acc = np.array([[1]], np.int32)
    sx, sw = _f32([1.0 + 3 * 2 ** -10]), _f32([1.0])
    b = _f32([3 * 2 ** -10])
    two = OG.rescale(acc, sx, sw, b, "bf16")[0, 0]
    single = OF.round_bf16(np.float32(1.0 + 6 * 2 ** -10))
    assert two == 1.0 and single == np.float32(1.0 + 2 ** -7)


def test_rescale_matches_torch_reference_statement():
    acc = torch.randint(-2 ** 28, 2 ** 28, (33, 40), dtype=torch.int32)
    sx, sw = torch.rand(33) * 1e-3, torch.rand(40) * 1e-3
    bias = torch.randn(40).bfloat16()
    for dt, name in ((torch.float16, "f16"), (torch.bfloat16, "bf16"), (torch.float32, "f32")):
        ref = OC.rescale(acc, sx, sw, bias, dt).float().numpy()
        got = OG.rescale(acc.numpy(), sx.numpy(), sw.numpy(), bias.float().numpy(), name)
        assert np.array_equal(got, ref), name


# ---------------------------------------------------------------- attention prep

def _colsum_literal(k):
    """The reference's loops (int8_attn_sm80.cu:100-142), one float32 add at a time."""
    k = _f32(k)
    B, L, H, D = k.shape
    nwin = -(-L // 128)
    out = np.zeros((B, H, D), np.float32)
    for b in range(B):
        for h in range(H):
            for d in range(D):
                total = np.float32(0)
                for w in range(nwin):
                    parts = []
                    for rg in range(16):
                        a = np.float32(0)
                        for r in range(w * 128 + rg, min(L, w * 128 + 128), 16):
                            a = np.float32(a + k[b, r, h, d])
                        parts.append(a)
                    sk = np.float32(0)
                    for a in parts:
                        sk = np.float32(sk + a)
                    total = np.float32(total + sk)
                out[b, h, d] = total
    return out


def test_k_colsum_matches_literal_loop_order():
    k = _f32(torch.randn(1, 300, 2, 8).half().float().numpy() + 0.5)
    assert np.array_equal(OA.k_colsum(k), _colsum_literal(k))
    np.testing.assert_allclose(OA.k_colsum(k), k.astype(np.float64).sum(1), rtol=1e-5)


def test_k_quantize_properties_and_fma_choice():
    k = torch.randn(2, 150, 3, 40).bfloat16().float().numpy() + 0.7
    ksum = OA.k_colsum(k)
    ki, ks = OA.k_quantize(k, ksum)
    assert ki.shape == (2, 3, 192, 40) and ks.shape == (2, 3, 3)
    assert not ki[:, :, 150:].any()
    blocks = np.abs(ki.astype(np.int32)).reshape(2, 3, 3, -1).max(-1)
    assert (blocks == 127).all() and np.abs(ki.astype(np.int32)).max() <= 127
    val = OA.k_smooth(k, ksum)
    amax = np.abs(np.concatenate([val, np.zeros((2, 3, 42, 40), np.float32)], 2).reshape(2, 3, 3, -1)).max(-1)
    assert np.array_equal(ks, (amax / np.float32(127)).astype(np.float32))
    # the smoothing is one rounding of k - ksum/L's exact product form
    inv_l = np.float32(1) / np.float32(150)
    exact = np.array([[_round_exact_to_f32(Fraction(float(k[0, r, 0, d])) - Fraction(float(ksum[0, 0, d])) *
                                           Fraction(float(inv_l))) for d in range(40)] for r in range(4)])
    assert np.array_equal(val[0, 0, :4], exact)
    # against the unfused form the codes differ in at most a few places, by one
    unfused = (k.transpose(0, 2, 1, 3) - (ksum[:, :, None, :] * inv_l).astype(np.float32)).astype(np.float32)
    assert np.abs(unfused - val).max() <= 2 * np.spacing(np.abs(val).max())


def test_q_quantize_properties():
    q = torch.randn(1, 100, 2, 64).bfloat16().float().numpy()
    q[0, 7, 1] = 0
    q8, qs = OA.q_quantize(q)
    assert (np.abs(q8.astype(np.int32)).max(-1)[qs > 0] == 127).all()
    assert qs[0, 1, 7] == 0 and not q8[0, 1, 7].any()


# ---------------------------------------------------------------- attention quantizer codes, exact

def _rne_int(x: Fraction) -> int:
    """Nearest integer to an exact rational, ties to even."""
    f = x.numerator // x.denominator
    rem = x - f
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and f % 2):
        f += 1
    return f


def _exact_attn_codes(rows) -> tuple[np.ndarray, np.ndarray]:
    """The reference's attention quantizer (int8_attn_sm80.cu:75-85, 369-378)
    in exact rational arithmetic: per row, inv = RN(127 / amax) (a float32
    division), code = rint_even(RN(x * inv)) (a float32 multiply, then
    __float2int_rn; no clamp), scale = RN(amax / 127); a zero row has codes 0
    and scale 0."""
    rows = _f32(rows)
    codes = np.zeros(rows.shape, np.int64)
    scales = np.zeros(rows.shape[0], np.float32)
    for i, row in enumerate(rows):
        amax = max(abs(Fraction(float(x))) for x in row)
        if amax == 0:
            continue
        inv = Fraction(float(_round_exact_to_f32(Fraction(127) / amax)))
        scales[i] = _round_exact_to_f32(amax / 127)
        for j, x in enumerate(row):
            codes[i, j] = _rne_int(Fraction(float(_round_exact_to_f32(Fraction(float(x)) * inv))))
    return codes, scales


def _boundary_rows(rng, n: int, d: int, dtype=torch.bfloat16) -> np.ndarray:
    """Rows whose codes separate the plausible roundings of the quantizer:
    each holds its absmax a and a/2 (the code-63/64 boundary, where x * RN(127/a)
    and x / RN(a/127) round differently for some a), +-a/2 and half-integer
    multiples of a/127 (exact ties when a = 127), and random fill."""
    rows = torch.randn(n, d, generator=torch.Generator().manual_seed(int(rng.integers(1 << 30)))).to(dtype).float()
    amax = rows.abs().amax(1)
    rows[:, 0] = amax
    rows[:, 1] = amax / 2
    rows[:, 2] = -amax / 2
    rows[: n // 4, 0] = 127.0             # a = 127: inv = 1 exactly, so x = k + 1/2 is a tie
    for j, t in enumerate((0.5, 1.5, 2.5, -2.5, 126.5, -3.5)):
        rows[: n // 4, 3 + j] = t
    rows[n - 1] = 0.0                     # zero row
    return rows.to(dtype).float().numpy()


def _attn_amaxes_with_boundary_cases(dtype=torch.bfloat16) -> list:
    """absmax values a (representable in ``dtype``) for which the divide form
    rint(RN(a/2 / RN(a/127))) differs from the multiply form rint(RN(a/2 * RN(127/a)))."""
    b = np.arange(0x3c00, 0x4100, dtype=np.uint32) << 16        # bf16 values in [2^-7, 8)
    a = b.view(np.float32)
    a = torch.tensor(a).to(dtype).float().numpy()
    half = (a / np.float32(2)).astype(np.float32)
    mul = np.rint((half * (np.float32(127) / a)).astype(np.float32))
    div = np.rint((half / (a / np.float32(127))).astype(np.float32))
    return sorted(set(a[mul != div].tolist()))


def _q_codes_pinned(q_quantize) -> bool:
    rows = _boundary_rows(np.random.default_rng(5), 48, 64)
    amaxes = _attn_amaxes_with_boundary_cases()
    for i, a in enumerate(amaxes[:16]):   # rows whose a/2 sits on a multiply/divide disagreement
        rows[12 + i, :] = np.clip(rows[12 + i, :], -a, a)
        rows[12 + i, 0], rows[12 + i, 1], rows[12 + i, 2] = a, a / 2, -a / 2
    exact_codes, exact_scales = _exact_attn_codes(rows)
    q8, qs = q_quantize(rows.reshape(1, 48, 1, 64))
    return (np.array_equal(q8[0, 0].astype(np.int64), exact_codes)
            and np.array_equal(qs[0, 0], exact_scales))


def _k_codes_pinned(k_quantize) -> bool:
    """K blocks of 64 keys whose column sums are exactly zero (key r + 16 is
    the negation of key r inside each group of 32, so every float32 partial sum
    returns to +-0), making the smoothed keys equal the keys; each block's
    codes then follow the exact quantizer over the block's 64 x D values."""
    D, L = 16, 192
    rng = np.random.default_rng(6)
    base = _boundary_rows(rng, L // 2, D)
    amaxes = _attn_amaxes_with_boundary_cases()
    k = np.zeros((L, D), np.float32)
    for g in range(L // 32):
        half = base[16 * (g % 3):16 * (g % 3) + 16].copy()   # g = 4: rows with a = 127 and exact ties
        if g < 3:                          # a block-wide absmax a with a/2 present
            a = amaxes[4 * g]
            half = np.clip(half, -a, a)
            half[0, 0], half[1, 0] = a, a / 2
        k[32 * g:32 * g + 16] = half
        k[32 * g + 16:32 * g + 32] = -half
    assert not OA.k_colsum(k.reshape(1, L, 1, D)).any()
    ki, ks = k_quantize(k.reshape(1, L, 1, D))
    blocks = k.reshape(L // 64, 64 * D)
    exact_codes, exact_scales = _exact_attn_codes(blocks)
    return (np.array_equal(ki[0, 0].reshape(L // 64, 64 * D).astype(np.int64), exact_codes)
            and np.array_equal(ks[0, 0], exact_scales))


def _divide_form_q(q):
    """Planted mistake: the linear quantizer's division instead of the multiply."""
    q = _f32(q).transpose(0, 2, 1, 3)
    amax = np.abs(q).max(axis=-1)
    s = (amax / np.float32(127.0)).astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        q8 = np.where(s[..., None] > 0, np.rint((q / s[..., None]).astype(np.float32)), 0).astype(np.int8)
    return q8, s


def _clamped_floor_q(q):
    """Planted mistake: the linear quantizer whole (scale floored at 1e-30, clamp)."""
    q = _f32(q).transpose(0, 2, 1, 3)
    s = np.maximum(np.abs(q).max(axis=-1) / np.float32(127.0), np.float32(1e-30)).astype(np.float32)
    return np.clip(np.rint((q / s[..., None]).astype(np.float32)), -128, 127).astype(np.int8), s


def _half_away_q(q):
    """Planted mistake: round half away from zero."""
    q = _f32(q).transpose(0, 2, 1, 3)
    amax = np.abs(q).max(axis=-1)
    with np.errstate(divide="ignore"):
        inv = np.where(amax > 0, np.float32(127.0) / amax, np.float32(0.0)).astype(np.float32)
    p = (q * inv[..., None]).astype(np.float32)
    return (np.sign(p) * np.floor(np.abs(p) + 0.5)).astype(np.int8), (amax / np.float32(127.0)).astype(np.float32)


def test_boundary_inputs_separate_multiply_and_divide_forms():
    amaxes = _attn_amaxes_with_boundary_cases()
    assert len(amaxes) >= 16
    codes_mul = _exact_attn_codes(np.array([[a, a / 2] for a in amaxes[:16]], np.float32))[0][:, 1]
    assert set(codes_mul.tolist()) <= {63, 64} and len(set(codes_mul.tolist())) == 2


def test_q_quantize_codes_exact():
    assert _q_codes_pinned(OA.q_quantize)


def test_k_quantize_codes_exact():
    assert _k_codes_pinned(OA.k_quantize)


@pytest.mark.parametrize("mutant", [_divide_form_q, _clamped_floor_q, _half_away_q])
def test_q_code_pin_catches_planted_mistakes(mutant):
    assert not _q_codes_pinned(mutant)


@pytest.mark.parametrize("mutant", [_divide_form_q, _clamped_floor_q, _half_away_q])
def test_k_code_pin_catches_planted_mistakes(mutant, monkeypatch):
    # the same mistakes in the K quantizer's per-block code step
    def k_mut(k, ksum=None):
        k = _f32(k)
        B, L, H, D = k.shape
        ks_ = OA.k_colsum(k) if ksum is None else ksum
        val = OA.k_smooth(k, ks_)                                        # [B, H, L, D]
        nblk = -(-L // 64)
        pad = np.zeros((B, H, nblk * 64, D), np.float32)
        pad[:, :, :L] = val
        blocks = pad.reshape(B * H * nblk, 1, 1, 64 * D).transpose(0, 2, 1, 3)   # rows = blocks
        c, s = mutant(blocks)
        return c.reshape(B, H, nblk * 64, D), s.reshape(B, H, nblk)
    assert not _k_codes_pinned(k_mut)


# ---------------------------------------------------------------- attention output

def _sdpa(q, k, v):
    t = [torch.tensor(x).transpose(1, 2) for x in (q, k, v)]
    return F.scaled_dot_product_attention(*t).transpose(1, 2).numpy()


def test_int8_attention_special_cases():
    k = _f32(RNG.standard_normal((1, 50, 1, 64)))
    v = _f32(RNG.standard_normal((1, 50, 1, 64)))
    # zero queries: uniform weights, output is the mean of V
    out = OA.int8_attention(np.zeros((1, 3, 1, 64), np.float32), k, v, None, "f16", "f32")
    np.testing.assert_allclose(out[0, :, 0], np.broadcast_to(v[0, :, 0].mean(0), (3, 64)), atol=1e-6)
    # a single key: output is that key's value row (rounded to the output type)
    out1 = OA.int8_attention(_f32(RNG.standard_normal((1, 4, 1, 64))), k[:, :1], v[:, :1], None, "bf16", "bf16")
    assert np.array_equal(out1[0, :, 0], np.broadcast_to(OF.round_bf16(v[0, 0, 0]), (4, 64)))


def test_int8_attention_close_to_sdpa_reference_bar():
    q = _f32(RNG.standard_normal((1, 200, 2, 128)))
    k = _f32(RNG.standard_normal((1, 300, 2, 128)) + 0.5)
    v = _f32(RNG.standard_normal((1, 300, 2, 128)))
    o = OA.int8_attention(q, k, v, None, "f16", "f32").astype(np.float64)
    ref = _sdpa(q, k, v).astype(np.float64)
    rel = np.linalg.norm(o - ref) / np.linalg.norm(ref)
    cos = (o.ravel() @ ref.ravel()) / (np.linalg.norm(o) * np.linalg.norm(ref))
    assert rel < 3e-2 and cos > 0.9995


def test_dropping_k_smoothing_fails_the_bar(monkeypatch):
    """Planted mistake: without the K mean subtraction a large key offset eats
    the int8 range and the result misses the reference's bar; with it, the
    same inputs pass."""
    q = _f32(RNG.standard_normal((1, 64, 1, 128)))
    k = _f32(RNG.standard_normal((1, 256, 1, 128)) + 20.0)
    v = _f32(RNG.standard_normal((1, 256, 1, 128)))
    ref = _sdpa(q, k, v).astype(np.float64)

    def rel(o):
        o = o.astype(np.float64)
        return np.linalg.norm(o - ref) / np.linalg.norm(ref)

    assert rel(OA.int8_attention(q, k, v, None, "bf16", "f32")) < 3e-2
    monkeypatch.setattr(OA, "k_colsum", lambda kk: np.zeros((1, 1, 128), np.float32))
    assert rel(OA.int8_attention(q, k, v, None, "bf16", "f32")) > 3e-2


@pytest.mark.parametrize("shift", [0.0, 40.0])
def test_int8_attention_is_shift_invariant_in_keys(shift):
    """Adding a constant vector to every key leaves softmax(q.k) unchanged; the
    mean smoothing removes it before quantization, so the codes are the same."""
    q = _f32(RNG.standard_normal((1, 20, 1, 64)))
    k = _f32(RNG.standard_normal((1, 64, 1, 64)))
    v = _f32(RNG.standard_normal((1, 64, 1, 64)))
    base = OA.int8_attention(q, k, v, None, "bf16", "f32")
    shifted = OA.int8_attention(q, (k + np.float32(shift)).astype(np.float32), v, None, "bf16", "f32")
    np.testing.assert_allclose(shifted, base, atol=3e-2)


# ---------------------------------------------------------------- GELU (fused MLP middle)

def test_gelu_oracle_closed_forms():
    """The erf form is x * Phi(x): Phi(1) = 0.8413447460685429, Phi(-1) =
    0.15865525393145707, 0 at 0, x for large x, 0 for very negative x."""
    from math import erf, sqrt
    x = np.array([0.0, 1.0, -1.0, 2.0, 8.0, -8.0, -30.0], np.float32)
    y = OQ.gelu(x, "none", "f16")
    exact = np.array([v * 0.5 * (1 + erf(v / sqrt(2))) for v in x.astype(np.float64)])
    assert np.array_equal(y, exact.astype(np.float16).astype(np.float32))
    assert y[0] == 0 and y[4] == 8 and y[6] == 0


def test_gelu_oracle_agrees_with_torch_after_rounding():
    """float32 torch GELU (CPU) rounded to bf16 / fp16 equals the oracle's
    except next to a rounding boundary. For x below about -3 both forms
    compute 1 + erf (or 1 + tanh) next to cancellation, so a one-ulp
    difference in the library function moves the (tiny) result by up to
    |x| 2^-24: those elements agree to 1e-5 absolute, far below any row's
    quantization step. The tanh form stays within 3e-3 of the erf form (its
    known approximation error)."""
    g = torch.Generator().manual_seed(3)
    x = (torch.randn(1 << 18, generator=g) * 3).numpy()
    for approx in ("none", "tanh"):
        ref = torch.nn.functional.gelu(torch.from_numpy(x), approximate=approx)
        for dt, tdt in (("bf16", torch.bfloat16), ("f16", torch.float16)):
            o = OQ.gelu(x, approx, dt)
            r = ref.to(tdt).float().numpy()
            big = np.abs(r) >= 1e-2
            assert (o[big] == r[big]).mean() > 0.999, (approx, dt, (o[big] == r[big]).mean())
            assert np.all(np.abs(o - r) <= np.maximum(np.abs(r) * 2 ** -7, 1e-5)), (approx, dt)
    a, b = OQ.gelu(x, "tanh", "f16"), OQ.gelu(x, "none", "f16")
    assert np.all(np.abs(a - b) <= 3e-3 + np.abs(b) * 2 ** -10)   # plus one fp16 ulp of rounding


def test_act_quantize_oracle_is_quantize_of_gelu():
    """The fused form equals quantize_activation(cat(prefix, gelu(x)))."""
    g = np.random.default_rng(4)
    x = g.standard_normal((5, 512)).astype(np.float32)
    pre = g.standard_normal((5, 256)).astype(np.float32)
    q, s = OQ.act_quantize(x, 256, "tanh", "bf16", prefix=pre)
    q2, s2 = OQ.quantize_activation(np.concatenate([pre, OQ.gelu(x, "tanh", "bf16")], 1), 256)
    assert np.array_equal(q, q2) and np.array_equal(s, s2)



def _geglu_torch(x2: np.ndarray, tdt) -> np.ndarray:
    """The reference statement (unet.py:148-155), x * F.gelu(gate) on the two
    chunks in the 16-bit dtype, as torch runs it on the GPU: the GELU in
    float32 rounded to the dtype (torch's opmath for half types; its CPU half
    kernel uses a coarser erf in the tail), then the product rounded once."""
    t = torch.from_numpy(x2).to(tdt)
    a, gate = t.chunk(2, dim=-1)
    return (a * F.gelu(gate.float()).to(tdt)).float().numpy()


@pytest.mark.parametrize("dt,tdt", [("f16", torch.float16), ("bf16", torch.bfloat16)])
def test_geglu_oracle_against_torch_statement(dt, tdt):
    """The GEGLU oracle equals torch's ops except next to a rounding boundary
    of the GELU. For gates below about -2.5 both compute 1 + erf next to
    cancellation, where one ulp of the float32 erf moves the GELU by up to
    |gate| 2^-24 (the same allowance as the GELU pin): those products agree to
    |x| 1e-5."""
    g = torch.Generator().manual_seed(21)
    x2 = (torch.randn(64, 1024, generator=g) * 2).to(tdt).float().numpy()
    o = OQ.geglu(x2, dt)
    r = _geglu_torch(x2, tdt)
    assert o.shape == (64, 512)
    x, gate = x2[:, :512], x2[:, 512:]
    core = gate >= -2.5
    assert (o[core] == r[core]).mean() > 0.999, (o[core] == r[core]).mean()
    assert np.all(np.abs(o - r) <= np.maximum(np.abs(r) * 2 ** -6, np.abs(x) * 1e-5))


def test_geglu_oracle_closed_forms_and_rounding_order():
    """gate = 0 gives 0; gate >= 8 has gelu(gate) = gate, so the result is
    round(x * gate); a planted form that skips the GELU's own rounding (one
    rounding of x * gelu(gate)) differs from torch's two-rounding statement."""
    x = np.array([[1.5, -2.25, 3.0, 0.7, 0.0, 9.0, 12.0, 1.0]], np.float32)
    o = OQ.geglu(x, "f16")
    assert o[0, 0] == 0 and o[0, 1] == np.float32(np.float16(-2.25 * 9.0))
    assert o[0, 2] == np.float32(np.float16(3.0 * 12.0))
    g = torch.Generator().manual_seed(22)
    x2 = (torch.randn(256, 1024, generator=g) * 2).half().float().numpy()
    one_rounding = OF.round_to((x2[:, :512] * OQ.gelu(x2[:, 512:], "none", "f32")).astype(np.float32), "f16")
    r = _geglu_torch(x2, torch.float16)
    assert (one_rounding != r).mean() > 10 * (OQ.geglu(x2, "f16") != r).mean() + 1e-4


def test_act_quantize_oracle_geglu_is_quantize_of_geglu():
    g = np.random.default_rng(23)
    x2 = g.standard_normal((6, 1024)).astype(np.float32)
    pre = g.standard_normal((6, 256)).astype(np.float32)
    q, s = OQ.act_quantize(x2, 256, "geglu", "f16", prefix=pre)
    q2, s2 = OQ.quantize_activation(np.concatenate([pre, OQ.geglu(x2, "f16")], 1), 256)
    assert np.array_equal(q, q2) and np.array_equal(s, s2)


# ---------------------------------------------------------------- QK RMSNorm + rotary (oracle/glue.py)

from oracle import glue as OGL  # noqa: E402


def _rot_table(L, half, seed=0):
    """FLUX-style rotation matrices [[cos, -sin], [sin, cos]] per (position, pair)."""
    ang = np.random.default_rng(seed).uniform(-np.pi, np.pi, (L, half))
    c, s = np.cos(ang), np.sin(ang)
    return np.stack([np.stack([c, -s], -1), np.stack([s, c], -1)], -2).astype(np.float32)


def test_glue_identity_table_leaves_the_norm():
    x = _f32(RNG.standard_normal((2, 5, 3, 64)))
    w = _f32(RNG.uniform(0.5, 1.5, 64))
    eye = np.broadcast_to(np.eye(2, dtype=np.float32), (5, 32, 2, 2))
    for half, wf in ((False, False), (True, True)):
        n = OGL.qk_norm(x, w, 1e-6, "bf16", wf)
        assert np.array_equal(OGL.qk_norm_rope(x, w, eye, 1e-6, "bf16", half, wf), n)


def test_glue_norm_against_float64():
    """w = 1: n is the dtype rounding of x / sqrt(mean(x^2) + eps), up to one
    float32 ulp of rrms before the rounding."""
    x = _f32(RNG.standard_normal((4, 7, 2, 128)) * 3)
    ones = np.ones(128, np.float32)
    for dt, ulp in (("bf16", 2.0 ** -8), ("f16", 2.0 ** -11)):
        n = OGL.qk_norm(x, ones, 1e-6, dt, False)
        exact = x.astype(np.float64) / np.sqrt((x.astype(np.float64) ** 2).mean(-1, keepdims=True) + 1e-6)
        assert np.all(np.abs(n - exact) <= ulp * np.abs(exact) + 1e-30)


def test_glue_rotation_direction_and_pair_layout():
    """(1, 0) turned by +90 degrees is (0, 1) with FLUX's matrix
    [[cos, -sin], [sin, cos]]; a transposed matrix or a swapped pair layout
    gives (0, -1) or moves other channels."""
    D, L = 8, 1
    f = _rot_table(L, D // 2)
    f[0, 1] = [[0.0, -1.0], [1.0, 0.0]]           # pair 1 turns by +90 degrees
    f[0, [0, 2, 3]] = np.eye(2, dtype=np.float32)
    n = np.zeros((1, L, 1, D), np.float32)
    n[..., 2] = 1.0                               # interleaved: pair 1 is channels (2, 3)
    out = OGL.rope(n, f, "f32", half_pairs=False)
    assert np.array_equal(out[0, 0, 0], [0, 0, 0, 1, 0, 0, 0, 0])
    n = np.zeros((1, L, 1, D), np.float32)
    n[..., 1] = 1.0                               # half split: pair 1 is channels (1, 5)
    out = OGL.rope(n, f, "f32", half_pairs=True)
    assert np.array_equal(out[0, 0, 0], [0, 0, 0, 0, 0, 1, 0, 0])
    # pair lengths are kept by rotations (to rounding)
    x = _f32(RNG.standard_normal((1, 3, 2, 16)))
    f = _rot_table(3, 8, seed=1)
    for half in (False, True):
        o = OGL.rope(x, f, "f32", half)
        pa = (lambda t: (t[..., :8], t[..., 8:])) if half else (lambda t: (t[..., 0::2], t[..., 1::2]))
        (xa, xb), (oa, ob) = pa(x), pa(o)
        np.testing.assert_allclose(oa ** 2 + ob ** 2, xa ** 2 + xb ** 2, rtol=1e-5)


def _torch_flux(x, scale, pe, dtype):
    """flux_dit.py's RMSNorm + apply_rope as torch CPU ops (the reference's
    reshape-and-broadcast route, not the oracle's slicing)."""
    xt = torch.from_numpy(x).to(dtype)
    xf = xt.float()
    rr = torch.rsqrt(torch.mean(xf ** 2, dim=-1, keepdim=True) + 1e-6)
    n = (xf * rr).to(dtype) * torch.from_numpy(scale).to(dtype)
    pe_t = torch.from_numpy(pe)[:, None]                       # [L, 1, D/2, 2, 2] over heads
    n_ = n.float().reshape(*n.shape[:-1], -1, 1, 2)
    out = pe_t[..., 0] * n_[..., 0] + pe_t[..., 1] * n_[..., 1]
    return out.reshape(*n.shape).to(dtype).float().numpy()


def _torch_anima(x, w, f, eps, dtype):
    """_fused.py's Anima q/k formulas as torch CPU ops on (x[:D/2], x[D/2:])."""
    xt = torch.from_numpy(x).to(dtype).float()
    half = x.shape[-1] // 2
    xa, xb = xt[..., :half], xt[..., half:]
    r = torch.rsqrt(((xa * xa).sum(-1) + (xb * xb).sum(-1)) / x.shape[-1] + eps)[..., None]
    wt = torch.from_numpy(w).float()
    na = (wt[:half] * (xa * r)).to(dtype).float()
    nb = (wt[half:] * (xb * r)).to(dtype).float()
    ft = torch.from_numpy(f)[:, None]                          # [L, 1, D/2, 2, 2]
    oa = (ft[..., 0, 0] * na + ft[..., 0, 1] * nb).to(dtype)
    ob = (ft[..., 1, 0] * na + ft[..., 1, 1] * nb).to(dtype)
    return torch.cat((oa, ob), -1).float().numpy()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_glue_against_the_reference_formulas_in_torch(dtype):
    """The oracle against torch statements of both reference formulas: equal
    except where the sum order or rsqrt moves rrms by a float32 ulp and a
    rounding flips (then within one dtype ulp of the pair's size)."""
    dt = {torch.bfloat16: "bf16", torch.float16: "f16"}[dtype]
    ulp = {"bf16": 2.0 ** -7, "f16": 2.0 ** -10}[dt]
    x = _f32(RNG.standard_normal((2, 40, 3, 128)) * 2)
    x = OF.round_to(x, dt)
    w = OF.round_to(_f32(RNG.uniform(0.5, 1.5, 128)), dt)
    pe = _rot_table(40, 64, seed=2)
    for got, want in ((OGL.qk_norm_rope(x, w, pe, 1e-6, dt), _torch_flux(x, w, pe, dtype)),
                      (OGL.qk_norm_rope(x, w, pe, 1e-5, dt, True, True), _torch_anima(x, w, pe, 1e-5, dtype))):
        diff = np.abs(got - want)
        assert (diff == 0).mean() > 0.99
        assert np.all(diff <= ulp * (np.abs(want) + 4.0))


# ---------------------------------------------------------------- LayerNorm-modulate + quantize (oracle/quant.py)

def _ln_mod_rows(x, sc1, shift, rows_per_mod, eps, dtype):
    """The modulated rows the oracle quantizes, recovered by quantizing with
    group 0 and a scale of 1 would be lossy; instead restate y in float64."""
    m = np.arange(x.shape[0]) // rows_per_mod
    x64 = x.astype(np.float64)
    mu = x64.mean(1, keepdims=True)
    var = ((x64 - mu) ** 2).mean(1, keepdims=True)
    return (x64 - mu) / np.sqrt(var + eps) * sc1[m].astype(np.float64) + shift[m].astype(np.float64)


def test_ln_mod_oracle_against_float64_layernorm():
    """Codes of the oracle equal the codes of the float64 LayerNorm-modulate
    rounded once to bf16, except where float32 statistics move a value across
    a bf16 rounding boundary (one step at most, on under 1% of elements)."""
    g = np.random.default_rng(7)
    x = (g.standard_normal((12, 512)) * 3 + 1).astype(np.float32)
    sc1 = OF.round_to(g.uniform(0.5, 1.5, (3, 512)).astype(np.float32), "bf16")
    sh = OF.round_to(g.standard_normal((3, 512)).astype(np.float32) * 0.1, "bf16")
    for group in (0, 256):
        q, s = OQ.ln_mod_quantize(x, sc1, sh, 4, 1e-6, group, "bf16")
        y = OF.round_to(_ln_mod_rows(x, sc1, sh, 4, 1e-6, "bf16").astype(np.float32), "bf16")
        q2, s2 = OQ.quantize_activation(y, group)
        assert np.all(np.abs(q.astype(int) - q2) <= 1) and (q == q2).mean() > 0.99
        np.testing.assert_allclose(s, s2, rtol=2 ** -7)


def _torch_ln_mod_codes(x, sc1, sh, rows_per_mod):
    """The reference's formula (``_fused.py:73-85``) as torch CPU ops: two-pass
    float32 mean / variance, ``y = xc * rsqrt(var + eps)``, ``y * sc1 + s``
    rounded to bf16, then the torch quantizer with ConvRot 256: (codes, scales)."""
    xt = torch.from_numpy(x)
    K = x.shape[1]
    xc = xt - xt.sum(1, keepdim=True) / K
    y = xc * torch.rsqrt((xc * xc).sum(1, keepdim=True) / K + 1e-6)
    m = torch.arange(x.shape[0]) // rows_per_mod
    out = (y * torch.from_numpy(sc1)[m] + torch.from_numpy(sh)[m]).to(torch.bfloat16)
    q, s = OC.quantize_rows(OC.rotate(out.float(), 256))
    return q.numpy(), s.numpy()


@pytest.mark.parametrize("offset", [0.0, 1000.0])
def test_ln_mod_oracle_against_torch_statement(offset):
    """The oracle against torch CPU ops of the reference's formula: codes equal
    except for float32 order effects (within one step, >99% equal), row scales
    within 1e-3. Codes are invariant to a per-row factor, so the row scales
    carry rstd: with a large row mean a planted one-pass variance
    (E[x^2] - mean^2 in float32) moves them by percents."""
    g = np.random.default_rng(8)
    x = (g.standard_normal((16, 768)) + offset).astype(np.float32)
    sc1 = OF.round_to(g.uniform(0.5, 1.5, (2, 768)).astype(np.float32), "bf16")
    sh = OF.round_to(g.standard_normal((2, 768)).astype(np.float32) * 0.1, "bf16")
    qt, st = _torch_ln_mod_codes(x, sc1, sh, 8)
    q, s = OQ.ln_mod_quantize(x, sc1, sh, 8, 1e-6, 256, "bf16")
    assert np.all(np.abs(q.astype(int) - qt) <= 1) and (q == qt).mean() > 0.99
    np.testing.assert_allclose(s, st, rtol=1e-3)
    if offset:
        m = np.arange(16) // 8
        mean32 = x.mean(1, dtype=np.float32, keepdims=True)
        var1 = (x * x).mean(1, dtype=np.float32, keepdims=True) - mean32 * mean32
        y1 = ((x - mean32) / np.sqrt(np.maximum(var1, 0) + 1e-6)).astype(np.float32)
        _, sb = OQ.quantize_activation(OF.round_to(y1 * sc1[m] + sh[m], "bf16"), 256)
        assert np.abs(sb / st - 1).max() > 1e-2
