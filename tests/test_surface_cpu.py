"""The operator surface on the CPU (no GPU): dispatch semantics of the
reference's attention module (``tests/test_attention_dispatch.py``), the
load-time parts of ``Int8Linear`` (``tests/test_int8.py:40-71``), the C ABI's
exported symbols and argument checks, and the absence of any CPU fallback
on the W8A8 hot path."""

from __future__ import annotations

import re
import subprocess
import sys
from pathlib import Path

import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

import diffucore_amd as D
from diffucore_amd import _attention, _int8, _lib

ROOT = Path(__file__).resolve().parent.parent
_CPU = D.DevicePolicy(device=torch.device("cpu"), compute_dtype=torch.float32)


def _rel(a, b):
    return ((a.float() - b.float()).norm() / b.float().norm()).item()


# ---------------------------------------------------------------- attention dispatch

def _ref_blhd(q, k, v):
    out = F.scaled_dot_product_attention(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2))
    return out.transpose(1, 2).reshape(q.shape[0], q.shape[1], -1)


def test_sdpa_branches_are_exact():
    torch.manual_seed(0)
    q, k, v = torch.randn(2, 64, 4, 32), torch.randn(2, 48, 4, 32), torch.randn(2, 48, 4, 32)
    assert torch.equal(D.attention_blhd(q, k, v, "sdpa"), _ref_blhd(q, k, v))
    qh, kh, vh = (torch.randn(2, 4, 64, 32) for _ in range(3))
    ref = F.scaled_dot_product_attention(qh, kh, vh).transpose(1, 2).reshape(2, 64, -1)
    assert torch.equal(D.attention_bhld(qh, kh, vh, "sdpa"), ref)


def test_int8_backend_falls_back_off_gpu():
    q = torch.randn(1, 16, 2, 128)
    assert torch.equal(D.attention_blhd(q, q, q, "int8_turing"), D.attention_blhd(q, q, q, "sdpa"))
    qh = torch.randn(1, 2, 16, 64)
    assert torch.equal(D.attention_bhld(qh, qh, qh, "int8_turing"), D.attention_bhld(qh, qh, qh, "sdpa"))


def test_null_keys_equal_padded():
    torch.manual_seed(0)
    q, k, v = torch.randn(1, 30, 4, 64), torch.randn(1, 7, 4, 64), torch.randn(1, 7, 4, 64)
    pad = (0, 0, 0, 0, 0, 5)
    assert torch.equal(D.attention_blhd(q, k, v, null_keys=5), D.attention_blhd(q, F.pad(k, pad), F.pad(v, pad)))


def test_int8_guard_needs_paired_shapes():
    """The per-call guard sends calls whose operands do not pair up (batch,
    heads, key/value lengths) or have an empty sequence to SDPA instead of the
    kernel's shape error."""
    ok = _attention._blhd_compatible
    z = torch.zeros
    assert ok(z(2, 64, 4, 64), z(2, 77, 4, 64), z(2, 77, 4, 64))
    assert not ok(z(2, 64, 4, 64), z(1, 77, 4, 64), z(1, 77, 4, 64))      # batch
    assert not ok(z(2, 64, 4, 64), z(2, 77, 2, 64), z(2, 77, 2, 64))      # heads
    assert not ok(z(2, 64, 4, 64), z(2, 77, 4, 64), z(2, 76, 4, 64))      # k / v lengths
    assert not ok(z(2, 0, 4, 64), z(2, 77, 4, 64), z(2, 77, 4, 64))       # no queries
    assert not ok(z(2, 64, 4, 64), z(2, 0, 4, 64), z(2, 0, 4, 64))        # no keys
    assert not ok(z(64, 4, 64), z(2, 77, 4, 64), z(2, 77, 4, 64))         # not 4-d
    # SDPA takes an empty key set on the int8 backend's fallback path
    q = torch.randn(1, 5, 2, 64)
    out = D.attention_blhd(q, torch.zeros(1, 0, 2, 64), torch.zeros(1, 0, 2, 64), "int8_turing")
    assert out.shape == (1, 5, 128)


def test_policy_resolution():
    assert D.resolve_attention_backend(_CPU) == "sdpa"
    auto = D.DevicePolicy(device=torch.device("cpu"), compute_dtype=torch.float32, attention="auto")
    assert D.resolve_attention_backend(auto) == "sdpa"
    for attn in ("int8_turing", "fa2_turing"):
        pol = D.DevicePolicy(device=torch.device("cpu"), compute_dtype=torch.float32, attention=attn)
        with pytest.raises(ValueError, match=attn):
            D.resolve_attention_backend(pol)
    pol = D.DevicePolicy(device=torch.device("cpu"), compute_dtype=torch.float16, attention="int8_turing",
                         compile=True)
    with pytest.raises(ValueError, match="compile"):
        D.resolve_attention_backend(pol)
    with pytest.raises(ValueError, match="attention"):
        D.DevicePolicy(device=torch.device("cpu"), attention="flash3")


def test_int8_requirements_on_a_gfx950_policy(monkeypatch):
    """With the device checks satisfied, the remaining requirement messages are
    the dtype and compile ones (and a missing library would be named)."""
    monkeypatch.setattr(_attention, "_is_gfx950", lambda d=None: True)
    pol = D.DevicePolicy(device=torch.device("cuda"), compute_dtype=torch.float32, attention="int8_turing")
    with pytest.raises(ValueError, match="fp16 or bf16"):
        D.resolve_attention_backend(pol)
    pol = D.DevicePolicy(device=torch.device("cuda"), compute_dtype=torch.bfloat16, attention="int8_turing")
    if _lib.lib() is not None:
        assert D.resolve_attention_backend(pol) == "int8_turing"
    monkeypatch.setattr(_lib, "lib", lambda: None)
    monkeypatch.setattr(_lib, "load_error", lambda: "libdiffucore_amd.so is not built")
    with pytest.raises(ValueError, match="not built"):
        D.resolve_attention_backend(pol)


class _SelfAttn(nn.Module):
    def __init__(self):
        super().__init__()
        self.attn_backend = "sdpa"


class _CrossAttn(_SelfAttn):
    is_selfattn = False


def test_stamping_self_and_cross_attention():
    holder = nn.ModuleList([_SelfAttn(), _CrossAttn(), nn.Linear(2, 2), _SelfAttn()])
    assert D.set_attention_backend(holder, "int8_turing") == 3
    assert [getattr(m, "attn_backend", None) for m in holder] == ["int8_turing", "sdpa", None, "int8_turing"]
    assert D.set_attention_backend(holder, "sdpa") == 3


def test_flux_harness_stamps_and_swaps():
    import flux_step as FS
    shape = FS.FluxShape(hidden=256, heads=2, depth=2, depth_single=3, context_dim=64, vec_dim=32,
                         axes=(16, 56, 56), img_hw=(4, 4), txt_len=8)
    with torch.device("meta"):
        model = FS.FluxDiT(shape)
    assert D.set_attention_backend(model, "int8_turing") == 5
    names = FS.block_linear_names(model)
    assert len(names) == 2 * 8 + 3 * 2
    assert all(isinstance(model.get_submodule(n), nn.Linear) for n in names)


# ---------------------------------------------------------------- Int8Linear (load time)

def test_hadamard_is_symmetric_and_self_inverse():
    h = _int8._hadamard(256, "cpu")
    torch.testing.assert_close(h, h.T)
    torch.testing.assert_close(h @ h, torch.eye(256), atol=1e-6, rtol=0)


def test_weight_round_trip_and_to_linear():
    torch.manual_seed(0)
    w = torch.randn(64, 512) * 0.02
    for group in (0, 256):
        q, s = D.quantize_weight(w, group)
        assert _rel(D.dequantize_weight(q, s, group), w) < 0.01
    lin = nn.Linear(512, 64)
    m = D.Int8Linear.from_linear(lin)
    back = m.to_linear(torch.float32)
    assert _rel(back.weight, lin.weight) < 0.01 and torch.equal(back.bias, lin.bias)


def test_scale_survives_dtype_cast():
    m = D.Int8Linear.from_linear(nn.Linear(256, 32))
    s = m.scale.clone()
    m.to(torch.float16)
    assert m.weight.dtype == torch.int8 and torch.equal(m.scale, s)


def test_group_must_divide_in_features():
    with pytest.raises(ValueError, match="multiple"):
        D.Int8Linear(320, 64, group=256)


@pytest.mark.parametrize("group,dtype,bias", [(256, torch.float32, True), (0, torch.float32, False),
                                              (256, torch.bfloat16, True), (0, torch.float16, True)])
def test_w8a8_on_cpu_tensors_is_the_reference_torch_path(group, dtype, bias):
    """CPU tensors run the reference's own torch statement of the W8A8 path
    (``_int8.py:200-207, 299-323``): rotate + per-row int8, ``torch._int_mm``
    (M <= 16 padded to 32), rescale. Codes, scales and outputs equal the
    oracle's CPU restatement of that path bit for bit, at M below and above
    the padding threshold; ``scaled_mm`` keeps its None answer on the CPU."""
    from oracle import cpu_path as CP
    torch.manual_seed(3)
    lin = nn.Linear(512, 96, bias=bias).to(dtype)
    m = D.Int8Linear.from_linear(lin, group)
    for rows in (5, 40):
        x = torch.randn(rows, 512).to(dtype)
        q, s = D.quantize_activation(x, group)
        q_ref, s_ref = CP.quantize_rows(CP.rotate(x.float(), group))
        assert torch.equal(q, q_ref) and torch.equal(s, s_ref)
        acc = D.int_mm(q, m.weight)
        assert acc.dtype == torch.int32 and torch.equal(acc, q.long().matmul(m.weight.long().T).int())
        y = m(x)
        want = CP.rescale(CP.int_mm(q_ref, m.weight), s_ref, m.scale, m.bias, dtype)
        assert y.dtype == dtype and torch.equal(y, want)
        ys = D.linear_group([m, m], [x, x])
        assert all(torch.equal(t, y) for t in ys)
    assert D.scaled_mm(torch.zeros(3, 16, dtype=torch.int8), torch.zeros(8, 16, dtype=torch.int8),
                       torch.ones(3), torch.ones(8), torch.float16) is None


def test_device_tensors_never_take_the_torch_path(monkeypatch):
    """The torch statement is only for CPU tensors: any other tensor goes to
    the HIP library, and with the library missing the call raises instead of
    running the torch ops (no silent fallback). A meta tensor stands in for a
    GPU tensor, with the GPU-device check disabled and the library made to
    look missing."""
    from diffucore_amd import _int8, _lib

    def missing():
        raise RuntimeError("libdiffucore_amd.so is not built")

    monkeypatch.setattr(_lib, "require", missing)
    monkeypatch.setattr(_int8, "_on_gpu", lambda t, what: None)
    x = torch.empty(4, 256, device="meta")
    q8 = torch.empty(4, 256, dtype=torch.int8, device="meta")
    for call in (lambda: _int8.quantize_activation(x, 256), lambda: _int8.int_mm(q8, q8),
                 lambda: _int8.rescale(torch.empty(4, 8, dtype=torch.int32, device="meta"),
                                       torch.empty(4, device="meta"), torch.empty(8, device="meta"), None,
                                       torch.float16)):
        with pytest.raises(RuntimeError, match="not built"):
            call()


def test_entry_points_refuse_host_tensors_before_any_launch():
    """Every wrapper that reaches the C ABI enters the device context first,
    and that refuses a CPU device: host pointers never reach a kernel."""
    from diffucore_amd import _attention as A
    from diffucore_amd import _lib
    with pytest.raises(RuntimeError, match="GPU tensors"):
        _lib.device_ctx(torch.device("cpu"))
    if _lib.lib() is None:
        pytest.skip(f"library not built: {_lib.load_error()}")
    q = torch.randn(1, 200, 2, 64, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="GPU tensors"):
        A.int8_attention(q, q, q, 0.125)
    with pytest.raises(RuntimeError, match="GPU tensors"):
        A.quantize_q(q)



def test_quantize_and_dequantize_linears():
    model = nn.Sequential(nn.Linear(512, 256), nn.GELU(), nn.Linear(256, 64))
    assert D.quantize_linears(model, ["0", "2"], "cpu", group=0) == 2
    assert isinstance(model[0], D.Int8Linear) and model[0].group == 0
    assert _int8.dequantize_linears(model, torch.float32) == 2
    assert type(model[0]) is nn.Linear


# ---------------------------------------------------------------- C ABI

def _declared_symbols() -> list[str]:
    text = (ROOT / "include" / "diffucore_amd.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(dc_[a-z0-9_]+)\s*\(", text)))


def test_header_and_binding_agree():
    assert _declared_symbols() == sorted(_lib.SYMBOLS)


@pytest.mark.skipif(not _lib.LIB_PATH.exists(), reason="library not built (run __graft_entry__.build())")
def test_library_exports_every_declared_symbol():
    so = _lib.lib()
    assert so is not None, _lib.load_error()
    for name in _declared_symbols():
        assert hasattr(so, name), name
    assert so.dc_abi_version() == _lib.ABI_VERSION


@pytest.mark.skipif(not _lib.LIB_PATH.exists(), reason="library not built")
def test_argument_checks_fail_before_any_launch():
    """Invalid arguments are rejected on the host, with a message, before any
    HIP call (so these run without a GPU)."""
    so = _lib.lib()
    assert so.dc_quantize_rows(None, _lib.BF16, 4, 300, 300, 256, None, 300, None, None) == 1
    assert b"group" in so.dc_last_error() or b"null" in so.dc_last_error()
    assert so.dc_quantize_rows(1, _lib.BF16, 4, 512, 512, 3, 1, 512, 1, None) == 1
    assert b"group" in so.dc_last_error()
    assert so.dc_quantize_rows(1, _lib.BF16, 0, 512, 512, 0, 1, 512, 1, None) == 0      # empty batch
    assert so.dc_w8a8_gemm(16, 24, 16, 24, 16, 16, None, -1, 16, _lib.BF16, 8, 4, 8, 24, None, 0, None) == 2
    assert b"K" in so.dc_last_error()
    assert so.dc_w8a8_gemm(16, 32, 16, 32, 16, 16, None, 7, 16, _lib.BF16, 8, 4, 8, 32, None, 0, None) == 1
    # split-K workspace: small M with long K splits (FLUX text MLP down: 4 slices of int32 partials), big M does not
    assert so.dc_w8a8_gemm_workspace_bytes(512, 3072, 12288, 12288, 12288) == 4 * 512 * 3072 * 4
    assert so.dc_w8a8_gemm_workspace_bytes(4096, 3072, 12288, 12288, 12288) == 0
    assert so.dc_w8a8_gemm_workspace_bytes(154, 1280, 2048, 2048, 2048) == 4 * 154 * 1280 * 4   # 20 tiles
    assert so.dc_w8a8_gemm_workspace_bytes(512, 3072, 2048, 2048, 2048) == 0   # 96 tiles: no 2048-deep split
    assert so.dc_w8a8_gemm_workspace_bytes(512, 3072, 100, 112, 112) == 0
    assert so.dc_int8_attn_workspace_bytes(1, 24, 4608, 4608, 128) > 24 * 4608 * 128
    assert so.dc_int8_attn_workspace_bytes(1, 1, 1, 1, 200) == 0
    st = (_lib.ctypes.c_int64 * 3)(8, 8, 8)
    assert so.dc_int8_attn_fwd(16, 16, 16, 16, _lib.BF16, 1, 1, 4, 4, 36, st, st, st, st, 0.1, 16, 1 << 20,
                               None) == 2
    assert b"head dim" in so.dc_last_error()
    assert so.dc_int8_attn_fwd(16, 16, 16, 16, _lib.F32, 1, 1, 4, 4, 64, st, st, st, st, 0.1, 16, 1 << 20,
                               None) == 1
    # the MFMA calibration probe: kind, vary, waves and iteration count checked before any HIP call
    assert so.dc_mfma_probe(2, 0, 1, 10, 16, None) == 1 and b"kind" in so.dc_last_error()
    assert so.dc_mfma_probe(0, 0, 3, 10, 16, None) == 1
    assert so.dc_mfma_probe(1, 1, 1, 0, 16, None) == 1
    assert so.dc_mfma_probe(0, 1, 2, 10, None, None) == 1 and b"null" in so.dc_last_error()
    # dc_qk_norm_rope: argument order (dtype, B, L, H, D, flags, eps, q, q_strides, q_weight, k, k_strides,
    # k_weight, weight_dtype, freqs, fb, fl, q_out, qo_strides, k_out, ko_strides, v, v_strides, v_out,
    # vo_strides, stream)
    none = [None] * 3

    def qk(dtype, B, D, flags=0, eps=1e-6, wdt=_lib.BF16):
        return so.dc_qk_norm_rope(dtype, B, 8, 2, D, flags, eps, 16, st, 16, *none, wdt, None, 0, 0, 16, st,
                                  None, None, None, None, None, None, None)

    assert qk(_lib.BF16, 0, 64) == 0                                      # empty batch
    assert qk(_lib.BF16, 1, 96) == 2 and b"D must be" in so.dc_last_error()
    assert qk(_lib.F32, 1, 64) == 1 and b"dtype" in so.dc_last_error()
    assert qk(_lib.BF16, 1, 64, wdt=_lib.F16) == 1 and b"weight_dtype" in so.dc_last_error()
    assert qk(_lib.BF16, 1, 64, flags=4) == 1 and b"flags" in so.dc_last_error()
    assert qk(_lib.BF16, 1, 64, eps=-1.0) == 1 and b"eps" in so.dc_last_error()
    # dc_int8_attn_fwd_noalloc: a call beyond its scratch is refused before any HIP call
    assert so.dc_int8_attn_fwd_noalloc(16, 16, 16, 16, _lib.BF16, 8, 32, 8192, 8192, 128, st, st, st, st, 0.1,
                                       None) == 4
    assert b"scratch" in so.dc_last_error()
    # dc_rescale: M or N beyond int range is rejected (the kernel indexes rows in int)
    assert so.dc_rescale(16, 4, 16, 16, None, -1, 16, _lib.BF16, 4, (1 << 31) + 5, 4, None) == 1
    assert b"too large" in so.dc_last_error()
    # dc_act_quantize_rows, GEGLU: x2 rows must hold 2 * K2 values
    assert so.dc_act_quantize_rows(None, 0, 0, 16, 256, 256, 3, _lib.F16, 4, 256, 16, 256, 16, None) == 1
    assert b"ld2" in so.dc_last_error()
    assert so.dc_act_quantize_rows(None, 0, 0, 16, 512, 256, 4, _lib.F16, 4, 256, 16, 256, 16, None) == 1
    assert b"unknown act" in so.dc_last_error()
    # dc_w8a8_gemm_grouped: counts, K, dtypes and each problem's pointers / strides
    P = _lib.GemmProblem
    probs = (P * 2)(P(16, 512, 16, 512, 16, 16, None, 16, 3072, 4096), P(16, 512, 16, 512, 16, 16, None, 16, 3072, 512))
    assert so.dc_w8a8_gemm_grouped(probs, 0, 3072, 512, -1, _lib.BF16, None) == 1
    assert so.dc_w8a8_gemm_grouped(probs, 5, 3072, 512, -1, _lib.BF16, None) == 1
    assert so.dc_w8a8_gemm_grouped(None, 2, 3072, 512, -1, _lib.BF16, None) == 1
    assert so.dc_w8a8_gemm_grouped(probs, 2, 3072, 320, -1, _lib.BF16, None) == 2 and b"256" in so.dc_last_error()
    assert so.dc_w8a8_gemm_grouped(probs, 2, 3072, 512, 9, _lib.BF16, None) == 1 and b"bias" in so.dc_last_error()
    assert so.dc_w8a8_gemm_grouped(probs, 2, 3072, 512, -1, 7, None) == 1 and b"out_dtype" in so.dc_last_error()
    bad = (P * 2)(P(16, 512, 16, 512, 16, 16, None, 16, 3072, 64), P(16, 500, 16, 512, 16, 16, None, 16, 3072, 64))
    assert so.dc_w8a8_gemm_grouped(bad, 2, 3072, 512, -1, _lib.BF16, None) == 2 and b"lda" in so.dc_last_error()
    bad = (P * 2)(P(16, 512, 16, 512, 16, 16, None, 16, 3072, 64), P(16, 512, None, 512, 16, 16, None, 16, 3072, 64))
    assert so.dc_w8a8_gemm_grouped(bad, 2, 3072, 512, -1, _lib.BF16, None) == 1 and b"null" in so.dc_last_error()
    bad = (P * 1)(P(16, 512, 16, 512, 16, 16, None, 16, 3072, -1))
    assert so.dc_w8a8_gemm_grouped(bad, 1, 3072, 512, -1, _lib.BF16, None) == 1 and b"negative" in so.dc_last_error()
    bad = (P * 1)(P(16, 512, 16, 512, None, 16, None, 16, 3072, 8))
    assert so.dc_w8a8_gemm_grouped(bad, 1, 3072, 512, -1, _lib.BF16, None) == 1 and b"scales" in so.dc_last_error()
    bad = (P * 1)(P(16, 512, 16, 512, 16, 16, None, 16, 3000, 8))
    assert so.dc_w8a8_gemm_grouped(bad, 1, 3072, 512, -1, _lib.BF16, None) == 1 and b"ldo" in so.dc_last_error()
    empty = (P * 2)(P(16, 512, 16, 512, 16, 16, None, 16, 3072, 0), P(None, 0, None, 0, None, None, None, None, 0, 0))
    assert so.dc_w8a8_gemm_grouped(empty, 2, 3072, 512, -1, _lib.BF16, None) == 0       # nothing to run
    # dc_w8a8_gemm_grouped_gated: the gates array, a float output, each residual and gate
    G = _lib.GemmGate
    gates = (G * 2)(G(16, 3072, 16), G(16, 3072, 16))
    gated = so.dc_w8a8_gemm_grouped_gated
    assert gated(probs, None, 2, 3072, 512, -1, _lib.BF16, None) == 1 and b"null" in so.dc_last_error()
    assert gated(probs, gates, 2, 3072, 512, -1, _lib.I32, None) == 1 and b"out_dtype" in so.dc_last_error()
    assert gated(probs, gates, 2, 3072, 320, -1, _lib.BF16, None) == 2 and b"256" in so.dc_last_error()
    assert gated(probs, (G * 2)(G(16, 3072, 16), G(None, 3072, 16)), 2, 3072, 512, -1, _lib.BF16, None) == 1
    assert b"residual or gate" in so.dc_last_error()
    assert gated(probs, (G * 2)(G(16, 3072, 16), G(16, 3072, None)), 2, 3072, 512, -1, _lib.BF16, None) == 1
    assert gated(probs, (G * 2)(G(16, 3000, 16), G(16, 3072, 16)), 2, 3072, 512, -1, _lib.BF16, None) == 1
    assert b"ldr" in so.dc_last_error()
    assert gated(empty, (G * 2)(G(None, 0, None), G(None, 0, None)), 2, 3072, 512, -1, _lib.BF16, None) == 0
    # the group plan (256 CUs when no device answers): FLUX's double-block pairs
    Ms = (_lib.ctypes.c_int64 * 2)(4096, 512)
    assert so.dc_w8a8_gemm_group_plan(Ms, 2, 9216, 3072) == 1          # 576 + 72 tiles: 3 rounds either way
    assert so.dc_w8a8_gemm_group_plan(Ms, 2, 3072, 3072) == 1          # 192 + 24: 1 round
    assert so.dc_w8a8_gemm_group_plan(Ms, 2, 12288, 3072) == 0         # 768 + 96: 4 rounds against 3
    assert so.dc_w8a8_gemm_group_plan(Ms, 2, 3072, 3000) == 0          # K not a multiple of 256
    assert so.dc_w8a8_gemm_group_plan(Ms, 1, 3072, 3072) == 0          # one problem
    assert so.dc_w8a8_gemm_group_plan(Ms, 0, 3072, 3072) == -1


def test_bench_cpu_configs_reports_every_shape(monkeypatch, capsys):
    """`bench.py --cpu-configs` (the reference's CPU path per config shape,
    sampled and scaled to a whole call) on two small shapes: one JSON line
    per shape plus config 1, each with a positive time, its sample and the
    thread count."""
    import json
    sys.path.insert(0, str(ROOT))
    import bench
    monkeypatch.setattr(bench, "ATTN_SHAPES", [("tiny_self", 1, 2, 300, 300, 40, torch.float16, 0.0)])
    monkeypatch.setattr(bench, "LIN_SHAPES", [("tiny_linear", 300, 512, 384, torch.bfloat16)])
    monkeypatch.setattr(bench, "cpu_cfg1", lambda budget_s: {"ms_per_call": 1.0, "TOPS": 1.0, "cores": 1})
    bench.cpu_configs(budget_s=0.01)
    rows = [json.loads(l) for l in capsys.readouterr().out.splitlines() if l.startswith("{")]
    assert [r["shape"] for r in rows] == ["cfg1_sd15_ff", "tiny_self", "tiny_linear"]
    att, lin = rows[1], rows[2]
    assert att["kind"] == "cpu_attention" and att["sample_queries"] == 300 and att["ms_per_call"] > 0
    assert lin["kind"] == "cpu_w8a8_linear" and lin["sample_rows"] == 256 and lin["group"] == 256
    assert lin["ms_per_call"] > 0 and lin["cores"] == torch.get_num_threads()


def test_bench_refuses_more_than_one_gpu():
    res = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                         timeout=120)
    assert res.returncode == 2 and "one GPU" in res.stderr


def test_quantize_row_index_formula():
    """The LDS quantize kernel finds a lane's row as int((t + 0.5) * fl(1 / lr))
    (float32) instead of t / lr: exact for every row width it launches
    (lr = 8 * G lanes, G = 1..128 groups of 256) and every lane t < 1024."""
    import numpy as np
    t = np.arange(1024, dtype=np.float32)
    for G in range(1, 129):
        lr = 8 * G
        inv = np.float32(1.0) / np.float32(lr)
        r = ((t + np.float32(0.5)) * inv).astype(np.float32).astype(np.int64)
        assert np.array_equal(r, np.arange(1024) // lr), lr


@pytest.mark.skipif(not _lib.LIB_PATH.exists(), reason="library not built")
def test_gemm_plan_choice_without_a_gpu():
    """The GEMM tile planner runs on the host (assuming 256 CUs when no device
    answers). FLUX-step shapes take the DMA-fed 256x256 kernel when K is a
    multiple of 256, the 192x256 tiles when they fill the last round better,
    192x128 tiles (one per CU) for the 512-row text qkv / MLP up whose 128x128
    tiles would load CUs unevenly, 2-per-CU 128x128 tiles for the shorter
    ones when they fit one round, and 256x256 tiles over several."""
    so = _lib.lib()
    assert so.dc_w8a8_gemm_plan(4608, 21504, 3072, 3072, 3072) == 3      # linear1
    assert so.dc_w8a8_gemm_plan(4608, 3072, 15360, 15360, 15360) == 3    # linear2
    assert so.dc_w8a8_gemm_plan(4096, 9216, 3072, 3072, 3072) == 1       # image qkv
    assert so.dc_w8a8_gemm_plan(512, 9216, 3072, 3072, 3072) == 4        # text qkv
    assert so.dc_w8a8_gemm_plan(512, 12288, 3072, 3072, 3072) == 4       # text MLP up
    assert so.dc_w8a8_gemm_plan(512, 3072, 3072, 3072, 3072) == 2        # text proj (64 tiles of 192x128)
    assert so.dc_w8a8_gemm_plan(2048, 1280, 1280, 1280, 1280) == 2       # SDXL level-2 q/k/v/o
    assert so.dc_w8a8_gemm_plan(8192, 5120, 640, 640, 640) == 0          # SDXL GEGLU: 5 rounds of 128x128 lose
    assert so.dc_w8a8_gemm_plan(8192, 640, 640, 640, 640) == 2           # SDXL q/k/v/o: 192x128 would pad N by 20%
    assert so.dc_w8a8_gemm_plan(4096, 12288, 272, 272, 272) == 0         # K % 256 != 0
    assert so.dc_w8a8_gemm_plan(0, 1, 16, 16, 16) == -1                  # invalid shape
    assert [_int8.gemm_plan(4608, 21504, 3072), _int8.gemm_plan(512, 9216, 3072)] == ["dma_256x256", "192x128"]


@pytest.mark.skipif(not _lib.LIB_PATH.exists(), reason="library not built")
def test_attention_work_split_without_a_gpu():
    """The attention work split runs on the host (512 resident workgroups, 2
    per CU on 256 CUs, when no device answers). SDXL's 640 query tiles at 4096
    tokens run 512 whole and share the last 128 (a quarter-full round) over
    512 stream-K workgroups; whole rounds and short key ranges run whole.
    Head dims above 64 run 256-query tiles, all whole (FLUX: 18 per head),
    when there are at least as many as CUs; fewer take 128-query tiles."""
    from diffucore_amd import _attention as A
    assert A.attn_plan(2, 10, 4096, 4096, 64, torch.float16) == {"dp_tiles": 512, "sk_blocks": 512, "sk_tiles": 128}
    assert A.attn_plan(1, 24, 4608, 4608, 128) == {"dp_tiles": 432, "sk_blocks": 0, "sk_tiles": 0}
    assert A.attn_plan(1, 4, 1024, 1024, 128) == {"dp_tiles": 32, "sk_blocks": 0, "sk_tiles": 0}
    assert A.attn_plan(2, 8, 4096, 4096, 40, torch.float16) == {"dp_tiles": 512, "sk_blocks": 0, "sk_tiles": 0}
    assert A.attn_plan(2, 10, 4096, 77, 64, torch.float16)["sk_blocks"] == 0
    ws = _lib.lib().dc_int8_attn_workspace_bytes(2, 10, 4096, 4096, 64)
    assert ws >= 2 * 512 * (128 * 64 + 256) * 4
