"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py
from the CPU oracle on small seeded inputs with the reference tests' edge
cases). On the CPU the oracle must still reproduce them; on the GPU the HIP
kernels must: codes, scales, key sums and the GEMM bit for bit, the attention
output within the oracle tolerance of tests/test_gpu_attn.py."""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import attn as OA
from oracle import gemm as OG
from oracle import quant as OQ

GOLDEN = Path(__file__).resolve().parent / "golden"
ATTN = [("attn_bf16_d128.npz", "bf16"), ("attn_f16_d40.npz", "f16")]
TORCH_DT = {"bf16": torch.bfloat16, "f16": torch.float16}


def _load(name):
    with np.load(GOLDEN / name) as z:
        return {k: z[k] for k in z.files}


def _bits_equal(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


def _ulp_close(a, b, dtype):
    """Equal, or one step of the 16-bit dtype apart (float64 BLAS order)."""
    step = 2.0 ** -8 if dtype == "bf16" else 2.0 ** -11
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return bool(np.all(np.abs(a - b) <= step * np.maximum(np.abs(b), 2.0 ** -14)))


# ---------------------------------------------------------------- oracle (CPU)

def test_oracle_reproduces_quant_fixture():
    g = _load("quant.npz")
    q0, s0 = OQ.quantize_rows(g["x_group0"])
    assert np.array_equal(q0, g["q_group0"]) and _bits_equal(s0, g["s_group0"])
    q1, s1 = OQ.quantize_activation(g["x_rot"], 256)
    assert np.array_equal(q1, g["q_rot"]) and _bits_equal(s1, g["s_rot"])


def test_oracle_reproduces_gemm_fixture():
    g = _load("gemm.npz")
    acc = OG.int_mm(g["q"], g["w"])
    assert np.array_equal(acc, g["acc"])
    for dt in ("f16", "bf16", "f32"):
        assert _bits_equal(OG.rescale(acc, g["sx"], g["sw"], None, dt), g[f"y_{dt}"])
        assert _bits_equal(OG.rescale(acc, g["sx"], g["sw"], g["bias_bf16"], dt), g[f"y_{dt}_bias"])


@pytest.mark.parametrize("name,dtype", ATTN)
def test_oracle_reproduces_attention_fixture(name, dtype):
    g = _load(name)
    ksum = OA.k_colsum(g["k"])
    assert _bits_equal(ksum, g["ksum"])
    ki, ks = OA.k_quantize(g["k"], ksum)
    assert np.array_equal(ki, g["k8"]) and _bits_equal(ks, g["ks"])
    q8, qs = OA.q_quantize(g["q"])
    assert np.array_equal(q8, g["q8"]) and _bits_equal(qs, g["qs"])
    D = g["q"].shape[-1]
    o = OA.int8_attention(g["q"], g["k"], g["v"], D ** -0.5, p_dtype=dtype, out_dtype=dtype)
    assert _ulp_close(o, g["o"], dtype)


# ---------------------------------------------------------------- HIP kernels (GPU)

@pytest.mark.gpu
def test_hip_quantize_matches_fixture(gpu):
    from diffucore_amd import _int8
    g = _load("quant.npz")
    q, s = _int8.quantize_activation(torch.from_numpy(g["x_group0"]).to(gpu), 0)
    assert np.array_equal(q.cpu().numpy(), g["q_group0"]) and _bits_equal(s.cpu().numpy(), g["s_group0"])
    x1 = torch.from_numpy(g["x_rot"]).to(torch.bfloat16).to(gpu)     # the values are bf16
    q, s = _int8.quantize_activation(x1, 256)
    assert np.array_equal(q.cpu().numpy(), g["q_rot"]) and _bits_equal(s.cpu().numpy(), g["s_rot"])


@pytest.mark.gpu
def test_hip_gemm_matches_fixture(gpu):
    from diffucore_amd import _int8
    g = _load("gemm.npz")
    q, w = torch.from_numpy(g["q"]).to(gpu), torch.from_numpy(g["w"]).to(gpu)
    sx, sw = torch.from_numpy(g["sx"]).to(gpu), torch.from_numpy(g["sw"]).to(gpu)
    bias = torch.from_numpy(g["bias_bf16"]).to(torch.bfloat16).to(gpu)
    assert np.array_equal(_int8.int_mm(q, w).cpu().numpy(), g["acc"])
    for dt, tdt in (("f16", torch.float16), ("bf16", torch.bfloat16), ("f32", torch.float32)):
        y = _int8.rescale(_int8.int_mm(q, w), sx, sw, None, tdt)
        assert _bits_equal(y.float().cpu().numpy(), g[f"y_{dt}"])
        lin = _int8.Int8Linear(q.shape[1], w.shape[0], bias=True, group=0, device=gpu)
        lin.weight.copy_(w)
        lin.scale_bits.copy_(sw.view(torch.int32))
        lin.bias = torch.nn.Parameter(bias, requires_grad=False)
        yb = lin.matmul_quantized(q, sx, tdt)
        assert _bits_equal(yb.float().cpu().numpy(), g[f"y_{dt}_bias"])


@pytest.mark.gpu
@pytest.mark.parametrize("name,dtype", ATTN)
def test_hip_attention_matches_fixture(gpu, name, dtype):
    from diffucore_amd import _attention as A
    g = _load(name)
    tdt = TORCH_DT[dtype]
    q, k, v = (torch.from_numpy(g[n]).to(tdt).to(gpu) for n in ("q", "k", "v"))
    B, Lq, H, D = q.shape
    Lk = k.shape[1]
    ws = torch.empty(A.workspace_bytes(B, H, Lq, Lk, D), device=gpu, dtype=torch.uint8)
    o = A.int8_attention(q, k, v, D ** -0.5, workspace=ws)
    views = A.workspace_views(ws, B, H, Lq, Lk, D)
    assert _bits_equal(views["ksum"].cpu().numpy(), g["ksum"])
    assert np.array_equal(views["k8"].cpu().numpy()[..., :D], g["k8"])
    assert _bits_equal(views["ks"].cpu().numpy(), g["ks"])
    q8, qs = A.quantize_q(q)
    assert np.array_equal(q8.cpu().numpy()[:, :, :Lq, :D], g["q8"])
    assert _bits_equal(qs.cpu().numpy()[:, :, :Lq], g["qs"])
    ref, out = g["o"].astype(np.float64), o.float().cpu().numpy().astype(np.float64)
    rel = np.linalg.norm(out - ref) / np.linalg.norm(ref)
    assert rel < {"bf16": 4e-3, "f16": 1e-3}[dtype], rel
