"""Seeded random-shape sweeps through the public entry points, each case
checked against the oracle end to end.

* W8A8 linear (``Int8Linear.forward``: rotate + quantize, GEMM, fused
  epilogue): random M, N, K, ConvRot group 0 or 256, output dtype and bias
  dtype. The output must equal, bit for bit, the oracle's
  ``rescale(int_mm(quantize_activation(x), W), ...)`` on the layer's own
  weight codes (reference ``_int8.py:87-97, 200-207, 313-323``).
* INT8 attention (``int8_attention``): random batch, heads, query and key
  lengths (down to one key) and head dims (multiples of 8 up to 128). K codes,
  block scales, key sums and Q codes bit-exact; the output within the
  oracle bound of ``tests/test_gpu_attn.py`` and the reference's fp32-SDPA bar
  (``tests/test_attention_dispatch.py:212-213``).

The cases come from one fixed numpy seed, so every run checks the same
shapes; each prints its parameters before it runs.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

from diffucore_amd import _attention as A
from diffucore_amd import _int8
from oracle import attn as OA
from oracle import gemm as OG
from oracle import quant as OQ
from tests._util import DT, cosine, np32, rel_l2

pytestmark = pytest.mark.gpu

_FLOATS = [torch.float16, torch.bfloat16, torch.float32]


def _linear_cases(n: int, seed: int):
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        group = int(rng.choice([0, 256]))
        K = int(rng.integers(1, 13)) * 256 if group else int(rng.integers(1, 257)) * 8
        M = int(rng.choice([1, 2, 31, 64, 255, 256, 257, 700, int(rng.integers(1, 1200))]))
        N = int(rng.choice([8, 16, 40, 256, 520, int(rng.integers(1, 200)) * 8]))
        dtype = _FLOATS[int(rng.integers(0, 3))]
        bias = [None, dtype, torch.float32][int(rng.integers(0, 3))]
        cases.append((i, M, N, K, group, dtype, bias))
    return cases


def _attn_cases(n: int, seed: int):
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        B, H = int(rng.integers(1, 3)), int(rng.integers(1, 5))
        Lq = int(rng.choice([1, 31, 33, 127, 129, 257, int(rng.integers(1, 600))]))
        Lk = int(rng.choice([1, 2, 63, 64, 65, 77, 129, 191, int(rng.integers(1, 700))]))
        D = int(rng.integers(1, 17)) * 8
        dtype = [torch.float16, torch.bfloat16][int(rng.integers(0, 2))]
        cases.append((i, B, H, Lq, Lk, D, dtype))
    return cases


LINEAR_CASES = _linear_cases(24, 20261)
ATTN_CASES = _attn_cases(24, 20262)


@pytest.mark.parametrize("i,M,N,K,group,dtype,bias_dtype", LINEAR_CASES)
def test_linear_sweep_bit_exact(gpu, i, M, N, K, group, dtype, bias_dtype):
    print(f"[sweep] linear {i}: M {M} N {N} K {K} group {group} {DT[dtype]} bias {bias_dtype}", flush=True)
    g = torch.Generator().manual_seed(100 + i)
    lin = nn.Linear(K, N, bias=bias_dtype is not None)
    with torch.no_grad():
        lin.weight.copy_(torch.randn(N, K, generator=g) * 0.02)
        if bias_dtype is not None:
            lin.bias.copy_(torch.randn(N, generator=g) * 0.5)
    layer = _int8.Int8Linear.from_linear(lin, group, device=gpu)
    if bias_dtype is not None:
        layer.bias = nn.Parameter(layer.bias.to(bias_dtype), requires_grad=False)
    x = torch.randn(M, K, generator=g)
    x[:, torch.randperm(K, generator=g)[: max(1, K // 200)]] *= 20    # outlier channels
    x = x.to(dtype)
    with torch.no_grad():
        y = layer(x.to(gpu))
    assert y.shape == (M, N) and y.dtype == dtype
    q_ref, s_ref = OQ.quantize_activation(np32(x), group)
    b = None if bias_dtype is None else np32(layer.bias)
    ref = OG.rescale(OG.int_mm(q_ref, layer.weight.cpu().numpy()), s_ref, layer.scale.cpu().numpy(), b, DT[dtype])
    assert np.array_equal(np32(y).view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("i,B,H,Lq,Lk,D,dtype", ATTN_CASES)
def test_attention_sweep(gpu, i, B, H, Lq, Lk, D, dtype):
    print(f"[sweep] attention {i}: B {B} H {H} Lq {Lq} Lk {Lk} D {D} {DT[dtype]}", flush=True)
    g = torch.Generator().manual_seed(200 + i)
    q = torch.randn(B, Lq, H, D, generator=g).to(dtype)
    k = (torch.randn(B, Lk, H, D, generator=g) + torch.randn(D, generator=g) * 2).to(dtype)
    v = torch.randn(B, Lk, H, D, generator=g).to(dtype)
    ws = torch.empty(A.workspace_bytes(B, H, Lq, Lk, D), device=gpu, dtype=torch.uint8)
    out = A.int8_attention(q.to(gpu), k.to(gpu), v.to(gpu), D ** -0.5, workspace=ws)
    views = A.workspace_views(ws, B, H, Lq, Lk, D)
    ksum = OA.k_colsum(np32(k))
    assert np.array_equal(views["ksum"].cpu().numpy().view(np.uint32), ksum.view(np.uint32))
    ki, ks = OA.k_quantize(np32(k), ksum)
    assert np.array_equal(views["ks"].cpu().numpy().view(np.uint32), ks.view(np.uint32))
    assert np.array_equal(views["k8"][..., :D].cpu().numpy(), ki)
    q8, qs = A.quantize_q(q.to(gpu))
    q8_ref, qs_ref = OA.q_quantize(np32(q))
    assert np.array_equal(q8[:, :, :Lq, :D].cpu().numpy(), q8_ref)
    assert np.array_equal(qs[:, :, :Lq].cpu().numpy().view(np.uint32), qs_ref.view(np.uint32))
    o = np32(out)
    assert out.shape == (B, Lq, H, D) and np.isfinite(o).all()
    ora = OA.int8_attention(np32(q), np32(k), np32(v), D ** -0.5, DT[dtype], DT[dtype])
    assert rel_l2(o, ora) < {torch.float16: 1e-3, torch.bfloat16: 4e-3}[dtype] and cosine(o, ora) > 0.99999
    ref = F.scaled_dot_product_attention(*(t.float().transpose(1, 2) for t in (q, k, v))).transpose(1, 2)
    assert rel_l2(o, np32(ref)) < 3e-2 and cosine(o, np32(ref)) > 0.9995
