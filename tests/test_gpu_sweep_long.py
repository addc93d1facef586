"""Long seeded sweeps (about a minute on one MI355X).

The same checks as ``tests/test_gpu_sweep.py`` over more random cases, plus
large shapes that take the DMA-fed kernels, multi-round grids, stream-K
attention plans and split-K GEMMs:

* W8A8 linear, large: activation codes and scales bit-exact against the
  oracle's quantizer; the int32 products against ``torch._int_mm`` (the
  vendor GEMM the reference's ``int_mm`` calls, ``_int8.py:200-207``) and,
  through the oracle's ``rescale`` (``:313-323``), the fused output bit for
  bit.
* INT8 attention, large: K codes, block scales, key sums and Q codes
  bit-exact against the oracle over the whole input; the output against the
  oracle's restatement on 48 random query rows (each row depends only on its
  own query and the whole K / V) and against float32 SDPA on every row.

Each case prints its parameters before it runs.
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
from tests.test_gpu_sweep import _attn_cases, _linear_cases

pytestmark = pytest.mark.gpu

ORACLE_REL = {torch.float16: 1e-3, torch.bfloat16: 4e-3}
_FLOATS = [torch.float16, torch.bfloat16, torch.float32]


def _big_linear_cases(n: int, seed: int):
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        group = int(rng.choice([0, 256]))
        K = int(rng.integers(1, 65)) * 256 if group else int(rng.integers(1, 513)) * 8
        M = int(rng.choice([4096, 4608, 8192, int(rng.integers(32, 6000))]))
        N = int(rng.choice([3072, 9216, 12288, 21504, int(rng.integers(1, 2800)) * 8]))
        dtype = _FLOATS[int(rng.integers(0, 3))]
        bias = [None, dtype, torch.float32][int(rng.integers(0, 3))]
        cases.append((i, M, N, K, group, dtype, bias))
    return cases


def _big_attn_cases(n: int, seed: int):
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        B, H = int(rng.integers(1, 3)), int(rng.integers(1, 33))
        Lq = int(rng.choice([4096, 4608, int(rng.integers(1, 6000))]))
        Lk = int(rng.choice([77, 4096, 4608, int(rng.integers(1, 6000))]))
        D = int(rng.choice([40, 64, 128, int(rng.integers(1, 17)) * 8]))
        dtype = [torch.float16, torch.bfloat16][int(rng.integers(0, 2))]
        cases.append((i, B, H, Lq, Lk, D, dtype))
    return cases


def _layer(K, N, group, bias_dtype, seed, gpu):
    g = torch.Generator().manual_seed(seed)
    lin = nn.Linear(K, N, bias=bias_dtype is not None)
    with torch.no_grad():
        lin.weight.copy_(torch.randn(N, K, generator=g) * 0.02)
        if bias_dtype is not None:
            lin.bias.copy_(torch.randn(N, generator=g) * 0.5)
    layer = _int8.Int8Linear.from_linear(lin, group, device=gpu)
    if bias_dtype is not None:
        layer.bias = nn.Parameter(layer.bias.to(bias_dtype), requires_grad=False)
    return layer, g


def _activation(M, K, dtype, g):
    x = torch.randn(M, K, generator=g)
    x[:, torch.randperm(K, generator=g)[: max(1, K // 200)]] *= 20    # outlier channels
    return x.to(dtype)


@pytest.mark.parametrize("i,M,N,K,group,dtype,bias_dtype", _linear_cases(160, 31337))
def test_linear_long_sweep_small(gpu, i, M, N, K, group, dtype, bias_dtype):
    print(f"[long sweep] linear {i}: M {M} N {N} K {K} group {group} {DT[dtype]} bias {bias_dtype}", flush=True)
    layer, g = _layer(K, N, group, bias_dtype, 5000 + i, gpu)
    x = _activation(M, K, dtype, g)
    with torch.no_grad():
        y = layer(x.to(gpu))
    q_ref, s_ref = OQ.quantize_activation(np32(x), group)
    b = None if bias_dtype is None else np32(layer.bias)
    ref = OG.rescale(OG.int_mm(q_ref, layer.weight.cpu().numpy()), s_ref, layer.scale.cpu().numpy(), b, DT[dtype])
    assert np.array_equal(np32(y).view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("i,M,N,K,group,dtype,bias_dtype", _big_linear_cases(24, 8675309))
def test_linear_long_sweep_large(gpu, i, M, N, K, group, dtype, bias_dtype):
    print(f"[long sweep] large linear {i}: M {M} N {N} K {K} group {group} {DT[dtype]} bias {bias_dtype}",
          flush=True)
    layer, g = _layer(K, N, group, bias_dtype, 6000 + i, gpu)
    x = _activation(M, K, dtype, g)
    xd = x.to(gpu)
    q, s = _int8.quantize_activation(xd, group)
    q_ref, s_ref = OQ.quantize_activation(np32(x), group)
    assert np.array_equal(q.cpu().numpy(), q_ref)
    assert np.array_equal(s.cpu().numpy().view(np.uint32), s_ref.view(np.uint32))
    with torch.no_grad():
        y = layer(xd)
    acc = torch._int_mm(q, layer.weight.t())
    assert torch.equal(_int8.int_mm(q, layer.weight), acc)
    b = None if bias_dtype is None else np32(layer.bias)
    ref = OG.rescale(acc.cpu().numpy(), s_ref, layer.scale.cpu().numpy(), b, DT[dtype])
    assert np.array_equal(np32(y).view(np.uint32), ref.view(np.uint32))


def _attn_inputs(B, H, Lq, Lk, D, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, Lq, H, D, generator=g).to(dtype)
    k = (torch.randn(B, Lk, H, D, generator=g) + torch.randn(D, generator=g) * 2).to(dtype)
    v = torch.randn(B, Lk, H, D, generator=g).to(dtype)
    return q, k, v


def _check_attention(gpu, B, H, Lq, Lk, D, dtype, seed, rows=None):
    q, k, v = _attn_inputs(B, H, Lq, Lk, D, dtype, seed)
    qd, kd, vd = q.to(gpu), k.to(gpu), v.to(gpu)
    ws = torch.empty(A.workspace_bytes(B, H, Lq, Lk, D), device=gpu, dtype=torch.uint8)
    out = A.int8_attention(qd, kd, vd, D ** -0.5, workspace=ws)
    views = A.workspace_views(ws, B, H, Lq, Lk, D)
    ksum = OA.k_colsum(np32(k))
    assert np.array_equal(views["ksum"].cpu().numpy().view(np.uint32), ksum.view(np.uint32))
    ki, ks = OA.k_quantize(np32(k), ksum)
    assert np.array_equal(views["ks"].cpu().numpy().view(np.uint32), ks.view(np.uint32))
    assert np.array_equal(views["k8"][..., :D].cpu().numpy(), ki)
    q8, qs = A.quantize_q(qd)
    q8_ref, qs_ref = OA.q_quantize(np32(q))
    assert np.array_equal(q8[:, :, :Lq, :D].cpu().numpy(), q8_ref)
    assert np.array_equal(qs[:, :, :Lq].cpu().numpy().view(np.uint32), qs_ref.view(np.uint32))
    o = np32(out)
    assert out.shape == (B, Lq, H, D) and np.isfinite(o).all()
    sel = slice(None) if rows is None else rows
    ora = OA.int8_attention(np32(q)[:, sel], np32(k), np32(v), D ** -0.5, DT[dtype], DT[dtype])
    r, c = rel_l2(o[:, sel], ora), cosine(o[:, sel], ora)
    assert r < ORACLE_REL[dtype] and c > 0.99999, (r, c)
    ref = F.scaled_dot_product_attention(*(t.float().transpose(1, 2) for t in (qd, kd, vd))).transpose(1, 2)
    r, c = rel_l2(o, np32(ref)), cosine(o, np32(ref))
    assert r < 3e-2 and c > 0.9995, (r, c)


@pytest.mark.parametrize("i,B,H,Lq,Lk,D,dtype", _attn_cases(160, 4711))
def test_attention_long_sweep_small(gpu, i, B, H, Lq, Lk, D, dtype):
    print(f"[long sweep] attention {i}: B {B} H {H} Lq {Lq} Lk {Lk} D {D} {DT[dtype]}", flush=True)
    _check_attention(gpu, B, H, Lq, Lk, D, dtype, 7000 + i)


@pytest.mark.parametrize("i,B,H,Lq,Lk,D,dtype", _big_attn_cases(32, 271828))
def test_attention_long_sweep_large(gpu, i, B, H, Lq, Lk, D, dtype):
    print(f"[long sweep] large attention {i}: B {B} H {H} Lq {Lq} Lk {Lk} D {D} {DT[dtype]} "
          f"plan {A.attn_plan(B, H, Lq, Lk, D, dtype)}", flush=True)
    rows = np.sort(np.random.default_rng(i).choice(Lq, size=min(Lq, 48), replace=False))
    _check_attention(gpu, B, H, Lq, Lk, D, dtype, 8000 + i, rows)
