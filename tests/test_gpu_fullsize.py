"""The hot path at the benchmark's full shapes, through properties that hold
at any size (the oracle covers smaller sizes bit for bit):

* int32 GEMM: row and column checksums against exact int64 identities,
  sum_n C[m, n] = A[m] . (sum_n W[n]) and sum_m C[m, n] = (sum_m A[m]) . W[n],
  for every kernel plan the FLUX step uses;
* fused epilogue: equal to the reference's unfused rescale(int_mm()) ops
  (_int8.py:322-323) on the exact int32 result;
* activation quantize: codes and scales bit-exact against the oracle;
* attention: the reference's bar against float32 SDPA
  (tests/test_attention_dispatch.py:212-213), a value tensor constant along
  the keys comes back exactly (softmax rows sum to one), and repeated calls
  agree bit for bit.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from diffucore_amd import _attention as A
from diffucore_amd import _int8
from oracle import quant as OQ
from tests._util import np32

pytestmark = pytest.mark.gpu

# FLUX 1024^2 linears (M, N, K): single linear1 / linear2, img qkv / MLP up / MLP down, txt MLP down
FLUX_GEMMS = [(4608, 21504, 3072), (4608, 3072, 15360), (4096, 9216, 3072), (4096, 12288, 3072),
              (4096, 3072, 12288), (512, 3072, 12288)]


def _operands(M, N, K, gpu, seed):
    g = torch.Generator(device=gpu).manual_seed(seed)
    a = torch.randint(-127, 128, (M, K), generator=g, device=gpu, dtype=torch.int8)
    w = torch.randint(-127, 128, (N, K), generator=g, device=gpu, dtype=torch.int8)
    return a, w


@pytest.mark.parametrize("M,N,K", FLUX_GEMMS)
def test_int_mm_checksums(gpu, M, N, K):
    a, w = _operands(M, N, K, gpu, M + N + K)
    c = _int8.int_mm(a, w)
    wsum = w.long().sum(0)                       # [K]
    assert torch.equal(c.long().sum(1), (a.long() * wsum).sum(1))
    asum = a.long().sum(0)                       # [K]
    assert torch.equal(c.long().sum(0), (w.long() * asum).sum(1))


@pytest.mark.parametrize("M,N,K", FLUX_GEMMS[:3])
def test_fused_epilogue_equals_unfused_ops(gpu, M, N, K):
    a, w = _operands(M, N, K, gpu, 7 * M + N)
    g = torch.Generator(device=gpu).manual_seed(3)
    sx = torch.rand(M, generator=g, device=gpu) * 1e-2
    sw = torch.rand(N, generator=g, device=gpu) * 1e-3
    bias = (torch.randn(N, generator=g, device=gpu) * 0.02).to(torch.bfloat16)
    lin = _int8.Int8Linear(K, N, bias=True, group=0, device=gpu)
    lin.weight.copy_(w)
    lin.scale_bits.copy_(sw.view(torch.int32))
    lin.bias = torch.nn.Parameter(bias, requires_grad=False)
    y = lin.matmul_quantized(a, sx, torch.bfloat16)
    acc = _int8.int_mm(a, w)
    ref = (acc.float() * (sx[:, None] * sw[None, :])).to(torch.bfloat16) + bias
    assert torch.equal(y, ref)


@pytest.mark.parametrize("M,K", [(4608, 3072), (4096, 12288), (4608, 15360)])
def test_quantize_bit_exact_at_flux_shapes(gpu, M, K):
    g = torch.Generator().manual_seed(K)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    q, s = _int8.quantize_activation(x.to(gpu), 256)
    q_ref, s_ref = OQ.quantize_activation(np32(x), 256)
    assert np.array_equal(s.cpu().numpy().view(np.uint32), s_ref.view(np.uint32))
    assert np.array_equal(q.cpu().numpy(), q_ref)


def _flux_qkv(gpu, seed=0):
    g = torch.Generator(device=gpu).manual_seed(seed)
    q, k, v = (torch.randn(1, 24, 4608, 128, generator=g, device=gpu).to(torch.bfloat16) for _ in range(3))
    return q, k, v


def test_flux_attention_against_fp32_sdpa(gpu):
    q, k, v = _flux_qkv(gpu)
    out = A.attention_bhld(q, k, v, "int8_turing").float()
    ref = F.scaled_dot_product_attention(q.float(), k.float(), v.float()).transpose(1, 2).reshape(1, 4608, -1)
    a, b = out.flatten(), ref.flatten()
    rel = ((a - b).norm() / b.norm()).item()
    cos = (a @ b / (a.norm() * b.norm())).item()
    assert rel < 3e-2 and cos > 0.9995, (rel, cos)


def test_flux_attention_constant_values_and_repeatability(gpu):
    q, k, _ = _flux_qkv(gpu, 1)
    c = torch.randn(24, 128, device=gpu).to(torch.bfloat16)
    v = c[None, :, None, :].expand(1, 24, 4608, 128).contiguous()
    out = A.attention_bhld(q, k, v, "int8_turing").reshape(1, 4608, 24, 128)
    assert torch.equal(out, c[None, None].expand_as(out))
    _, _, v2 = _flux_qkv(gpu, 2)
    o1 = A.attention_bhld(q, k, v2, "int8_turing")
    o2 = A.attention_bhld(q, k, v2, "int8_turing")
    assert torch.equal(o1, o2)
