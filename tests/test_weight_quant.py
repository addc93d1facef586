"""Parity of the load-time weight quantizer (``quantize_weight``,
reference ``_int8.py:87-102``) with the oracle: rotate by the ConvRot
Hadamard as a float32 matmul, then the per-row quantizer
``clamp(rint(w / max(amax / 127, 1e-30)), -128, 127)``.

Group 0 has no matmul, so codes and scales are bit-exact. With the rotation
the two sides run float32 matmuls of different summation order (torch's BLAS,
numpy's), so a rotated value can differ in its last bits and a code sitting on
a rounding boundary can move by one step: the bar is every code within one
step, at most 0.5% of codes different, and scales within 16 float32 ulps. On the GPU, torch divides by the Python scalar
127.0 through its rounded reciprocal, so group-0 scales there are within one
ulp of the oracle's quotient rather than equal to it.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from diffucore_amd import _int8
from oracle import quant as OQ


def _weights(n: int, k: int, seed: int) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(n, k, generator=g) * 0.02
    w[:, torch.randperm(k, generator=g)[: max(1, k // 200)]] *= 20.0     # outlier input channels
    w[3] = 0.0                                                             # an all-zero row
    return w


def _compare(q, s, w, group, on_gpu=False):
    oq, os_ = OQ.quantize_weight(w.cpu().float().numpy(), group)
    q, s = q.cpu().numpy(), s.cpu().numpy()
    if group == 0 and on_gpu:
        # torch's GPU division by a Python scalar multiplies by the rounded
        # reciprocal, so amax / 127.0 can land one ulp from the CPU's quotient
        # (the reference runs the same op on the same device); codes then
        # differ only where a quotient sits on a rounding boundary
        assert np.all(np.abs(s - os_) <= np.spacing(os_))
        d = np.abs(q.astype(np.int32) - oq.astype(np.int32))
        assert d.max() <= 1 and (d != 0).mean() <= 1e-4
        return float((d != 0).mean())
    if group == 0:
        assert np.array_equal(q, oq) and np.array_equal(s, os_)
        return 0.0
    diff = np.abs(q.astype(np.int32) - oq.astype(np.int32))
    assert diff.max() <= 1
    rate = float((diff != 0).mean())
    assert rate <= 5e-3, rate
    ulp = np.spacing(np.maximum(np.abs(os_), np.float32(1e-30)))
    # the row maximum of a 256-term float32 sum taken in another order (BLAS
    # blocking; on the GPU also the reciprocal division): a few ulps
    assert (np.abs(s - os_) <= 16 * ulp).all(), (np.abs(s - os_) / ulp).max()
    assert s[3] == np.float32(1e-30) and not q[3].any()
    return rate


@pytest.mark.parametrize("group", [0, 256])
@pytest.mark.parametrize("shape", [(1280, 320), (640, 512), (96, 3072)])
def test_quantize_weight_matches_oracle_cpu(shape, group):
    n, k = shape
    if group and k % group:
        pytest.skip("K not a multiple of the group")
    w = _weights(n, k, 11 + n)
    q, s = _int8.quantize_weight(w, group)
    _compare(q, s, w, group)


def test_quantize_weight_rejects_a_wrong_group():
    with pytest.raises(ValueError):            # not a power of 4
        _int8.quantize_weight(torch.zeros(4, 96), 32)


@pytest.mark.gpu
@pytest.mark.parametrize("group", [0, 256])
def test_quantize_weight_matches_oracle_gpu(gpu, group):
    w = _weights(1280, 768, 7)
    q, s = _int8.quantize_weight(w.to(gpu), group)
    assert q.is_cuda and s.is_cuda
    _compare(q, s, w, group, on_gpu=True)
