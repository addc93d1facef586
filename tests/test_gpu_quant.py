"""dc_quantize_rows on the GPU: int8 codes and scales bit-exact against the
oracle (reference ``_quantize_rows``, ``_int8.py:87-97``; butterfly rotation
``_int8.py:363-372`` in this build's documented order)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from diffucore_amd import _int8
from oracle import quant as OQ
from tests._util import np32

pytestmark = pytest.mark.gpu


def _x(M, K, dtype, seed, outliers=0.0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g)
    if outliers:
        idx = torch.randperm(K, generator=g)[: max(1, int(K * outliers))]
        x[:, idx] *= 20
    return x.to(dtype)


@pytest.mark.parametrize("M,K,dtype", [
    (8192, 320, torch.float32),      # SD1.5 cfg1 shape (x fp32)
    (333, 2048, torch.float16),
    (4608, 3072, torch.bfloat16),    # FLUX hidden
    (64, 15360, torch.bfloat16),     # FLUX linear2 input
    (130, 12288, torch.float16),
    (7, 40, torch.float16),
    (5, 100, torch.bfloat16),        # K % 8 != 0: generic kernel
    (1, 8, torch.float32),
])
def test_codes_bit_exact_group0(gpu, M, K, dtype):
    x = _x(M, K, dtype, seed=M + K, outliers=0.005)
    q, s = _int8.quantize_activation(x.to(gpu), 0)
    q_ref, s_ref = OQ.quantize_rows(np32(x))
    assert np.array_equal(s.cpu().numpy().view(np.uint32), s_ref.view(np.uint32))
    assert np.array_equal(q.cpu().numpy(), q_ref)


@pytest.mark.parametrize("M,K,dtype", [
    (4608, 3072, torch.bfloat16), (200, 15360, torch.bfloat16), (96, 12288, torch.float16),
    (33, 256, torch.float32), (9, 1280, torch.float16),
])
def test_codes_bit_exact_convrot(gpu, M, K, dtype):
    x = _x(M, K, dtype, seed=K, outliers=0.005)
    q, s = _int8.quantize_activation(x.to(gpu), 256)
    q_ref, s_ref = OQ.quantize_activation(np32(x), 256)
    assert np.array_equal(s.cpu().numpy().view(np.uint32), s_ref.view(np.uint32))
    assert np.array_equal(q.cpu().numpy(), q_ref)
    # against the matmul form of the rotation the codes may differ by one step
    q_mm, _ = OQ.quantize_rows(OQ.rotate_matmul(np32(x), 256))
    diff = np.abs(q.cpu().numpy().astype(np.int32) - q_mm.astype(np.int32))
    assert diff.max() <= 1 and (diff != 0).mean() < 1e-2


# shapes that select each kernel configuration: rows of 1/2/4/8 groups of 256
# reduced inside the wave (8-64 lanes), other multiples of 256 packed several
# rows per workgroup with 8/16/32/64-lane segment maxima combined in LDS (with
# batches that leave the last workgroup part-empty), up to 128 groups per row;
# rows that are not a multiple of 256 (short ones in the wave kernel, long
# ones in the generic kernel)
CONFIG_SHAPES = [
    (333, 768, 256, torch.bfloat16), (1000, 1280, 0, torch.float16), (999, 1536, 256, torch.float16),
    (777, 3072, 0, torch.bfloat16), (300, 5120, 256, torch.float16), (129, 12288, 0, torch.bfloat16),
    (65, 15360, 256, torch.float32), (3, 32512, 256, torch.bfloat16), (5, 32768, 0, torch.float16),
    (64, 2304, 0, torch.float16), (50, 2600, 0, torch.bfloat16), (100, 700, 0, torch.float16),
    (4097, 512, 256, torch.bfloat16), (4097, 1024, 0, torch.float16), (1025, 2048, 256, torch.bfloat16),
    # rows of 36 / 44 / 60 groups (288 / 352 / 480 lanes): one row per workgroup of 320 / 384 / 512
    # threads instead of two rows in a workgroup above 512 threads
    (301, 9216, 256, torch.bfloat16), (77, 11264, 0, torch.float16), (1001, 15360, 256, torch.bfloat16),
]


@pytest.mark.parametrize("M,K,group,dtype", CONFIG_SHAPES)
def test_every_kernel_configuration(gpu, M, K, group, dtype):
    x = _x(M, K, dtype, seed=M ^ K, outliers=0.005)
    q, s = _int8.quantize_activation(x.to(gpu), group)
    q_ref, s_ref = OQ.quantize_activation(np32(x), group)
    assert np.array_equal(s.cpu().numpy().view(np.uint32), s_ref.view(np.uint32))
    assert np.array_equal(q.cpu().numpy(), q_ref)


@pytest.mark.parametrize("col0", [48, 44])   # 16-byte aligned rows (vector kernel) / not (generic kernel)
def test_zero_rows_and_strided_input(gpu, col0):
    x = torch.randn(16, 600, dtype=torch.float16)
    x[3] = 0
    xd = x.to(gpu)
    xs = xd[:, col0:col0 + 512]           # ldx = 600, K = 512
    q, s = _int8.quantize_activation(xs, 0)
    q_ref, s_ref = OQ.quantize_rows(np32(x[:, col0:col0 + 512]))
    assert np.array_equal(q.cpu().numpy(), q_ref)
    assert np.array_equal(s.cpu().numpy(), s_ref)
    assert s[3].item() == np.float32(1e-30) and (q[3] == 0).all()


def _steps(x: np.ndarray, k: np.ndarray) -> np.ndarray:
    """x moved by k float32 ulps (k in -2..2)."""
    out = x.copy()
    for _ in range(2):
        up, dn = k > 0, k < 0
        out[up] = np.nextafter(out[up], np.float32(np.inf))
        out[dn] = np.nextafter(out[dn], np.float32(-np.inf))
        k = k - np.sign(k)
    return out


@pytest.mark.parametrize("K", [256, 1280, 3072, 15360])
def test_codes_at_and_around_ties(gpu, K):
    """Quotients x / s on half-integers and 1-2 ulps either side, where a
    reciprocal-based rounding would part from rint(x / s): element 0 of each
    row fixes amax, the others are fl(h * s) for half-integers h, nudged."""
    rng = np.random.default_rng(K)
    rows = 64
    x = np.zeros((rows, K), np.float32)
    for r in range(rows):
        amax = np.float32(rng.uniform(0.25, 8.0)) if r else np.float32(15.875)   # row 0: s = 1/8 exactly
        s = np.float32(amax / np.float32(127.0))
        h = (rng.integers(-127, 127, K - 1) + 0.5).astype(np.float32)
        xr = (h * s).astype(np.float32)
        if r % 2:
            xr = _steps(xr, rng.integers(-2, 3, K - 1))
        x[r, 0], x[r, 1:] = amax, np.clip(xr, -amax, amax)
    q, sc = _int8.quantize_activation(torch.from_numpy(x).to(gpu), 0)
    q_ref, s_ref = OQ.quantize_rows(x)
    assert np.array_equal(sc.cpu().numpy().view(np.uint32), s_ref.view(np.uint32))
    assert np.array_equal(q.cpu().numpy(), q_ref)


@pytest.mark.parametrize("K", [256, 3072, 12288])
def test_rotated_codes_at_exact_ties(gpu, K):
    """Inputs whose rotation is exact and lands on m / 16 with max 254 / 16,
    so s = 1/8 and every odd m is a tie m / 2 (ties to even): x = z H / 16 for
    integer z, which the butterfly inverts exactly."""
    rng = np.random.default_rng(K)
    G = K // 256
    z = rng.integers(-20, 21, (8, K)).astype(np.float64)
    z[:, ::256] = 254                       # the max of every row: 254 / 16
    H = OQ.hadamard(256).astype(np.float64) * 16          # +-1 entries
    x = (z.reshape(8, G, 256) @ H / 256).reshape(8, K).astype(np.float32)
    y = OQ.rotate_butterfly(x, 256)
    assert np.array_equal(y, (z / 16).astype(np.float32))   # the rotation is exact here
    q, sc = _int8.quantize_activation(torch.from_numpy(x).to(gpu), 256)
    q_ref, s_ref = OQ.quantize_activation(x, 256)
    assert (s_ref == np.float32(0.125)).all()
    assert np.array_equal(sc.cpu().numpy(), s_ref)
    assert np.array_equal(q.cpu().numpy(), q_ref)


def test_empty_batch(gpu):
    q, s = _int8.quantize_activation(torch.zeros(0, 256, device=gpu, dtype=torch.bfloat16), 256)
    assert q.shape == (0, 256) and s.shape == (0,)
