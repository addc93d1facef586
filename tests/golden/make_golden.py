"""Writes the golden fixtures in this directory from the CPU oracle.

The reference stores no numeric golden vectors for this path, so the fixtures
freeze the oracle's outputs on small seeded inputs: tests/test_golden.py
checks that the oracle still reproduces them (on the CPU) and that the HIP
kernels reproduce them (on the GPU). Inputs are chosen so the fixtures also
hold the edge cases the reference tests exercise: outlier channels, an
all-zero row, quotients exactly on half-integers, ragged key counts and a
padded head dim.

    python tests/golden/make_golden.py
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent))

from oracle import attn as OA  # noqa: E402
from oracle import fp as OF  # noqa: E402
from oracle import gemm as OG  # noqa: E402
from oracle import quant as OQ  # noqa: E402


def bf16_values(x: np.ndarray) -> np.ndarray:
    return OF.round_bf16(np.asarray(x, np.float32))


def f16_values(x: np.ndarray) -> np.ndarray:
    return np.asarray(x, np.float32).astype(np.float16).astype(np.float32)


def quant_fixture(rng) -> dict:
    x0 = rng.standard_normal((24, 320)).astype(np.float32)
    x0[:, rng.permutation(320)[:2]] *= 20          # 0.5% outlier channels
    x0[5] = 0.0                                     # zero row: scale 1e-30, codes 0
    amax = np.float32(15.875)                       # s = 1/8: exact half-integer quotients
    x0[7, 0] = amax
    x0[7, 1:] = ((rng.integers(-127, 127, 319) + 0.5) / 8).astype(np.float32)
    q0, s0 = OQ.quantize_rows(x0)
    x1 = bf16_values(rng.standard_normal((16, 512)) * 3)
    q1, s1 = OQ.quantize_activation(x1, 256)
    return {"x_group0": x0, "q_group0": q0, "s_group0": s0, "x_rot": x1, "q_rot": q1, "s_rot": s1}


def gemm_fixture(rng) -> dict:
    M, N, K = 37, 72, 96
    q = rng.integers(-127, 128, (M, K)).astype(np.int8)
    w = rng.integers(-127, 128, (N, K)).astype(np.int8)
    sx = (rng.random(M) * 1e-2).astype(np.float32)
    sw = (rng.random(N) * 1e-3).astype(np.float32)
    bias = bf16_values(rng.standard_normal(N) * 0.5)
    acc = OG.int_mm(q, w)
    out = {"q": q, "w": w, "sx": sx, "sw": sw, "bias_bf16": bias, "acc": acc}
    for dt in ("f16", "bf16", "f32"):
        out[f"y_{dt}"] = OG.rescale(acc, sx, sw, None, dt)
        out[f"y_{dt}_bias"] = OG.rescale(acc, sx, sw, bias, dt)
    return out


def attn_fixture(rng, B, L, Lk, H, D, dtype) -> dict:
    rnd = bf16_values if dtype == "bf16" else f16_values
    q = rnd(rng.standard_normal((B, L, H, D)))
    k = rnd(rng.standard_normal((B, Lk, H, D)) + rng.standard_normal((H, D)) * 2)
    v = rnd(rng.standard_normal((B, Lk, H, D)))
    ksum = OA.k_colsum(k)
    ki, ks = OA.k_quantize(k, ksum)
    q8, qs = OA.q_quantize(q)
    o = OA.int8_attention(q, k, v, D ** -0.5, p_dtype=dtype, out_dtype=dtype)
    return {"q": q, "k": k, "v": v, "ksum": ksum, "k8": ki, "ks": ks, "q8": q8, "qs": qs, "o": o}


def main() -> None:
    rng = np.random.default_rng(20260101)
    np.savez_compressed(HERE / "quant.npz", **quant_fixture(rng))
    np.savez_compressed(HERE / "gemm.npz", **gemm_fixture(rng))
    np.savez_compressed(HERE / "attn_bf16_d128.npz", **attn_fixture(rng, 1, 70, 131, 2, 128, "bf16"))
    np.savez_compressed(HERE / "attn_f16_d40.npz", **attn_fixture(rng, 2, 33, 77, 2, 40, "f16"))
    for p in sorted(HERE.glob("*.npz")):
        print(p.name, p.stat().st_size)


if __name__ == "__main__":
    main()
