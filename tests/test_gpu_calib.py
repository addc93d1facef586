"""dc_mfma_probe on the GPU: the MFMA calibration behind bench.py's measured
ceiling runs every configuration, writes its per-wave sink, and reports a
rate between a tenth of the published peak and the peak (int8 5.0 POP/s,
bf16 2.5 PFLOP/s), so a broken launch or a mis-counted workload shows."""

from __future__ import annotations

import pytest
import torch

import bench

pytestmark = pytest.mark.gpu


def test_mfma_probe_rates_within_the_peak(gpu):
    torch.cuda.set_device(gpu)
    out = bench.mfma_ceiling(iters=20000)
    assert out["units"] > 0
    for key, rate in out.items():
        if key.startswith("int8"):
            assert 500 < rate <= 1.05 * 5000, (key, rate)
        elif key.startswith("bf16"):
            assert 250 < rate <= 1.05 * 2500, (key, rate)
    print("[calib]", {k: v for k, v in out.items() if k not in ("what",)})
