"""The quantize kernel forms each int8 code without a division: Markstein's
quotient correction (q = x * fl(1/s); r = fma(-q, s, x); fma(r, fl(1/s), q)
is fl(x / s) whenever nothing underflows) on the butterfly's 16-fold values.
This checks that form on the CPU against rint of an IEEE float32 division
(the reference's ``torch.round(x / scale)``, ``_int8.py:87-97``) over random
and adversarial quotients (within 3 ulps of every half-integer code
boundary), and that two plausible mistakes in it (no correction; the residual
taken against the unscaled s) are caught. The GPU tests compare the kernel's
codes with the oracle's division bit for bit on top of this.
"""

from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import pytest

SRC = Path(__file__).resolve().parent / "markstein_check.c"

pytestmark = pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    exe = tmp_path_factory.mktemp("mk") / "markstein_check"
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-fno-fast-math", "-o", str(exe), str(SRC), "-lm"],
                   check=True)
    return exe


def _run(exe, scales, mode):
    return subprocess.run([str(exe), str(scales), str(mode)], capture_output=True, text=True, timeout=120)


def test_kernel_codes_equal_ieee_division(checker):
    out = _run(checker, 20000, 1)
    assert out.returncode == 0, out.stdout
    assert "code mismatches 0" in out.stdout
    assert int(out.stdout.split("tested ")[1].split()[0]) > 50_000_000


@pytest.mark.parametrize("mode", [0, 2])
def test_planted_mistakes_are_caught(checker, mode):
    out = _run(checker, 500, mode)
    assert out.returncode == 1 and "mismatch:" in out.stdout
