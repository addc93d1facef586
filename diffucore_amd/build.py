"""Build ``libdiffucore_amd.so`` (the gfx950 kernels behind the C ABI in
``include/diffucore_amd.h``) in-tree with hipcc.

Run ``python -m diffucore_amd.build``. The library sits next to this file so it
travels with the source tree; it is loaded by :mod:`diffucore_amd._lib`.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
LIB = PKG / "libdiffucore_amd.so"
SOURCES = ["quant.hip", "qknorm.hip", "gemm.hip", "attn.hip", "calib.hip", "capi.cpp"]
ARCH = "gfx950"

FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-shared", "-fPIC",
    # reproducible float32 arithmetic: only explicit fmaf() contracts
    "-ffp-contract=off",
    # no packed-fp32 VALU instructions
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # register-staged tile arrays stay in registers: never let the backend
    # move a private array into spare LDS (it adds an LDS round trip per tile)
    "-mllvm", "-disable-promote-alloca-to-lds",
    "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (needs ROCm)")


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{res.stderr[-4000:]}")


def build(verbose: bool = False) -> Path:
    """Compile every HIP source into ``LIB`` (always recompiles): one object
    per source, compiled in parallel, then linked."""
    with tempfile.TemporaryDirectory(prefix="dc_build_") as tmpdir:
        objs = [str(Path(tmpdir) / (Path(s).stem + ".o")) for s in SOURCES]
        compile_flags = [f for f in FLAGS if f != "-shared"]
        cmds = [[hipcc(), *compile_flags, "-c", "-o", o, str(CSRC / s)] for s, o in zip(SOURCES, objs)]
        workers = max(1, min(len(cmds), os.cpu_count() or 1, 16))
        with ThreadPoolExecutor(max_workers=workers) as pool:
            for f in [pool.submit(_run, c, verbose) for c in cmds]:
                f.result()
        tmp = LIB.with_suffix(".so.tmp")
        _run([hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *objs], verbose)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    out = build(verbose="-v" in sys.argv)
    print(f"built {out}")
