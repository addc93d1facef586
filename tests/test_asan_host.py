"""The C ABI's host-side argument checks under AddressSanitizer (CPU only, no
GPU call).

The library is built with AddressSanitizer on hipcc's host pass only
(``-Xarch_host -fsanitize=address``; the gfx950 device code is built as
usual and never runs here: the checks return before any launch), then a child
process with the sanitizer runtime preloaded makes each entry point's invalid
calls - null pointers, negative or oversized sizes, bad dtypes, misaligned
pointers and strides, a workspace too small, a call beyond the no-allocation
scratch, an in-place residual with its own row stride, the MFMA probe's bad
kinds and counts - and the valid empty calls that return before any HIP work.
Every call must return its error code, and any sanitizer report (a non-zero
exit, or "AddressSanitizer" on stderr) fails the test. The sources are the
library's own list (``diffucore_amd.build.SOURCES``)."""

from __future__ import annotations

import glob
import os
import shutil
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))
from diffucore_amd.build import CSRC, SOURCES  # noqa: E402  (the library's own source list)


def _asan_runtime() -> str | None:
    hits = glob.glob("/opt/rocm/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so")
    return hits[0] if hits else None


CHILD = r'''
import ctypes, sys
ctypes.CDLL(None).__asan_init                    # the sanitizer runtime is loaded
so = ctypes.CDLL(sys.argv[1])
P, I, I64, F, SZ = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float, ctypes.c_size_t
def sig(name, res, args):
    f = getattr(so, name); f.restype, f.argtypes = res, args; return f
last = sig("dc_last_error", ctypes.c_char_p, [])
qrows = sig("dc_quantize_rows", I, [P, I, I64, I64, I64, I, P, I64, P, P])
gemm = sig("dc_w8a8_gemm", I, [P, I64, P, I64, P, P, P, I, P, I, I64, I64, I64, I64, P, SZ, P])
gws = sig("dc_w8a8_gemm_workspace_bytes", SZ, [I64] * 5)
resc = sig("dc_rescale", I, [P, I64, P, P, P, I, P, I, I64, I64, I64, P])
actq = sig("dc_act_quantize_rows", I, [P, I64, I64, P, I64, I64, I, I, I64, I, P, I64, P, P])
lnq = sig("dc_ln_mod_quantize_rows", I, [P, I, I64, I64, I64, P, P, I, I64, I64, F, I, P, I64, P, P])
S3 = ctypes.POINTER(I64)
afwd = sig("dc_int8_attn_fwd", I, [P, P, P, P, I, I, I, I, I, I, S3, S3, S3, S3, F, P, SZ, P])
anoa = sig("dc_int8_attn_fwd_noalloc", I, [P, P, P, P, I, I, I, I, I, I, S3, S3, S3, S3, F, P])
aws = sig("dc_int8_attn_workspace_bytes", SZ, [I] * 5)
qq = sig("dc_int8_attn_quantize_q", I, [P, I, I, I, I, I, S3, P, P, P])
class Prob(ctypes.Structure):
    _fields_ = [("a", P), ("lda", I64), ("w", P), ("ldw", I64), ("sx", P), ("sw", P), ("bias", P), ("out", P),
                ("ldo", I64), ("M", I64)]
grp = sig("dc_w8a8_gemm_grouped", I, [P, I, I64, I64, I, I, P])
class Gate(ctypes.Structure):
    _fields_ = [("res", P), ("ldr", I64), ("gate", P)]
ggrp = sig("dc_w8a8_gemm_grouped_gated", I, [P, P, I, I64, I64, I, I, P])
gplan = sig("dc_w8a8_gemm_group_plan", I, [ctypes.POINTER(I64), I, I64, I64])
probe = sig("dc_mfma_probe", I, [I, I, I, I, P, P])
BF16, F16, F32 = 1, 0, 2
probs = (Prob * 4)(Prob(16, 512, 16, 512, 16, 16, None, 16, 3072, 64), Prob(16, 500, 16, 512, 16, 16, None, 16, 3072, 64),
                   Prob(16, 512, None, 512, 16, 16, None, 16, 3072, 64), Prob(16, 512, 16, 512, 16, 16, None, 16, 3072, 0))
Ms = (I64 * 4)(4096, 512, 0, 77)
gates = (Gate * 4)(Gate(16, 3072, 16), Gate(None, 3072, 16), Gate(16, 3000, 16), Gate(None, 0, None))
# a residual that is the output itself, with a row stride other than the output's
inplace_p = (Prob * 1)(Prob(16, 512, 16, 512, 16, 16, None, 4096, 3072, 64))
inplace_g = (Gate * 1)(Gate(4096, 3328, 16))
st = (I64 * 3)(8, 8, 8)
bad = (I64 * 3)(8, 12, 8)
checks = [
    (qrows(None, BF16, 4, 512, 512, 256, None, 512, None, None), 1),
    (qrows(16, BF16, 4, 512, 512, 3, 16, 512, 16, None), 1),
    (qrows(16, BF16, 0, 512, 512, 0, 16, 512, 16, None), 0),
    (qrows(16, 7, 4, 512, 512, 0, 16, 512, 16, None), 1),
    (gemm(16, 24, 16, 24, 16, 16, None, -1, 16, BF16, 8, 4, 8, 24, None, 0, None), 2),
    (gemm(16, 32, 16, 32, 16, 16, None, 7, 16, BF16, 8, 4, 8, 32, None, 0, None), 1),
    (gemm(None, 32, 16, 32, 16, 16, None, -1, 16, BF16, 8, 4, 8, 32, None, 0, None), 1),
    (gemm(16, 32, 16, 32, 16, 16, None, -1, 16, BF16, 8, (1 << 31) + 1, 8, 32, None, 0, None), 1),
    (gemm(16, 32, 16, 32, 16, 16, None, -1, 16, BF16, 8, 0, 8, 32, None, 0, None), 0),
    (resc(16, 4, 16, 16, None, -1, 16, BF16, 4, (1 << 31) + 5, 4, None), 1),
    (resc(None, 4, 16, 16, None, -1, 16, BF16, 4, 4, 4, None), 1),
    (actq(None, 0, 0, 16, 256, 256, 3, F16, 4, 256, 16, 256, 16, None), 1),
    (actq(None, 0, 0, 16, 512, 256, 9, F16, 4, 256, 16, 256, 16, None), 1),
    (actq(None, 0, 0, 16, 512, 300, 1, F16, 4, 256, 16, 300, 16, None), 2),
    (lnq(16, BF16, 4, 512, 512, 16, 16, BF16, 512, 4, -1.0, 256, 16, 512, 16, None), 1),
    (lnq(None, BF16, 4, 512, 512, 16, 16, BF16, 512, 4, 1e-6, 256, 16, 512, 16, None), 1),
    (afwd(16, 16, 16, 16, BF16, 1, 1, 4, 4, 36, st, st, st, st, 0.1, 16, 1 << 20, None), 2),
    (afwd(16, 16, 16, 16, F32, 1, 1, 4, 4, 64, st, st, st, st, 0.1, 16, 1 << 20, None), 1),
    (afwd(16, 16, 16, 16, BF16, 1, 1, 4, 4, 64, st, bad, st, st, 0.1, 16, 1 << 20, None), 2),
    (afwd(16, 16, 16, 16, BF16, 1, 1, 4, 4, 64, st, st, st, st, 0.1, 16, 8, None), 4),
    (afwd(16, 16, 16, 16, BF16, 1, 1, 4, 0, 64, st, st, st, st, 0.1, 16, 1 << 20, None), 1),
    (afwd(17, 16, 16, 16, BF16, 1, 1, 4, 4, 64, st, st, st, st, 0.1, 16, 1 << 20, None), 2),
    (anoa(16, 16, 16, 16, BF16, 8, 32, 8192, 8192, 128, st, st, st, st, 0.1, None), 4),
    (anoa(16, 16, 16, 16, BF16, 1, 1, 4, 4, 200, st, st, st, st, 0.1, None), 2),
    (qq(None, BF16, 1, 1, 4, 64, st, 16, 16, None), 1),
    (grp(probs, 0, 3072, 512, -1, BF16, None), 1),
    (grp(probs, 5, 3072, 512, -1, BF16, None), 1),
    (grp(probs, 2, 3072, 320, -1, BF16, None), 2),
    (grp(probs, 2, 3072, 512, -1, BF16, None), 2),
    (grp(ctypes.byref(probs, 2 * ctypes.sizeof(Prob)), 2, 3072, 512, -1, BF16, None), 1),
    (grp(ctypes.byref(probs, 3 * ctypes.sizeof(Prob)), 1, 3072, 512, -1, BF16, None), 0),
    (ggrp(probs, None, 1, 3072, 512, -1, BF16, None), 1),
    (ggrp(probs, gates, 1, 3072, 512, -1, 3, None), 1),
    (ggrp(ctypes.byref(probs, 0), ctypes.byref(gates, ctypes.sizeof(Gate)), 1, 3072, 512, -1, BF16, None), 1),
    (ggrp(ctypes.byref(probs, 0), ctypes.byref(gates, 2 * ctypes.sizeof(Gate)), 1, 3072, 512, -1, BF16, None), 1),
    (ggrp(ctypes.byref(probs, 3 * ctypes.sizeof(Prob)), ctypes.byref(gates, 3 * ctypes.sizeof(Gate)), 1, 3072, 512,
          -1, BF16, None), 0),
    (ggrp(inplace_p, inplace_g, 1, 3072, 512, -1, BF16, None), 1),
    (probe(2, 1, 1, 10, 16, None), 1),
    (probe(0, 2, 1, 10, 16, None), 1),
    (probe(0, 1, 3, 10, 16, None), 1),
    (probe(0, 1, 1, 0, 16, None), 1),
    (probe(1, 0, 2, 10, None, None), 1),
    (gplan(Ms, 4, 3072, 3072), 1),
    (gplan(Ms, 9, 3072, 3072), -1),
]
for i, (rc, want) in enumerate(checks):
    if rc != want:
        print(f"check {i}: rc {rc} != {want}: {last()}", file=sys.stderr)
        sys.exit(3)
    if rc:
        assert last(), i
assert gws(512, 3072, 12288, 12288, 12288) == 4 * 512 * 3072 * 4
assert aws(1, 1, 1, 1, 200) == 0
print("asan child ok", len(checks))
'''


@pytest.fixture(scope="module")
def asan_lib(tmp_path_factory):
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    rt = _asan_runtime()
    if not Path(hipcc).exists() or rt is None:
        pytest.skip("hipcc or the clang AddressSanitizer runtime is not available")
    tmp = tmp_path_factory.mktemp("asan")
    out = tmp / "libdiffucore_amd_asan.so"
    flags = ["--offload-arch=gfx950", "-O1", "-g", "-std=c++17", "-fPIC", "-Xarch_host", "-fsanitize=address",
             "-Xarch_host", "-fno-omit-frame-pointer", "-w"]
    srcs = tuple(SOURCES)
    # one compile per source, in parallel, then the link
    procs = [subprocess.Popen([hipcc, *flags, "-c", str(CSRC / s), "-o", str(tmp / f"{s}.o")],
                              stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True) for s in srcs]
    for s, p in zip(srcs, procs):
        _, err = p.communicate(timeout=900)
        if p.returncode != 0:
            pytest.fail(f"ASan host build of {s} failed:\n{err[-3000:]}")
    res = subprocess.run([hipcc, "--offload-arch=gfx950", "-shared", "-fPIC", "-Xarch_host", "-fsanitize=address",
                          "-shared-libsan", "-o", str(out), *[str(tmp / f"{s}.o") for s in srcs]],
                         capture_output=True, text=True, timeout=600)
    if res.returncode != 0:
        pytest.fail(f"ASan host link failed:\n{res.stderr[-3000:]}")
    return out, rt


def test_argument_checks_under_address_sanitizer(asan_lib):
    lib, rt = asan_lib
    env = dict(os.environ, LD_PRELOAD=rt, ASAN_OPTIONS="detect_leaks=0:abort_on_error=0:exitcode=23")
    res = subprocess.run([sys.executable, "-c", CHILD, str(lib)], capture_output=True, text=True, env=env,
                         timeout=300)
    assert "AddressSanitizer" not in res.stderr, res.stderr[-4000:]
    assert res.returncode == 0, (res.returncode, res.stderr[-4000:])
    assert "asan child ok" in res.stdout
