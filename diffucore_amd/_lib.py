"""ctypes binding of ``libdiffucore_amd.so`` (C ABI in include/diffucore_amd.h).

The library links ``libamdhip64.so.7``; it is opened after ``import torch`` so
the dynamic loader resolves it to the HIP runtime torch already loaded, and
raw device pointers and ``hipStream_t`` handles from torch are valid in it.
"""

from __future__ import annotations

import contextlib
import ctypes
import functools
from pathlib import Path

import torch  # noqa: F401  (loads torch's HIP runtime first)

LIB_PATH = Path(__file__).resolve().parent / "libdiffucore_amd.so"

F16, BF16, F32, I32, NONE = 0, 1, 2, 3, -1
ABI_VERSION = 13

_DTYPE = {torch.float16: F16, torch.bfloat16: BF16, torch.float32: F32, torch.int32: I32}

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I = ctypes.c_int
_SIGS = {
    "dc_last_error": (ctypes.c_char_p, []),
    "dc_abi_version": (_I, []),
    "dc_quantize_rows": (_I, [_P, _I, _I64, _I64, _I64, _I, _P, _I64, _P, _P]),
    "dc_w8a8_gemm": (_I, [_P, _I64, _P, _I64, _P, _P, _P, _I, _P, _I, _I64, _I64, _I64, _I64, _P, ctypes.c_size_t, _P]),
    "dc_w8a8_gemm_workspace_bytes": (ctypes.c_size_t, [_I64, _I64, _I64, _I64, _I64]),
    "dc_w8a8_gemm_plan": (_I, [_I64, _I64, _I64, _I64, _I64]),
    "dc_w8a8_gemm_grouped": (_I, [_P, _I, _I64, _I64, _I, _I, _P]),
    "dc_w8a8_gemm_grouped_gated": (_I, [_P, _P, _I, _I64, _I64, _I, _I, _P]),
    "dc_w8a8_gemm_group_plan": (_I, [ctypes.POINTER(_I64), _I, _I64, _I64]),
    "dc_rescale": (_I, [_P, _I64, _P, _P, _P, _I, _P, _I, _I64, _I64, _I64, _P]),
    "dc_ln_mod_quantize_rows": (_I, [_P, _I, _I64, _I64, _I64, _P, _P, _I, _I64, _I64, ctypes.c_float, _I, _P, _I64, _P, _P]),
    "dc_act_quantize_rows": (_I, [_P, _I64, _I64, _P, _I64, _I64, _I, _I, _I64, _I, _P, _I64, _P, _P]),
    "dc_qk_norm_rope": (_I, [_I, _I64, _I64, _I64, _I64, _I, ctypes.c_float,
                             _P, ctypes.POINTER(_I64), _P, _P, ctypes.POINTER(_I64), _P, _I,
                             _P, _I64, _I64, _P, ctypes.POINTER(_I64), _P, ctypes.POINTER(_I64),
                             _P, ctypes.POINTER(_I64), _P, ctypes.POINTER(_I64), _P]),
    "dc_int8_attn_workspace_bytes": (ctypes.c_size_t, [_I, _I, _I, _I, _I]),
    "dc_int8_attn_plan": (_I, [_I, _I, _I, _I, _I, _I] + [ctypes.POINTER(_I)] * 3),
    "dc_int8_attn_fwd": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _I,
                              ctypes.POINTER(_I64), ctypes.POINTER(_I64), ctypes.POINTER(_I64),
                              ctypes.POINTER(_I64), ctypes.c_float, _P, ctypes.c_size_t, _P]),
    "dc_int8_attn_fwd_noalloc": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _I,
                                      ctypes.POINTER(_I64), ctypes.POINTER(_I64), ctypes.POINTER(_I64),
                                      ctypes.POINTER(_I64), ctypes.c_float, _P]),
    "dc_int8_attn_quantize_q": (_I, [_P, _I, _I, _I, _I, _I, ctypes.POINTER(_I64), _P, _P, _P]),
    "dc_mfma_probe": (_I, [_I, _I, _I, _I, _P, _P]),
    "dc_mfma_probe_units": (_I, []),
}
SYMBOLS = tuple(_SIGS)

MAX_GROUP = 4   # DC_GEMM_MAX_GROUP


class GemmProblem(ctypes.Structure):
    """``dc_gemm_problem``: one problem of ``dc_w8a8_gemm_grouped``."""
    _fields_ = [("a", _P), ("lda", _I64), ("w", _P), ("ldw", _I64), ("sx", _P), ("sw", _P), ("bias", _P),
                ("out", _P), ("ldo", _I64), ("M", _I64)]


class GemmGate(ctypes.Structure):
    """``dc_gemm_gate``: one problem's residual and gate for
    ``dc_w8a8_gemm_grouped_gated``."""
    _fields_ = [("res", _P), ("ldr", _I64), ("gate", _P)]

_load_error = ""


@functools.cache
def lib():
    """The loaded library, or None (the reason is in :func:`load_error`)."""
    global _load_error
    if not LIB_PATH.exists():
        _load_error = f"{LIB_PATH.name} is not built (run python -m diffucore_amd.build)"
        return None
    try:
        so = ctypes.CDLL(str(LIB_PATH))
    except OSError as e:
        _load_error = f"cannot load {LIB_PATH.name}: {e}"
        return None
    for name, (res, args) in _SIGS.items():
        fn = getattr(so, name)
        fn.restype, fn.argtypes = res, args
    if so.dc_abi_version() != ABI_VERSION:
        _load_error = f"{LIB_PATH.name} ABI {so.dc_abi_version()} != {ABI_VERSION}: rebuild it"
        return None
    return so


def load_error() -> str:
    return "" if lib() is not None else _load_error


def require():
    """The library, or a loud RuntimeError: the product path has no fallback."""
    so = lib()
    if so is None:
        raise RuntimeError(f"diffucore_amd: HIP kernels unavailable: {_load_error}")
    return so


def dtype_code(dt: torch.dtype) -> int:
    try:
        return _DTYPE[dt]
    except KeyError:
        raise TypeError(f"diffucore_amd: unsupported dtype {dt}") from None


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = require().dc_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed (code {rc}): {msg}")


# torch's raw current-stream query (the handle only, no Stream object: about
# 0.1 us against 3 us per call); the public API where it is missing
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_ptr(device: torch.device) -> int:
    """The ``hipStream_t`` of torch's current stream on ``device``."""
    if _raw_stream is not None:
        return _raw_stream(torch.cuda.current_device() if device.index is None else device.index)
    return torch.cuda.current_stream(device).cuda_stream


def device_ctx(device: torch.device):
    """``torch.cuda.device(device)`` when ``device`` is not the current one,
    else a no-op context (entering torch's costs about 3 us per call). A
    device that is not a GPU raises: the kernels take device pointers only."""
    if device.type != "cuda":
        raise RuntimeError(f"diffucore_amd: the HIP kernels take GPU tensors (got a {device} tensor)")
    if device.index is None or device.index == torch.cuda.current_device():
        return contextlib.nullcontext()
    return torch.cuda.device(device)


_I64X3 = ctypes.c_int64 * 3


def strides3(t: torch.Tensor):
    """The first three strides of ``t`` as a C ``int64_t[3]``."""
    s = t.stride()
    return _I64X3(s[0], s[1], s[2])


@functools.cache
def device_is_gfx950(index: int) -> bool:
    try:
        name = torch.cuda.get_device_properties(index).gcnArchName
    except Exception:  # noqa: BLE001  no device / not ROCm
        return False
    return name.split(":")[0] == "gfx950"
