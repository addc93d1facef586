"""The slice of the reference's ``DevicePolicy`` that configures this path
(``src/diffucore/runtime/__init__.py:55-132``): where the backbone runs, its
compute dtype, the attention backend and whether linears go W8A8."""

from __future__ import annotations

from dataclasses import dataclass

import torch


ATTENTION_BACKENDS = ("sdpa", "auto", "fa2_turing", "int8_turing")


@dataclass
class DevicePolicy:
    device: torch.device
    compute_dtype: torch.dtype = torch.float16
    # one of ATTENTION_BACKENDS: "sdpa" is exact and the default;
    # "int8_turing" runs self-attention on the INT8 kernels (fp16 / bf16);
    # "fa2_turing" never runs on MI355X; "auto" picks the best that can
    attention: str = "sdpa"
    # W8A8-quantize the backbone's block linears when loading
    int8: bool = False
    compile: bool = False

    def __post_init__(self):
        if self.attention not in ATTENTION_BACKENDS:
            allowed = ", ".join(repr(b) for b in ATTENTION_BACKENDS)
            raise ValueError(f"attention must be one of {allowed}; got {self.attention!r}")
