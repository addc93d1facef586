"""The slice of the reference's ``DevicePolicy`` that configures this path
(``src/diffucore/runtime/__init__.py:55-132``): where the backbone runs, its
compute dtype, the attention backend and whether linears go W8A8."""

from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass
class DevicePolicy:
    device: torch.device
    compute_dtype: torch.dtype = torch.float16
    # "sdpa" (default, exact), "int8_turing" (the INT8 kernels: fp16/bf16,
    # self-attention), "fa2_turing" (never available on MI355X) or "auto".
    attention: str = "sdpa"
    # quantize the backbone's block linears to W8A8 at load
    int8: bool = False
    compile: bool = False

    def __post_init__(self):
        if self.attention not in ("sdpa", "auto", "fa2_turing", "int8_turing"):
            raise ValueError(
                f"attention must be 'sdpa', 'auto', 'fa2_turing', or 'int8_turing'; "
                f"got {self.attention!r}"
            )
