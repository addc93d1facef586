"""diffucore_amd: diffucore's quantized denoiser hot path (INT8 flash attention
and W8A8 linears) as hand-written gfx950 (MI355X) HIP kernels behind a C ABI,
with the reference's Python operator surface on top."""

from ._attention import (attention_bhld, attention_blhd, fa2_turing_available, int8_attention,
                         int8_turing_available, resolve_attention_backend, set_attention_backend)
from ._int8 import (GROUP, Int8Embedding, Int8Linear, act_quantize, adopt_int8_embedding, adopt_int8_layers,
                    dequantize_linears, dequantize_weight, fuse_linears, geglu_quantize, gelu_quantize,
                    int8_fast_available, int8_geglu_ff,
                    int8_layers, int8_mlp, int_mm, linear_group, ln_mod_quantize, matmul_quantized_gated,
                    matmul_quantized_group, lora_seed, quantize_activation,
                    quantize_linears, quantize_weight, rescale, scaled_mm, shared_qkv)
from ._qknorm import flux_qk_norm_rope, norm_rope, qk_norm_rope, qk_ok, set_fused_glue
from .runtime import DevicePolicy

__all__ = sorted([
    "GROUP", "DevicePolicy", "Int8Embedding", "Int8Linear", "act_quantize", "adopt_int8_embedding",
    "adopt_int8_layers", "attention_bhld", "attention_blhd", "dequantize_linears", "dequantize_weight",
    "fa2_turing_available", "flux_qk_norm_rope", "fuse_linears", "geglu_quantize", "gelu_quantize",
    "int8_attention", "int8_geglu_ff",
    "int8_fast_available", "int8_layers", "int8_mlp", "int8_turing_available", "int_mm", "linear_group",
    "ln_mod_quantize", "matmul_quantized_gated", "matmul_quantized_group",
    "lora_seed", "norm_rope", "qk_norm_rope", "qk_ok", "quantize_activation", "quantize_linears",
    "quantize_weight", "rescale", "resolve_attention_backend", "scaled_mm", "set_attention_backend",
    "set_fused_glue", "shared_qkv",
])
