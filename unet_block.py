"""Synthetic SD1.5 / SDXL UNet transformer block for measuring the hot path in
place (the SD1.5 and SDXL benchmark configs).

Restates the reference's ``CrossAttention``, ``GEGLU``, ``FeedForward`` and
``BasicTransformerBlock`` (``src/diffucore/models/unet.py:122-183``): self-
attention, cross-attention over the text context, and a GEGLU feed-forward
(dim -> 2 x 4 dim -> dim), each behind a LayerNorm with a residual. As in the
reference, the attention modules carry an ``attn_backend`` slot and no
``is_selfattn`` flag, so ``set_attention_backend(block, "int8_turing")``
stamps the INT8 backend on the cross-attention as well, and
``quantize_linears`` swaps any of the block's linears for W8A8 layers. With
W8A8 ``proj`` and ``out`` layers the feed-forward runs the fused GEGLU middle
(``int8_geglu_ff``), where the reference would run ``x * F.gelu(gate)`` on the
dequantized activations.

This is a measurement and test harness (``bench.py --shapes``,
``tests/test_gpu_unet.py``), not a product model.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn as nn
import torch.nn.functional as F

from diffucore_amd import attention_bhld
from diffucore_amd._int8 import Int8Linear, int8_geglu_ff


@dataclass(frozen=True)
class UNetLevel:
    """One transformer level of a UNet at a given latent size: ``tokens`` =
    latent pixels at that level, ``dim`` channels in ``heads`` heads, a text
    context of ``ctx_len`` x ``ctx_dim``, batch 2 (the CFG pair)."""
    name: str
    dim: int
    heads: int
    tokens: int
    ctx_dim: int
    ctx_len: int = 77
    batch: int = 2


# the SD1.5 config: 512^2, the first (highest-resolution) level;
# the SDXL config: 1024^2, its two transformer levels
SD15_L1 = UNetLevel("sd15_l1", 320, 8, 4096, 768)
SDXL_L1 = UNetLevel("sdxl_l1", 640, 10, 4096, 2048)
SDXL_L2 = UNetLevel("sdxl_l2", 1280, 20, 1024, 2048)
LEVELS = (SD15_L1, SDXL_L1, SDXL_L2)


class CrossAttention(nn.Module):
    def __init__(self, query_dim: int, context_dim: int, heads: int, dim_head: int):
        super().__init__()
        inner = dim_head * heads
        self.heads, self.dim_head = heads, dim_head
        self.to_q = nn.Linear(query_dim, inner, bias=False)
        self.to_k = nn.Linear(context_dim, inner, bias=False)
        self.to_v = nn.Linear(context_dim, inner, bias=False)
        self.to_out = nn.Sequential(nn.Linear(inner, query_dim), nn.Dropout(0.0))
        self.attn_backend = "sdpa"
        # W8A8 only (see to_int8): the projections that share an input stacked
        # into one layer (one quantization, one GEMM; bit-identical results)
        self.qkv_fused = None
        self.kv_fused = None

    def forward(self, x: torch.Tensor, context: torch.Tensor | None = None) -> torch.Tensor:
        if context is None and self.qkv_fused is not None:
            q, k, v = self.qkv_fused(x).chunk(3, dim=-1)
        elif self.kv_fused is not None:
            q = self.to_q(x)
            k, v = self.kv_fused(x if context is None else context).chunk(2, dim=-1)
        else:
            context = x if context is None else context
            q, k, v = self.to_q(x), self.to_k(context), self.to_v(context)
        b = x.shape[0]

        def split(t):
            return t.view(b, -1, self.heads, self.dim_head).transpose(1, 2)

        return self.to_out(attention_bhld(split(q), split(k), split(v), self.attn_backend))


class GEGLU(nn.Module):
    def __init__(self, dim_in: int, dim_out: int):
        super().__init__()
        self.proj = nn.Linear(dim_in, dim_out * 2)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        x, gate = self.proj(x).chunk(2, dim=-1)
        return x * F.gelu(gate)


class FeedForward(nn.Module):
    def __init__(self, dim: int, mult: int = 4):
        super().__init__()
        self.net = nn.Sequential(GEGLU(dim, dim * mult), nn.Dropout(0.0), nn.Linear(dim * mult, dim))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        proj, out = self.net[0].proj, self.net[2]
        if isinstance(proj, Int8Linear) and isinstance(out, Int8Linear):
            return int8_geglu_ff(x, proj, out)
        return self.net(x)


class BasicTransformerBlock(nn.Module):
    def __init__(self, dim: int, heads: int, context_dim: int):
        super().__init__()
        dim_head = dim // heads
        self.attn1 = CrossAttention(dim, dim, heads, dim_head)
        self.ff = FeedForward(dim)
        self.attn2 = CrossAttention(dim, context_dim, heads, dim_head)
        self.norm1, self.norm2, self.norm3 = nn.LayerNorm(dim), nn.LayerNorm(dim), nn.LayerNorm(dim)

    def forward(self, x: torch.Tensor, context: torch.Tensor) -> torch.Tensor:
        x = x + self.attn1(self.norm1(x))
        x = x + self.attn2(self.norm2(x), context)
        return x + self.ff(self.norm3(x))


def linear_names(block: BasicTransformerBlock) -> list[str]:
    """The block's linears a W8A8 swap replaces: q/k/v/out of both attentions
    and the GEGLU feed-forward's two (the SDXL config)."""
    names = []
    for a in ("attn1", "attn2"):
        names += [f"{a}.to_q", f"{a}.to_k", f"{a}.to_v", f"{a}.to_out.0"]
    return names + ["ff.net.0.proj", "ff.net.2"]


def group_for(layer: nn.Linear) -> int:
    """ConvRot group 256 where the input width allows it, none otherwise
    (SD1.5's 320- and SDXL's 640-wide inputs)."""
    return 256 if layer.in_features % 256 == 0 else 0


@torch.no_grad()
def build(level: UNetLevel, device, dtype=torch.float16, seed: int = 0) -> BasicTransformerBlock:
    """Random-init block: linear weights and biases N(0, 0.02), LayerNorms at
    their defaults (weight 1, bias 0)."""
    torch.manual_seed(seed)
    blk = BasicTransformerBlock(level.dim, level.heads, level.ctx_dim).to(device=device, dtype=dtype)
    g = torch.Generator(device=device).manual_seed(seed)
    for name, p in blk.named_parameters():
        if ".norm" not in f".{name}" and not name.startswith("norm"):
            p.normal_(0.0, 0.02, generator=g)
    return blk


@torch.no_grad()
def to_int8(blk: BasicTransformerBlock, device) -> BasicTransformerBlock:
    """Swap every block linear for a W8A8 layer (per layer group, see
    :func:`group_for`), stack the self-attention's q / k / v and the
    cross-attention's k / v into one layer each (``fuse_linears``), and stamp
    the INT8 attention backend."""
    from diffucore_amd import fuse_linears, quantize_linears, set_attention_backend
    for name in linear_names(blk):
        layer = blk.get_submodule(name)
        quantize_linears(blk, [name], device, group_for(layer))
    blk.attn1.qkv_fused = fuse_linears([blk.attn1.to_q, blk.attn1.to_k, blk.attn1.to_v])
    blk.attn2.kv_fused = fuse_linears([blk.attn2.to_k, blk.attn2.to_v])
    set_attention_backend(blk, "int8_turing")
    return blk


def inputs(level: UNetLevel, device, dtype=torch.float16, seed: int = 1):
    g = torch.Generator(device=device).manual_seed(seed)
    x = torch.randn(level.batch, level.tokens, level.dim, generator=g, device=device).to(dtype)
    ctx = torch.randn(level.batch, level.ctx_len, level.ctx_dim, generator=g, device=device).to(dtype)
    return x, ctx
