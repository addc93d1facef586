"""The drop-in inside an SD1.5 / SDXL UNet transformer block (benchmark
configs 2 and 3) on the GPU: the reference's BasicTransformerBlock
(``unet.py:122-183``, restated in ``unet_block.py``) at the config shapes,
batch 2, fp16, with every linear swapped for W8A8 by ``quantize_linears`` and
``int8_turing`` stamped by ``set_attention_backend``, against the same block
run eagerly in fp16 (SDPA, fp16 linears). Bounds are stated per test; the
measured values are printed."""

from __future__ import annotations

import copy

import pytest
import torch
import torch.nn.functional as F

import unet_block as UB
from diffucore_amd import Int8Linear, set_attention_backend
from tests._util import cosine, np32, rel_l2

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("level", UB.LEVELS, ids=[lv.name for lv in UB.LEVELS])
def test_int8_block_against_fp16_eager(gpu, level):
    """W8A8 linears (ConvRot 256 where the width allows it), INT8
    self-attention, exact cross-attention (77 keys: SDPA) and the fused GEGLU
    middle, against the fp16 block: rel L2 < 3e-2 and cosine > 0.999 on the
    block output's update (block(x) - x, which the residual would otherwise
    dominate)."""
    blk = UB.build(level, gpu)
    x, ctx = UB.inputs(level, gpu)
    with torch.no_grad():
        ref = blk(x, ctx) - x
        q = UB.to_int8(copy.deepcopy(blk), gpu)
        assert all(isinstance(q.get_submodule(n), Int8Linear) for n in UB.linear_names(q))
        assert q.attn1.attn_backend == q.attn2.attn_backend == "int8_turing"
        out = q(x, ctx) - x
    torch.cuda.synchronize()
    r, c = rel_l2(np32(out), np32(ref)), cosine(np32(out), np32(ref))
    print(f"\n[unet] {level.name}: int8 block vs fp16 rel_l2 {r:.4g} cos {c:.6f}")
    assert out.dtype == torch.float16 and torch.isfinite(out).all()
    assert r < 3e-2 and c > 0.999


def test_cross_attention_stamped_int8_is_exact(gpu):
    """The UNet's cross-attention carries no is_selfattn flag, so the INT8
    backend is stamped on it too (as in the reference); with a 77-token
    context it runs exact SDPA: bit-identical to the module stamped sdpa."""
    level = UB.SDXL_L1
    blk = UB.build(level, gpu)
    x, ctx = UB.inputs(level, gpu)
    a = blk.attn2
    assert set_attention_backend(blk, "int8_turing") == 2 and a.attn_backend == "int8_turing"
    with torch.no_grad():
        y8 = a(blk.norm2(x), ctx)
        a.attn_backend = "sdpa"
        ys = a(blk.norm2(x), ctx)
    assert torch.equal(y8, ys)


@pytest.mark.parametrize("level", [UB.SD15_L1, UB.SDXL_L2], ids=["sd15_l1", "sdxl_l2"])
def test_geglu_feed_forward_fused_matches_eager_int8(gpu, level):
    """The fused GEGLU middle against the same W8A8 layers run eagerly
    (proj, chunk, x * gelu(gate), out): rel L2 < 2e-3."""
    blk = UB.to_int8(UB.build(level, gpu), gpu)
    x, _ = UB.inputs(level, gpu)
    h = blk.norm3(x)
    with torch.no_grad():
        fused = blk.ff(h)
        proj, out = blk.ff.net[0].proj, blk.ff.net[2]
        a, gate = proj(h).chunk(2, dim=-1)
        eager = out(a * F.gelu(gate))
    assert rel_l2(np32(fused), np32(eager)) < 2e-3
