"""Layers adopted from a ComfyUI int8 checkpoint, and LoRA-merged layers, run
on the GPU kernels: their forward is the oracle's W8A8 linear on the adopted
codes bit for bit (reference ``_int8.py:458-498, 148-156``;
``tests/test_int8.py:74-91``)."""

from __future__ import annotations

import json

import numpy as np
import pytest
import torch
import torch.nn as nn

import diffucore_amd as D
from oracle import gemm as OG
from oracle import quant as OQ
from tests._util import np32, rel_l2

pytestmark = pytest.mark.gpu


def _tag(group: int) -> torch.Tensor:
    meta = {"format": "int8_tensorwise", **({"convrot": True, "convrot_groupsize": group} if group else {})}
    return torch.tensor(list(json.dumps(meta).encode()), dtype=torch.uint8)


def _oracle_forward(layer: D.Int8Linear, x: torch.Tensor) -> np.ndarray:
    qa, sa = OQ.quantize_activation(np32(x).reshape(-1, layer.in_features), layer.group)
    bias = np32(layer.bias) if layer.bias is not None else None
    return OG.w8a8_linear(qa, sa, layer.weight.cpu().numpy(), layer.scale.cpu().numpy(), bias, "bf16")


def test_adopted_checkpoint_runs_on_the_kernels(gpu):
    torch.manual_seed(2)
    ref = nn.Sequential(nn.Linear(1024, 768, bias=False), nn.Linear(768, 512))
    sd = {"1.bias": ref[1].bias.detach().clone()}
    for name, group in (("0", 256), ("1", 0)):
        q, s = D.quantize_weight(ref.get_submodule(name).weight.detach(), group)
        sd.update({f"{name}.weight": q, f"{name}.weight_scale": s[:, None], f"{name}.comfy_quant": _tag(group)})
    with torch.device("meta"):
        model = nn.Sequential(nn.Linear(1024, 768, bias=False), nn.Linear(768, 512))
    model.load_state_dict(D.adopt_int8_layers(model, sd, D.int8_layers(sd)), strict=True, assign=True)
    model = model.to(gpu, torch.bfloat16)
    assert model[0].scale.dtype == torch.float32            # .to(dtype) leaves the scale bits alone

    x = torch.randn(4, 300, 1024, device=gpu, dtype=torch.bfloat16)
    h = model[0](x)
    assert np.array_equal(np32(h).reshape(-1, 768).view(np.uint32), _oracle_forward(model[0], x).view(np.uint32))
    y = model[1](h)
    assert np.array_equal(np32(y).reshape(-1, 512).view(np.uint32), _oracle_forward(model[1], h).view(np.uint32))
    want = ref.to(gpu).float()(x.float())
    assert rel_l2(np32(y), np32(want)) < 0.03


def test_lora_merged_layer_runs_on_the_kernels(gpu):
    """``add_delta_`` on the device re-quantizes with a seeded device
    generator: deterministic per seed, unbiased, and the merged layer's
    forward is the oracle's on the new codes."""
    torch.manual_seed(3)
    lin = nn.Linear(1280, 640).to(gpu)
    down, up = torch.randn(16, 1280, device=gpu) * 0.02, torch.randn(640, 16, device=gpu) * 0.02
    delta = up @ down
    layers = [D.Int8Linear.from_linear(lin, 256) for _ in range(3)]
    before = D.dequantize_weight(layers[0].weight, layers[0].scale, 256)
    seed = D.lora_seed("blocks.0.attn.qkv", "style.safetensors")
    for m, s in zip(layers, (seed, seed, seed + 1)):
        m.add_delta_(delta, s)
    assert torch.equal(layers[0].weight, layers[1].weight) and torch.equal(layers[0].scale_bits, layers[1].scale_bits)
    assert not torch.equal(layers[0].weight, layers[2].weight)
    moved = D.dequantize_weight(layers[0].weight, layers[0].scale, 256) - before
    gain = float((moved * delta).sum() / (delta * delta).sum())
    assert 0.9 < gain < 1.1

    x = torch.randn(2, 200, 1280, device=gpu, dtype=torch.bfloat16)
    y = layers[0](x)
    assert np.array_equal(np32(y).reshape(-1, 640).view(np.uint32), _oracle_forward(layers[0], x).view(np.uint32))
    want = x.float() @ (lin.weight + delta).t() + lin.bias
    assert rel_l2(np32(y), np32(want)) < 0.03


def test_int8_embedding_on_the_device(gpu):
    torch.manual_seed(4)
    table = torch.randn(1000, 768) * 0.02
    q, s = D.quantize_weight(table, 256)
    emb = D.Int8Embedding(1000, 768, 256, device=gpu)
    emb.weight.copy_(q.to(gpu))
    emb.scale_bits.copy_(s.view(torch.int32).to(gpu))
    emb.out_dtype = torch.bfloat16
    ids = torch.randint(0, 1000, (2, 77), device=gpu)
    got = emb(ids)
    assert got.dtype == torch.bfloat16 and got.shape == (2, 77, 768)
    want = OQ.dequantize_weight(q.numpy(), s.numpy(), 256)[ids.cpu().numpy()]
    assert rel_l2(np32(got), want) < 5e-3
