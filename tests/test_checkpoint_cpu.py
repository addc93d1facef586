"""Checkpoint ingestion and LoRA merging on the CPU (load-side torch ops; the
GEMM itself is covered by the GPU tests): ComfyUI ``int8_tensorwise`` files
(reference ``_int8.py:458-498``, its tests ``tests/test_int8.py:74-98`` and
``tests/test_moss_image.py:283-309``), ``Int8Embedding`` (``_int8.py:173-197``)
and the seeded stochastic rounding of ``add_delta_`` / ``lora_seed``
(``_int8.py:148-156, 518-520``)."""

from __future__ import annotations

import json

import pytest
import torch
import torch.nn as nn

import diffucore_amd as D
from tests._util import rel_l2


def _tag(**meta) -> torch.Tensor:
    return torch.tensor(list(json.dumps(meta).encode()), dtype=torch.uint8)


def _comfy(prefix: str, w: torch.Tensor, group: int, tensorwise: bool = False) -> dict:
    """One layer as a ComfyUI int8 file stores it: int8 codes, ``weight_scale``
    ``[N, 1]`` (or one value for the tensor) and the JSON tag."""
    if tensorwise:
        scale = w.abs().max() / 127.0
        q = torch.clamp(torch.round(w / scale), -128, 127).to(torch.int8)
        ws = scale.reshape(())
    else:
        q, s = D.quantize_weight(w, group)
        ws = s[:, None]
    meta = {"format": "int8_tensorwise"}
    if group:
        meta.update(convrot=True, convrot_groupsize=group)
    return {f"{prefix}.weight": q, f"{prefix}.weight_scale": ws, f"{prefix}.comfy_quant": _tag(**meta)}


def _net(device=None):
    return nn.Sequential(nn.Linear(512, 256, bias=False, device=device), nn.Linear(256, 128, device=device),
                         nn.Linear(256, 64, device=device))


def test_adopts_a_comfy_int8_checkpoint():
    torch.manual_seed(1)
    ref = _net()
    sd = {"1.bias": ref[1].bias.detach().clone(), "2.weight": ref[2].weight.detach().clone(),
          "2.bias": ref[2].bias.detach().clone()}
    sd.update(_comfy("0", ref[0].weight.detach(), 256))
    sd.update(_comfy("1", ref[1].weight.detach(), 0, tensorwise=True))
    codes = {n: sd[f"{n}.weight"].clone() for n in ("0", "1")}
    scale1 = sd["1.weight_scale"].clone()

    layers = D.int8_layers(sd)
    assert layers == {"0": 256, "1": 0}
    with torch.device("meta"):
        model = _net()
    model.load_state_dict(D.adopt_int8_layers(model, sd, layers), strict=True, assign=True)
    assert isinstance(model[0], D.Int8Linear) and model[0].group == 256 and model[0].bias is None
    assert isinstance(model[1], D.Int8Linear) and model[1].group == 0 and model[1].bias is not None
    assert type(model[2]) is nn.Linear
    for n in ("0", "1"):
        assert torch.equal(model.get_submodule(n).weight, codes[n])
    # a tensor-wide scale is spread over every row, bit for bit
    assert scale1.dim() == 0 and torch.equal(model[1].scale, scale1.float().expand(128))
    for i in (0, 1):
        w = D.dequantize_weight(model[i].weight, model[i].scale, model[i].group)
        assert rel_l2(w.numpy(), ref[i].weight.detach().numpy()) < 0.01

    x = torch.randn(8, 512)
    assert D.dequantize_linears(model, torch.float32) == 2
    assert all(type(m) is nn.Linear for m in model)
    with torch.no_grad():
        assert rel_l2(model[1](model[0](x)).numpy(), ref[1](ref[0](x)).numpy()) < 0.02


def test_adopted_names_match_the_layer_state_dict():
    with torch.device("meta"):
        model = _net()
    sd = _comfy("0", torch.randn(256, 512), 256)
    D.adopt_int8_layers(model, sd, D.int8_layers(sd))
    assert set(sd) == {"0.weight", "0.scale_bits"} and sd["0.scale_bits"].dtype == torch.int32
    assert set(model[0].state_dict()) == set(k[2:] for k in sd)


def test_rejects_other_quantized_formats():
    with pytest.raises(ValueError, match="nvfp4"):
        D.int8_layers({"blocks.0.mlp.layer1.comfy_quant": _tag(format="nvfp4")})
    assert D.int8_layers({"a.weight": torch.zeros(2, 2)}) == {}
    # convrot without a group size means the default group
    assert D.int8_layers({"a.comfy_quant": _tag(format="int8_tensorwise", convrot=True)}) == {"a": 256}
    # a tag stored in a wider integer dtype holds the same byte values (the reference reads bytes(tag.tolist()))
    wide = _tag(format="int8_tensorwise", convrot=True, convrot_groupsize=64).to(torch.int64)
    assert D.int8_layers({"a.comfy_quant": wide}) == {"a": 64}


def test_int8_embedding_rows_equal_the_dequantized_table():
    torch.manual_seed(0)
    table = torch.randn(50, 512) * 0.02
    q, scale = D.quantize_weight(table, 256)
    emb = D.Int8Embedding(50, 512, 256)
    emb.weight.copy_(q)
    emb.scale_bits.copy_(scale.view(torch.int32))
    ids = torch.tensor([[3, 7, 3], [0, 49, 10]])
    full = D.dequantize_weight(q, scale, 256)
    got = emb(ids)
    assert got.shape == (2, 3, 512) and got.dtype == torch.float32
    torch.testing.assert_close(got, full[ids], rtol=1e-5, atol=1e-8)
    assert rel_l2(got.numpy(), table[ids].numpy()) < 0.01
    emb.out_dtype = torch.bfloat16
    assert emb(ids).dtype == torch.bfloat16
    with pytest.raises(ValueError, match="multiple"):
        D.Int8Embedding(10, 320, 256)


def test_int8_embedding_adopts_a_comfy_table():
    torch.manual_seed(0)
    table = torch.randn(40, 256) * 0.02
    holder = nn.Module()
    holder.embed_tokens = nn.Embedding(40, 256, device="meta")
    sd = {("embed_tokens." + k.split(".", 1)[1]): v for k, v in _comfy("x", table, 256).items()}
    group = D.int8_layers(sd).pop("embed_tokens")
    q, scale = sd["embed_tokens.weight"], sd["embed_tokens.weight_scale"].reshape(-1)
    holder.load_state_dict(D.adopt_int8_embedding(holder, sd, "embed_tokens", group), strict=True, assign=True)
    assert isinstance(holder.embed_tokens, D.Int8Embedding) and holder.embed_tokens.group == 256
    ids = torch.tensor([[5, 39, 0]])
    torch.testing.assert_close(holder.embed_tokens(ids), D.dequantize_weight(q, scale, 256)[ids],
                               rtol=1e-5, atol=1e-8)


def _crc32_bitwise(data: bytes) -> int:
    """CRC-32 (ISO-HDLC: reflected polynomial 0xEDB88320, init and final xor
    0xFFFFFFFF), one bit at a time."""
    crc = 0xFFFFFFFF
    for byte in data:
        crc ^= byte
        for _ in range(8):
            crc = (crc >> 1) ^ (0xEDB88320 if crc & 1 else 0)
    return crc ^ 0xFFFFFFFF


def test_lora_seed_is_crc32_of_name_and_path():
    assert _crc32_bitwise(b"123456789") == 0xCBF43926            # the CRC-32 check value
    for name, path in (("blocks.0.attn.qkv", "/loras/style.safetensors"), ("", ""), ("a|b", "c")):
        assert D.lora_seed(name, path) == _crc32_bitwise(f"{name}|{path}".encode())


def _layer(seed: int, group: int = 256) -> D.Int8Linear:
    torch.manual_seed(seed)
    return D.Int8Linear.from_linear(nn.Linear(512, 384, bias=False), group)


@pytest.mark.parametrize("group", [0, 256])
def test_add_delta_is_unbiased_below_half_a_step(group):
    """A delta of a fifth of a quantization step: round-to-nearest would keep
    none of it; the stochastic rounding keeps it on average."""
    m = _layer(3, group)
    before = D.dequantize_weight(m.weight, m.scale, group)
    g = torch.Generator().manual_seed(5)
    delta = torch.randn(384, 512, generator=g) * (0.2 * m.scale.mean())
    m.add_delta_(delta, D.lora_seed("layer", "a.safetensors"))
    moved = D.dequantize_weight(m.weight, m.scale, group) - before
    gain = float((moved * delta).sum() / (delta * delta).sum())
    assert 0.9 < gain < 1.1
    # round-to-nearest re-quantization of the same sum keeps far less
    q, s = D.quantize_weight(before + delta, group)
    gain_rtn = float(((D.dequantize_weight(q, s, group) - before) * delta).sum() / (delta * delta).sum())
    assert gain_rtn < 0.5


def test_add_delta_is_deterministic_per_seed():
    delta = torch.randn(384, 512, generator=torch.Generator().manual_seed(6)) * 1e-4
    a, b, c = _layer(4), _layer(4), _layer(4)
    a.add_delta_(delta, 11)
    b.add_delta_(delta, 11)
    c.add_delta_(delta, 12)
    assert torch.equal(a.weight, b.weight) and torch.equal(a.scale_bits, b.scale_bits)
    assert not torch.equal(a.weight, c.weight)
    assert a.weight.dtype == torch.int8 and a.scale.dtype == torch.float32
