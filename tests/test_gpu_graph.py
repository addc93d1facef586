"""The hot path's calls captured once as a HIP graph (torch.cuda.CUDAGraph),
as bench.py times the FLUX step, then replayed: every replay must equal the
eager calls bit for bit. Replays alternate with eager work and host
synchronizations, the outputs are overwritten with NaN before each replay
(so a replay that skips a write shows), and new values written into the
captured input buffers must reach the next replay.

Covered: the quantize kernel, each GEMM plan the FLUX step uses (DMA-fed
256 x 256, 192 x 128 at the text MLP-up shape, 192 x 256 / 128 x 128,
split-K with its workspace and epilogue pass, a grouped launch of two
layers, the same pair with the gated residual epilogue) and the INT8 attention (K statistics, K quantize, attention): the
DMA-fed kernel with 256-query tiles at the FLUX shape, with 128-query tiles
and stream-K pieces plus their merge at SDXL's 4096-token self-attention and
with whole 128-query tiles at head dim 64, and the register-staged 128-query
kernel on a head-dim-128 grid too small for 256-query tiles, stream-K pieces
included.
"""

from __future__ import annotations

import pytest
import torch
from torch import nn

from diffucore_amd import _int8, attention_bhld

pytestmark = pytest.mark.gpu

BF16 = torch.bfloat16
# (M, K, N): DMA-fed 256 x 256 plan, split-K (M = 512, K = 3072), 192 x 128
# tiles (FLUX's text MLP up), a ragged one; the last two run as one grouped
# launch (dc_w8a8_gemm_grouped)
LINEARS = [(4096, 512, 4096), (512, 3072, 3072), (512, 3072, 12288), (1000, 768, 1280), (1024, 512, 1024),
           (300, 512, 1024)]
NS = len(LINEARS) - 2   # the layers called one by one
ATTN = [(1, 24, 4608, 128), (2, 10, 4096, 64), (1, 4, 1000, 64), (1, 4, 4096, 128)]


def _case(gpu, seed):
    g = torch.Generator(device=gpu).manual_seed(seed)
    torch.manual_seed(seed)
    layers = [_int8.Int8Linear.from_linear(nn.Linear(k, n, bias=True).to(gpu).to(BF16), 256) for _, k, n in LINEARS]
    xs = [torch.randn(m, k, generator=g, device=gpu).to(BF16) for m, k, _ in LINEARS]
    # residuals and one-row gates for the gated pair (the last two layers)
    xs += [torch.randn(m, n, generator=g, device=gpu).to(BF16) for m, _, n in LINEARS[NS:]]
    xs += [torch.randn(n, generator=g, device=gpu).to(BF16) for _, _, n in LINEARS[NS:]]
    qkvs = [[torch.randn(b, h, l, d, generator=g, device=gpu).to(BF16) for _ in range(3)] for b, h, l, d in ATTN]
    return layers, xs, qkvs


def _step(layers, xs, qkvs):
    ys = [layer.matmul_quantized(*_int8.quantize_activation(x, layer.group), BF16)
          for layer, x in zip(layers[:NS], xs[:NS])]
    ys += _int8.linear_group(layers[NS:], xs[NS:NS + 2])
    qs = [_int8.quantize_activation(x, layer.group) for layer, x in zip(layers[NS:], xs[NS:NS + 2])]
    ys += _int8.matmul_quantized_gated([(layer, *q, r, gt) for layer, q, r, gt
                                        in zip(layers[NS:], qs, xs[NS + 2:NS + 4], xs[NS + 4:NS + 6])], BF16)
    return ys + [attention_bhld(q, k, v, "int8_turing") for q, k, v in qkvs]


def test_graph_replays_equal_eager_calls(gpu):
    layers, xs, qkvs = _case(gpu, 3)
    m, k, n = LINEARS[0]
    assert _int8.gemm_plan(m, n, k) == "dma_256x256"
    if torch.cuda.get_device_properties(gpu).multi_processor_count == 256:
        assert _int8.gemm_plan(LINEARS[2][0], LINEARS[2][2], LINEARS[2][1]) == "192x128"
    assert _int8.gemm_group_plan([LINEARS[NS][0], LINEARS[NS + 1][0]], LINEARS[NS][2], LINEARS[NS][1])
    assert all(x.data_ptr() % 16 == 0 for x in xs[NS + 2:])   # the gated pair takes the fused epilogue
    with torch.no_grad():
        want = [t.clone() for t in _step(layers, xs, qkvs)]
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            _step(layers, xs, qkvs)
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            outs = _step(layers, xs, qkvs)
        g = torch.Generator(device=gpu).manual_seed(9)
        for rep in range(3):
            # eager work of the same kernels on other data, then a host sync
            other = torch.randn(512, 3072, generator=g, device=gpu).to(BF16)
            layers[1](other)
            attention_bhld(*[t.flip(2) for t in qkvs[1]], "int8_turing")
            torch.cuda.synchronize()
            for t in outs:
                t.fill_(float("nan"))
            graph.replay()
            torch.cuda.synchronize()
            for i, (got, ref) in enumerate(zip(outs, want)):
                assert torch.equal(got, ref), f"replay {rep}, output {i}"

        # new inputs in the captured buffers reach the next replay
        for x in xs:
            x.mul_(-0.5).add_(0.25)
        for qkv in qkvs:
            qkv[1].add_(1.0)
        want2 = [t.clone() for t in _step(layers, xs, qkvs)]
        graph.replay()
        torch.cuda.synchronize()
        for i, (got, ref, old) in enumerate(zip(outs, want2, want)):
            assert torch.equal(got, ref), f"new inputs, output {i}"
            assert not torch.equal(got, old), f"output {i} did not change"
