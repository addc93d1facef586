"""dc_int8_attn_fwd_noalloc (the entry point that allocates nothing: its
workspace is a scratch array the library keeps on each GPU) against
dc_int8_attn_fwd with a caller workspace, through the C ABI: the same kernels
and work split, so the outputs are identical bit for bit. Two calls in a row,
the second smaller, so the second reuses the first's scratch contents."""

from __future__ import annotations

import ctypes

import pytest
import torch

from diffucore_amd import _attention, _lib

pytestmark = pytest.mark.gpu


def _noalloc(q, k, v, sm_scale, out=None):
    so = _lib.require()
    B, Lq, H, D = q.shape
    if out is None:
        out = torch.empty(B, Lq, H, D, device=q.device, dtype=q.dtype)
    with torch.cuda.device(q.device):
        rc = so.dc_int8_attn_fwd_noalloc(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
                                         _lib.dtype_code(q.dtype), B, H, Lq, k.shape[1], D,
                                         _lib.strides3(q), _lib.strides3(k), _lib.strides3(v), _lib.strides3(out),
                                         ctypes.c_float(sm_scale), _lib.stream_ptr(q.device))
    _lib.check(rc, "dc_int8_attn_fwd_noalloc")
    return out


def _qkv(B, H, Lq, Lk, D, dtype, dev, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, Lq, H, D, generator=g).to(dtype).to(dev)
    k = (torch.randn(B, Lk, H, D, generator=g) + torch.randn(H, D, generator=g) * 2).to(dtype).to(dev)
    v = torch.randn(B, Lk, H, D, generator=g).to(dtype).to(dev)
    return q, k, v


@pytest.mark.parametrize("shapes", [
    # FLUX 1024^2 joint attention, then a smaller SD1.5-like call (head dim 40, ragged keys)
    [(1, 24, 4608, 4608, 128, torch.bfloat16), (2, 8, 1000, 77, 40, torch.float16)],
    # an SDXL-like call whose work split uses stream-K partials in the scratch, then a smaller one
    [(2, 10, 4096, 4096, 64, torch.float16), (1, 2, 300, 700, 64, torch.float16)],
])
def test_noalloc_matches_workspace_entry(gpu, shapes):
    for i, (B, H, Lq, Lk, D, dtype) in enumerate(shapes):
        print(f"[noalloc] call {i}: B{B} H{H} Lq{Lq} Lk{Lk} D{D} {dtype}", flush=True)
        q, k, v = _qkv(B, H, Lq, Lk, D, dtype, gpu, seed=100 + i)
        ref = _attention.int8_attention(q, k, v, D ** -0.5)
        out = _noalloc(q, k, v, D ** -0.5)
        torch.cuda.synchronize()
        assert torch.equal(out, ref), (i, (out.float() - ref.float()).abs().max().item())


def test_noalloc_strided_views_and_repeat(gpu):
    """(B, H, L, D) transposed views as the UNet / FLUX modules pass them; a
    repeated call gives the same bits."""
    g = torch.Generator().manual_seed(7)
    qkv = torch.randn(2, 1024, 3, 8, 64, generator=g).half().to(gpu)
    q, k, v = qkv[:, :, 0], qkv[:, :, 1], qkv[:, :, 2]
    ref = _attention.int8_attention(q, k, v, 0.125)
    a = _noalloc(q, k, v, 0.125)
    b = _noalloc(q, k, v, 0.125)
    assert torch.equal(a, ref) and torch.equal(b, ref)


def test_noalloc_rejects_calls_beyond_its_scratch(gpu):
    so = _lib.require()
    B, H, L, D = 8, 32, 8192, 128           # k8 alone is 268 MB
    assert so.dc_int8_attn_workspace_bytes(B, H, L, L, D) > (64 << 20)
    st = (ctypes.c_int64 * 3)(L * H * D, H * D, D)
    rc = so.dc_int8_attn_fwd_noalloc(16, 16, 16, 16, _lib.BF16, B, H, L, L, D, st, st, st, st,
                                     ctypes.c_float(0.1), None)
    assert rc == 4 and b"scratch" in so.dc_last_error()


def test_noalloc_graph_replays(gpu):
    """Captured in a HIP graph after one eager call on the device (which looks
    up the scratch array's address; the header asks for that call before any
    capture), then replayed three times between eager calls of other shapes
    that overwrite the scratch: each replay equals the eager bits, and new
    values in the captured inputs reach the next replay."""
    q, k, v = _qkv(2, 10, 1024, 1024, 64, torch.float16, gpu, seed=21)
    want = _attention.int8_attention(q, k, v, 0.125)
    out = _noalloc(q, k, v, 0.125)
    assert torch.equal(out, want)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        _noalloc(q, k, v, 0.125, out)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        _noalloc(q, k, v, 0.125, out)
    for rep in range(3):
        other = _qkv(1, 24, 700, 900, 128, torch.bfloat16, gpu, seed=30 + rep)
        _noalloc(*other, 128 ** -0.5)
        torch.cuda.synchronize()
        out.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), rep
    k.add_(1.0)
    want2 = _attention.int8_attention(q, k, v, 0.125)
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(out, want2) and not torch.equal(out, want)
