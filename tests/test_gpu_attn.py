"""dc_int8_attn_fwd on the GPU.

* K smoothing / quantization and Q quantization: bit-exact against the oracle
  (reference ``int8_attn_sm80.cu:38-142, 341-388``), read back from the
  documented workspace.
* Output: against the oracle's restatement of the algorithm (tight bound) and
  against float32 SDPA with the reference's own bar, rel L2 < 3e-2 and
  cosine > 0.9995 (``tests/test_attention_dispatch.py:198-213``).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from diffucore_amd import _attention as A
from oracle import attn as OA
from tests._util import DT, cosine, max_abs, np32, rel_l2

pytestmark = pytest.mark.gpu

# tolerance against the oracle's restatement (same quantization, exact softmax):
# the output itself is rounded to the 16-bit type on both sides, so the bound
# scales with that type's precision (bf16 ulp 2^-8, fp16 ulp 2^-11)
ORACLE_REL = {torch.float16: 1e-3, torch.bfloat16: 4e-3}
ORACLE_COS = 0.99999


def _ref_blhd(q, k, v):
    out = F.scaled_dot_product_attention(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2))
    return out.transpose(1, 2)


def _inputs(B, Lq, Lk, H, D, dtype, seed=0, k_offset=0.5):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, Lq, H, D, generator=g)
    k = torch.randn(B, Lk, H, D, generator=g) + k_offset
    v = torch.randn(B, Lk, H, D, generator=g)
    return q.to(dtype), k.to(dtype), v.to(dtype)


def _run(q, k, v, gpu):
    B, Lq, H, D = q.shape
    Lk = k.shape[1]
    qd, kd, vd = q.to(gpu), k.to(gpu), v.to(gpu)
    ws = torch.empty(A.workspace_bytes(B, H, Lq, Lk, D), device=gpu, dtype=torch.uint8)
    out = A.int8_attention(qd, kd, vd, D ** -0.5, workspace=ws)
    return out, A.workspace_views(ws, B, H, Lq, Lk, D)


CASES = [
    # the reference's own shapes (tests/test_attention_dispatch.py:199-200), head dim 128
    (1, 1024, 1024, 4, 128, torch.float16), (2, 1000, 1000, 2, 128, torch.float16),
    (1, 700, 77, 4, 128, torch.float16), (1, 70, 3953, 2, 128, torch.float16),
    # extensions: bf16 (FLUX), head dim 64 (SDXL), 40 (SD1.5, padded to 64)
    (1, 1024, 1024, 4, 128, torch.bfloat16), (2, 300, 500, 3, 64, torch.float16),
    (2, 257, 77, 2, 40, torch.float16), (1, 333, 190, 2, 40, torch.bfloat16),
    # head dims between 64 and 128 (padded to 128; V channels past D clamped in the loads)
    (1, 300, 333, 2, 96, torch.bfloat16), (2, 513, 129, 3, 72, torch.float16),
]
# grids of at least one 256-query tile per CU, which run the 8-wave DMA-fed
# kernel: head dims 128 / 96 / 72, ragged key ranges, a ragged last query tile
WIDE_CASES = [
    (1, 1024, 300, 64, 128, torch.bfloat16), (2, 1024, 333, 64, 96, torch.float16),
    (1, 1200, 129, 52, 72, torch.bfloat16),
]
CASES += WIDE_CASES


@pytest.mark.parametrize("B,Lq,Lk,H,D,dtype", WIDE_CASES)
def test_wide_cases_run_256_query_tiles(gpu, B, Lq, Lk, H, D, dtype):
    """On MI355X (256 CUs) these shapes take whole 256-query tiles; the small
    head-dim-128 shapes above take 128-query tiles."""
    if torch.cuda.get_device_properties(gpu).multi_processor_count != 256:
        pytest.skip("tile counts are for 256 CUs")
    assert A.attn_plan(B, H, Lq, Lk, D, dtype) == {"dp_tiles": (Lq + 255) // 256 * B * H, "sk_blocks": 0,
                                                   "sk_tiles": 0}
    assert A.attn_plan(1, 4, 1024, 1024, 128, dtype) == {"dp_tiles": 32, "sk_blocks": 0, "sk_tiles": 0}


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_wide_kernel_growing_logits_rescale(gpu, dtype):
    """Keys aligned ever more with the queries: the row maxima grow by ~6 (log2
    units) per 64-key tile, from ~8 in the first tile to ~100 in the last, so
    the wide kernel's lazy maximum (P against the running maximum, rescaled
    when a tile's probabilities sum past 2^12) rescales O every few tiles; in
    float16 an unrescaled P would overflow. Against the oracle's exact online
    softmax."""
    B, Lq, Lk, H, D = 1, 1024, 1024, 64, 128
    g = torch.Generator().manual_seed(3)
    u = torch.randn(D, generator=g)
    u /= u.norm()
    q = (8 * u + 0.1 * torch.randn(B, Lq, H, D, generator=g)).to(dtype)
    k = (100 * torch.linspace(0, 1, Lk).view(1, Lk, 1, 1) * u + torch.randn(B, Lk, H, D, generator=g)).to(dtype)
    v = torch.randn(B, Lk, H, D, generator=g).to(dtype)
    if torch.cuda.get_device_properties(gpu).multi_processor_count == 256:
        assert A.attn_plan(B, H, Lq, Lk, D, dtype)["dp_tiles"] == 256   # whole 256-query tiles
    out, _ = _run(q, k, v, gpu)
    o = np32(out)
    assert np.isfinite(o).all()
    ora = OA.int8_attention(np32(q), np32(k), np32(v), D ** -0.5, DT[dtype], DT[dtype])
    r, c = rel_l2(o, ora), cosine(o, ora)
    print(f"[attn] growing logits {DT[dtype]}: vs oracle rel {r:.2e} cos {c:.7f}")
    assert r < ORACLE_REL[dtype] and c > ORACLE_COS


@pytest.mark.parametrize("B,Lq,Lk,H,D,dtype", CASES)
def test_codes_and_scales_bit_exact(gpu, B, Lq, Lk, H, D, dtype):
    q, k, v = _inputs(B, Lq, Lk, H, D, dtype)
    _, ws = _run(q, k, v, gpu)
    ksum = OA.k_colsum(np32(k))
    assert np.array_equal(ws["ksum"].cpu().numpy().view(np.uint32), ksum.view(np.uint32))
    ki, ks = OA.k_quantize(np32(k), ksum)
    assert np.array_equal(ws["ks"].cpu().numpy().view(np.uint32), ks.view(np.uint32))
    assert np.array_equal(ws["k8"][..., :D].cpu().numpy(), ki)
    assert not ws["k8"][..., D:].any()
    q8_ref, qs_ref = OA.q_quantize(np32(q))
    q8, qs = A.quantize_q(q.to(gpu))
    assert np.array_equal(q8[:, :, :Lq, :D].cpu().numpy(), q8_ref)
    assert not q8[..., D:].any() and not q8[:, :, Lq:].any()
    assert np.array_equal(qs[:, :, :Lq].cpu().numpy().view(np.uint32), qs_ref.view(np.uint32))


@pytest.mark.parametrize("B,H,Lk,D,dtype", [
    # the FLUX key set; 469 windows summed into one head's ksum; 5160 windows
    # over 40 heads with a ragged last window at head dim 64
    (1, 24, 4608, 128, torch.bfloat16), (1, 1, 60000, 128, torch.float16),
    (1, 40, 16421, 64, torch.float16),
])
def test_k_preparation_large_key_sets_bit_exact(gpu, B, H, Lk, D, dtype):
    print(f"[attn] K preparation B {B} H {H} Lk {Lk} D {D} {DT[dtype]}", flush=True)
    q, k, v = _inputs(B, 64, Lk, H, D, dtype, seed=5)
    _, ws = _run(q, k, v, gpu)
    ksum = OA.k_colsum(np32(k))
    assert np.array_equal(ws["ksum"].cpu().numpy().view(np.uint32), ksum.view(np.uint32))
    ki, ks = OA.k_quantize(np32(k), ksum)
    assert np.array_equal(ws["ks"].cpu().numpy().view(np.uint32), ks.view(np.uint32))
    assert np.array_equal(ws["k8"][..., :D].cpu().numpy(), ki)
    assert not ws["k8"][..., D:].any()


@pytest.mark.parametrize("B,Lq,Lk,H,D,dtype", CASES)
def test_output_close_to_oracle_and_sdpa(gpu, B, Lq, Lk, H, D, dtype):
    q, k, v = _inputs(B, Lq, Lk, H, D, dtype)
    out, _ = _run(q, k, v, gpu)
    assert out.shape == (B, Lq, H, D) and out.dtype == dtype
    o = np32(out)
    assert np.isfinite(o).all()
    ora = OA.int8_attention(np32(q), np32(k), np32(v), D ** -0.5, DT[dtype], DT[dtype])
    r, c = rel_l2(o, ora), cosine(o, ora)
    print(f"[attn] {B},{Lq},{Lk},{H},{D},{DT[dtype]}: vs oracle rel {r:.2e} cos {c:.7f} maxabs {max_abs(o, ora):.2e}")
    assert r < ORACLE_REL[dtype] and c > ORACLE_COS
    ref = np32(_ref_blhd(q.float(), k.float(), v.float()))
    r, c = rel_l2(o, ref), cosine(o, ref)
    print(f"[attn]   vs fp32 SDPA rel {r:.2e} cos {c:.7f}")
    assert r < 3e-2 and c > 0.9995


def test_bhld_and_strided_inputs(gpu):
    torch.manual_seed(0)
    q, k, v = (torch.randn(1, 3, 600, 128, device=gpu).half() for _ in range(3))
    ref = F.scaled_dot_product_attention(q.float(), k.float(), v.float()).transpose(1, 2).reshape(1, 600, -1)
    assert rel_l2(np32(A.attention_bhld(q, k, v, "int8_turing")), np32(ref)) < 3e-2
    qkv = torch.randn(1, 500, 2, 3 * 128, device=gpu).half()   # packed: stride(2) = 384
    q, k, v = qkv[..., :128], qkv[..., 128:256], qkv[..., 256:]
    ref = _ref_blhd(q.float(), k.float(), v.float()).reshape(1, 500, -1)
    out = A.attention_blhd(q, k, v, "int8_turing")
    assert rel_l2(np32(out), np32(ref)) < 3e-2


def test_flat_scores_large_v(gpu):
    """Every p = 1 with large same-sign V (tests/test_attention_dispatch.py:229-238):
    the reference needs a per-head P scale against fp16 partial overflow; the
    float32 PV accumulation here cannot overflow."""
    q = torch.zeros(1, 256, 2, 128, device=gpu).half()
    k = torch.randn(1, 1024, 2, 128, device=gpu).half()
    v = (torch.rand(1, 1024, 2, 128, device=gpu) * 200 + 900).half()
    out = A.attention_blhd(q, k, v, "int8_turing")
    assert torch.isfinite(out).all()
    assert rel_l2(np32(out), np32(_ref_blhd(q.float(), k.float(), v.float()).reshape(1, 256, -1))) < 1e-3


def test_zero_query_is_mean_of_v(gpu):
    q = torch.zeros(1, 64, 1, 64, device=gpu, dtype=torch.bfloat16)
    k = torch.randn(1, 300, 1, 64, device=gpu, dtype=torch.bfloat16)
    v = torch.randn(1, 300, 1, 64, device=gpu, dtype=torch.bfloat16)
    out = A.attention_blhd(q, k, v, "int8_turing")
    mean = v.float().mean(1, keepdim=True).expand(1, 64, 1, 64).reshape(1, 64, -1)
    assert max_abs(np32(out), np32(mean)) < 1e-2


def test_other_head_dims_fall_back_to_sdpa(gpu):
    torch.manual_seed(0)
    for D in (36, 256):
        q = torch.randn(1, 256, 2, D, device=gpu).half()
        assert torch.equal(A.attention_blhd(q, q, q, "int8_turing"), A.attention_blhd(q, q, q, "sdpa"))


def test_short_key_ranges_take_sdpa(gpu):
    """Key ranges of at most SHORT_KEYS (cross-attention over a 77-token text
    context) run exact SDPA on the int8_turing backend, as a UNet stamps it
    on its cross-attention too (unet.py:122-145 has no is_selfattn); one key
    more runs the INT8 kernels, within the reference's bar."""
    torch.manual_seed(1)
    q = torch.randn(2, 8, 4096, 40, device=gpu).half()                  # SD1.5 level-1 cross-attention
    for lk in (77, A.SHORT_KEYS):
        k, v = (torch.randn(2, 8, lk, 40, device=gpu).half() for _ in range(2))
        assert torch.equal(A.attention_bhld(q, k, v, "int8_turing"), A.attention_bhld(q, k, v, "sdpa"))
    k, v = (torch.randn(2, 8, A.SHORT_KEYS + 1, 40, device=gpu).half() for _ in range(2))
    out = A.attention_bhld(q, k, v, "int8_turing")
    ref = F.scaled_dot_product_attention(q.float(), k.float(), v.float()).transpose(1, 2).reshape(2, 4096, -1)
    assert not torch.equal(out, A.attention_bhld(q, k, v, "sdpa"))
    assert rel_l2(np32(out), np32(ref)) < 3e-2 and cosine(np32(out), np32(ref)) > 0.9995


def test_deterministic(gpu):
    q, k, v = _inputs(1, 500, 700, 3, 128, torch.bfloat16, seed=3)
    outs = [_run(q, k, v, gpu)[0] for _ in range(3)]
    assert all(torch.equal(outs[0], o) for o in outs[1:])


@pytest.mark.parametrize("B,H,L,D,dtype", [(2, 10, 4096, 64, torch.float16), (2, 10, 4096, 64, torch.bfloat16),
                                             (1, 4, 4096, 128, torch.bfloat16), (1, 24, 4096, 128, torch.bfloat16)])
# head dim 64: the DMA-fed kernel's stream-K pieces; (1, 4, 4096, 128): a grid
# too small for 256-row tiles, the register-staged kernel's pieces; FLUX-like
# (1, 24, 4096, 128) runs whole 256-row tiles and stays as a plain repeat test
def test_stream_k_repeat_calls_identical(gpu, B, H, L, D, dtype):
    """Launches with stream-K pieces and their merge give the same bits on
    every call (regression: the merge kernel once declared less LDS than its
    factor / 1 / l / slot layout uses, and tiles merged with another
    workgroup's factors now and then)."""
    if A.attn_plan(B, H, L, L, D, dtype)["sk_blocks"] == 0 and H < 24:
        pytest.skip("no stream-K split at this shape on this device")
    g = torch.Generator(device=gpu).manual_seed(12)
    q = torch.randn(B, L, H, D, device=gpu, generator=g).to(dtype)
    k = (torch.randn(B, L, H, D, device=gpu, generator=g) + 0.5).to(dtype)
    v = torch.randn(B, L, H, D, device=gpu, generator=g).to(dtype)
    first = A.int8_attention(q, k, v, D ** -0.5).clone()
    for _ in range(12):
        assert torch.equal(A.int8_attention(q, k, v, D ** -0.5), first)


def test_stream_k_pieces_match_whole_tiles(gpu):
    """Query tiles past the last whole round of workgroups run as stream-K
    pieces (ranges of key tiles) whose partial O, row maxima and row sums a
    merge kernel combines. Heads run that way agree per query tile with the
    same heads run whole (they differ only in where the running maximum sits
    when P is rounded to bf16), and the heads run whole in both launches are
    bit-identical."""
    B, L, D, dtype = 1, 4096, 64, torch.float16
    H = 20                       # SDXL's 2 x 10 heads at 4096 tokens: 640 query tiles, 512 run whole
    pl = A.attn_plan(B, H, L, L, D, dtype)
    per_head = L // 128
    if pl["sk_blocks"] == 0 or pl["dp_tiles"] % per_head:
        pytest.skip(f"no stream-K split at this shape on this device: {pl}")
    h_dp = pl["dp_tiles"] // per_head           # heads run whole in the H = 24 launch
    n_sk = H - h_dp
    # the stream-K heads first, then as many whole heads, as one launch run whole
    order = list(range(h_dp, H)) + list(range(0, h_dp))[: max(0, h_dp - n_sk)]
    order = order[:h_dp] if len(order) > h_dp else order
    pl2 = A.attn_plan(B, len(order), L, L, D, dtype)
    if pl2["sk_blocks"] != 0:
        pytest.skip(f"no whole-round launch for the comparison on this device: {pl2}")
    g = torch.Generator(device=gpu).manual_seed(11)
    q = torch.randn(B, L, H, D, device=gpu, generator=g).to(dtype)
    k = (torch.randn(B, L, H, D, device=gpu, generator=g) + 0.5).to(dtype)
    v = torch.randn(B, L, H, D, device=gpu, generator=g).to(dtype)
    out = A.int8_attention(q, k, v, D ** -0.5)
    idx = torch.tensor(order, device=gpu)
    out2 = A.int8_attention(q[:, :, idx].contiguous(), k[:, :, idx].contiguous(), v[:, :, idx].contiguous(), D ** -0.5)
    for j, hh in enumerate(order):
        if hh < h_dp:
            assert torch.equal(out[:, :, hh], out2[:, :, j]), hh
            continue
        a, b_ = out[0, :, hh].float(), out2[0, :, j].float()
        ref = F.scaled_dot_product_attention(q[:, :, hh:hh + 1].transpose(1, 2).float(),
                                             k[:, :, hh:hh + 1].transpose(1, 2).float(),
                                             v[:, :, hh:hh + 1].transpose(1, 2).float())[0, 0]
        for t0 in range(0, L, 128):
            sl = slice(t0, t0 + 128)
            assert (a[sl] - b_[sl]).norm() / b_[sl].norm() < 5e-3, (hh, t0)
            assert (a[sl] - ref[sl]).norm() / ref[sl].norm() < 3e-2, (hh, t0)


@pytest.mark.parametrize("dtype,D", [(torch.float16, 128), (torch.bfloat16, 64)])
def test_null_keys_int8(gpu, dtype, D):
    """``attention_blhd(..., "int8_turing", null_keys=n)`` (Anima's callers,
    anima_dit.py:304; reference test_attention_dispatch.py:303-305): the n
    all-zero key/value rows are padded back before the INT8 kernels run, so
    the call equals the INT8 call on the padded K/V bit for bit, and stays
    within the oracle bound on those padded inputs and the reference's SDPA
    bar."""
    B, Lq, Lk, H, n = 2, 300, 500, 3, 7
    q, k, v = _inputs(B, Lq, Lk, H, D, dtype, seed=5)
    qd, kd, vd = q.to(gpu), k.to(gpu), v.to(gpu)
    out = A.attention_blhd(qd, kd, vd, "int8_turing", null_keys=n)
    pad = (0, 0, 0, 0, 0, n)
    kp, vp = F.pad(kd, pad), F.pad(vd, pad)
    want = A.attention_blhd(qd, kp, vp, "int8_turing")
    assert torch.equal(out, want)
    assert not torch.equal(out, A.attention_blhd(qd, kd, vd, "int8_turing"))
    o = np32(out).reshape(B, Lq, H, D)
    ora = OA.int8_attention(np32(q), np32(kp), np32(vp), D ** -0.5, DT[dtype], DT[dtype])
    assert rel_l2(o, ora) < ORACLE_REL[dtype] and cosine(o, ora) > ORACLE_COS
    ref = np32(_ref_blhd(q.float().to(gpu), kp.float(), vp.float()))
    assert rel_l2(o, ref) < 3e-2 and cosine(o, ref) > 0.9995


@pytest.mark.parametrize("B,H,L,D,dtype,sk", [(2, 10, 4096, 64, torch.float16, True),
                                                (1, 4, 1024, 128, torch.float16, False),
                                                (1, 4, 4096, 128, torch.float16, True)])
def test_growing_logits_rescale_128_query_tiles(gpu, B, H, L, D, dtype, sk):
    """The growing-logits case (row maxima rising from ~8 to ~100 over the key
    range, so the lazy maximum rescales O every few tiles; an unrescaled
    float16 P would overflow) on 128-query tiles: at head dim 64 with the
    DMA-fed kernel's stream-K pieces and their merge (SDXL's 2 x 10 heads at
    4096 tokens), and at head dim 128 on grids too small for 256-query tiles
    (the register-staged kernel, whole tiles and stream-K pieces). Finite, and
    within the oracle bound."""
    pl = A.attn_plan(B, H, L, L, D, dtype)
    if torch.cuda.get_device_properties(gpu).multi_processor_count == 256:
        assert (pl["sk_blocks"] > 0) == sk
        assert pl["dp_tiles"] + pl["sk_tiles"] == B * H * L // 128
    g = torch.Generator().manual_seed(4)
    u = torch.randn(D, generator=g)
    u /= u.norm()
    q = (8 * u + 0.1 * torch.randn(B, L, H, D, generator=g)).to(dtype)
    k = (100 * torch.linspace(0, 1, L).view(1, L, 1, 1) * u + torch.randn(B, L, H, D, generator=g)).to(dtype)
    v = torch.randn(B, L, H, D, generator=g).to(dtype)
    out, _ = _run(q, k, v, gpu)
    assert torch.isfinite(out).all()
    # the last batch's last 2 heads: query tiles past the whole rounds, which
    # the stream-K pieces run where there are any (the oracle is per (batch, head))
    sl = (slice(B - 1, B), slice(None), slice(H - 2, H))
    o = np32(out[sl])
    ora = OA.int8_attention(np32(q[sl]), np32(k[sl]), np32(v[sl]), D ** -0.5, DT[dtype], DT[dtype])
    r, c = rel_l2(o, ora), cosine(o, ora)
    print(f"[attn] growing logits 128-query tiles {B},{H},{L},{D}: vs oracle rel {r:.2e} cos {c:.7f}")
    assert r < ORACLE_REL[dtype] and c > ORACLE_COS


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("D", [64, 40])
def test_growing_logits_rescale_dma_kernel_head_dim_64(gpu, D, dtype):
    """The growing-logits case on the DMA-fed kernel at Dp = 64 (4 waves, 128
    query rows per workgroup): a plan without stream-K pieces, row maxima
    rising from ~8 to ~100 over the keys, so O is rescaled every few tiles.
    Finite, and within the oracle bound."""
    B, H, L = 1, 4, 1024
    assert A.attn_plan(B, H, L, L, D, dtype) == {"dp_tiles": B * H * L // 128, "sk_blocks": 0, "sk_tiles": 0}
    g = torch.Generator().manual_seed(5)
    u = torch.randn(D, generator=g)
    u /= u.norm()
    q = (8 * u + 0.1 * torch.randn(B, L, H, D, generator=g)).to(dtype)
    k = (100 * torch.linspace(0, 1, L).view(1, L, 1, 1) * u + torch.randn(B, L, H, D, generator=g)).to(dtype)
    v = torch.randn(B, L, H, D, generator=g).to(dtype)
    out, _ = _run(q, k, v, gpu)
    assert torch.isfinite(out).all()
    o = np32(out)
    ora = OA.int8_attention(np32(q), np32(k), np32(v), D ** -0.5, DT[dtype], DT[dtype])
    r, c = rel_l2(o, ora), cosine(o, ora)
    print(f"[attn] growing logits Dp 64 DMA kernel D {D} {DT[dtype]}: vs oracle rel {r:.2e} cos {c:.7f}")
    assert r < ORACLE_REL[dtype] and c > ORACLE_COS


@pytest.mark.parametrize("H,D", [(256, 128), (64, 64)])
def test_long_v_row_stride_takes_128_query_kernel(gpu, H, D):
    """A V whose row stride puts a 64-key tile past 2^31 bytes (the DMA-fed
    kernel's 32-bit offsets) runs the 128-query register-staged kernel with
    whole tiles: same inputs, V laid out with an L-stride of 2^23 elements,
    against the same V contiguous, within the oracle bound of each other. At
    head dim 128 the grid is one that otherwise takes 256-query tiles; at 64
    one that otherwise takes the 4-wave DMA-fed kernel."""
    B, Lq, Lk, dtype = 1, 512, 130, torch.bfloat16
    pl = A.attn_plan(B, H, Lq, Lk, D, dtype)
    if pl["sk_blocks"] or (D == 128 and pl["dp_tiles"] != B * H * 2):
        pytest.skip("this grid does not take the DMA-fed kernel on this device")
    q, k, v = _inputs(B, Lq, Lk, H, D, dtype, seed=8)
    qd, kd, vd = q.to(gpu), k.to(gpu), v.to(gpu)
    vsl = 1 << 23
    store = torch.zeros((Lk - 1) * vsl + H * D, device=gpu, dtype=dtype)
    vs = store.as_strided((B, Lk, H, D), (Lk * vsl, vsl, D, 1))
    vs.copy_(vd)
    ws = torch.empty(A.workspace_bytes(B, H, Lq, Lk, D), device=gpu, dtype=torch.uint8)
    out = A.int8_attention(qd, kd, vs, D ** -0.5, workspace=ws)
    base = A.int8_attention(qd, kd, vd, D ** -0.5, workspace=ws)
    assert np.isfinite(np32(out)).all()
    assert rel_l2(np32(out), np32(base)) < ORACLE_REL[dtype]
    ora = OA.int8_attention(np32(q), np32(k), np32(v), D ** -0.5, DT[dtype], DT[dtype])
    assert rel_l2(np32(out), ora) < ORACLE_REL[dtype] and cosine(np32(out), ora) > ORACLE_COS
