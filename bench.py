"""Benchmark: INT8 attention + W8A8 GEMM TOPS at FLUX 1024^2 on one MI355X.

A step is one pass of the hot path of one FLUX.1-schnell denoise step at
1024 x 1024 (4096 image + 512 text tokens, 24 heads of 128): in forward order,
19 double-stream blocks (img/txt qkv, joint INT8 attention, img/txt proj,
img/txt MLP up and down) and 38 single-stream blocks (linear1, INT8 attention,
linear2). Every linear is a W8A8 ``Int8Linear`` with its own random weights
(quantize kernel + fused-epilogue GEMM; a double block's img linear and its
txt twin share one grouped GEMM launch where the library's plan expects that
to pay, as flux_step runs them); every attention is
``attention_bhld(..., "int8_turing")``. Algorithmic work is 74.36 TOP per
step (GEMM 2*M*N*K, attention 4*B*H*S^2*D). Inputs are resident in HBM.

The timed steps issue the calls one by one from Python with no events between
them. (Replaying the step captured as a HIP graph measured the same time: the
host stays ahead of the GPU.) A separate pass of as many steps carries HIP
events around every kernel call (on torch's current stream, where the kernels
run) for the per-kernel times: GEMM, attention, quantize, and GEMM per kernel
plan. The roofline is reported for the DMA-fed 256 x 256 GEMM kernel (the
largest share of the step): algorithmic 2*M*N*K ops and M*K + N*K + 2*M*N +
scale/bias bytes per launch, averaged over its launches, over its average
launch time.

The same run also measures, and adds to the JSON line:
  * the full synthetic FLUX-schnell denoise step (flux_step.py) with INT8
    attention + W8A8 linears against the same step with bf16 SDPA and bf16
    linears, ms per step and the final-latent deviation after 4 steps;
  * the reference's CPU path (torch CPU ops, oracle/cpu_path.py) on a bounded
    row sample of the same workload;
  * the MFMA-only throughput this device sustains (dc_mfma_probe), next to
    the published peak in the roofline object.

Benchmark configs (the shapes --shapes and --cpu-configs cover):
  1. a W8A8 linear on x fp32 [8192, 320] with outlier channels, W [1280, 320],
     group 0, fp32 out (the reference's CPU-runnable case);
  2. SD1.5 at 512^2: self-attention 2 x 8 x 4096 (D 40), cross-attention over
     77 context tokens, the transformer block's W8A8 linears;
  3. SDXL at 1024^2: self-attention 2 x 10 x 4096 and 2 x 20 x 1024 (D 64),
     cross-attention, the block's linears;
  4. FLUX.1 at 1024^2, per call: joint attention 1 x 24 x 4608 (D 128, bf16)
     and every W8A8 linear shape;
  5. one FLUX.1-schnell denoise step (the hot path above, and flux_step.py).

    python bench.py [--steps K] [--warmup W] [--no-full] [--no-cpu]
    python bench.py --copy-calibration   # 1 GiB device copy for counter scaling
    python bench.py --cpu-configs        # the reference's CPU path at every config shape (host cores only)
    python bench.py --mfma-ceiling       # MFMA-only throughput (int8, bf16)
    python bench.py --shapes             # per-shape report for every benchmark config (+ the GEMM A/B)
    python bench.py --gemm-ab            # same-process GEMM A/B against torch._int_mm (hipBLASLt)
"""

from __future__ import annotations

import argparse
import ctypes
import hashlib
import json
import os
import platform
import sys
import time
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "INT8 attn + W8A8 GEMM TOPS (% int8 MFMA peak) at FLUX 1024²; ms/denoise step"
INT8_PEAK_TOPS = 5000.0        # MI355X dense int8 MFMA
HBM_PEAK_GBS = 8000.0


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


# ---------------------------------------------------------------- hot path

class HotPath:
    """The hot-path calls of one FLUX denoise step, in forward order."""

    def __init__(self, model, shape, device):
        from diffucore_amd import _int8
        self.ops = []   # (kind, fn_quant, fn_gemm or fn_attn, algorithmic ops, bytes for quant)
        dt = torch.bfloat16
        g = torch.Generator(device=device).manual_seed(1)
        n_img = shape.img_hw[0] * shape.img_hw[1]
        L = n_img + shape.txt_len
        H, D, h, m = shape.heads, shape.head_dim, shape.hidden, shape.mlp

        def act(rows, cols):
            return torch.randn(rows, cols, generator=g, device=device).to(dt)

        self.acts = {
            "img": act(n_img, h), "txt": act(shape.txt_len, h), "img_h": act(n_img, m), "txt_h": act(shape.txt_len, m),
            "x": act(L, h), "x_h": act(L, h + m),
        }
        qkv = [torch.randn(1, H, L, D, generator=g, device=device).to(dt) for _ in range(3)]
        qkv[1] += 0.5
        self.qkv = qkv
        attn_ops = 4 * 1 * H * L * L * D

        def lin(layer, key):
            x = self.acts[key]
            return ("gemm", layer, x, 2 * x.shape[0] * layer.out_features * layer.in_features)

        def pair(la, ka, lb, kb):
            # a double block's img linear and its txt twin: one grouped launch
            # when the library's plan expects it to pay, as flux_step runs them
            xa, xb = self.acts[ka], self.acts[kb]
            if _int8.gemm_group_plan([xa.shape[0], xb.shape[0]], la.out_features, la.in_features):
                return [("group", (la, lb), (xa, xb), 2 * (xa.shape[0] + xb.shape[0]) * la.out_features * la.in_features)]
            return [lin(la, ka), lin(lb, kb)]

        for blk in model.double_blocks:
            self.ops += pair(blk.img_qkv, "img", blk.txt_qkv, "txt")
            self.ops.append(("attn", None, None, attn_ops))
            self.ops += pair(blk.img_proj, "img", blk.txt_proj, "txt")
            self.ops += pair(blk.img_mlp[0], "img", blk.txt_mlp[0], "txt")
            self.ops += pair(blk.img_mlp[2], "img_h", blk.txt_mlp[2], "txt_h")
        for blk in model.single_blocks:
            self.ops.append(lin(blk.linear1, "x"))
            self.ops.append(("attn", None, None, attn_ops))
            self.ops.append(lin(blk.linear2, "x_h"))
        assert all(isinstance(op[1], _int8.Int8Linear) for op in self.ops if op[0] == "gemm")
        assert all(isinstance(la, _int8.Int8Linear) for op in self.ops if op[0] == "group" for la in op[1])
        self.total_ops = sum(op[3] for op in self.ops)
        # which GEMM kernel each launch runs (dc_w8a8_gemm_plan; grouped
        # launches always run the DMA-fed 256 x 256 kernel)
        self.plans = [_int8.gemm_plan(op[2].shape[0], op[1].out_features, op[1].in_features) if op[0] == "gemm"
                      else "dma_256x256" if op[0] == "group" else None for op in self.ops]
        self.ws = None

    def run(self, recs=None):
        """One step. With ``recs`` (a list), HIP events on torch's current
        stream (where every kernel of this package is launched) bracket each
        quantize, GEMM and attention call and are appended as
        ``(kind, start, end, ops, bytes, gemm plan or None)``."""
        from diffucore_amd import _int8, attention_bhld
        q, k, v = self.qkv
        if recs is None:
            for kind, layer, x, _ in self.ops:
                if kind == "gemm":
                    layer.matmul_quantized(*_int8.quantize_activation(x, layer.group), x.dtype)
                elif kind == "group":
                    qs = [_int8.quantize_activation(xi, li.group) for li, xi in zip(layer, x)]
                    _int8.matmul_quantized_group([(li, *qi) for li, qi in zip(layer, qs)], x[0].dtype)
                else:
                    attention_bhld(q, k, v, "int8_turing")
            return
        for (kind, layer, x, ops), plan in zip(self.ops, self.plans):
            if kind == "group":
                ev = [torch.cuda.Event(enable_timing=True) for _ in range(len(x) + 2)]
                ev[0].record()
                qs = []
                for i, (li, xi) in enumerate(zip(layer, x)):
                    qs.append(_int8.quantize_activation(xi, li.group))
                    ev[i + 1].record()
                    recs.append(("quant", ev[i], ev[i + 1], 0, xi.numel() * xi.element_size() + xi.numel() +
                                 4 * xi.shape[0], None))
                _int8.matmul_quantized_group([(li, *qi) for li, qi in zip(layer, qs)], x[0].dtype)
                ev[-1].record()
                K, N = layer[0].in_features, layer[0].out_features
                gbytes = sum(xi.shape[0] * K + N * K + 4 * (xi.shape[0] + N) + 2 * N + 2 * xi.shape[0] * N for xi in x)
                recs.append(("gemm", ev[len(x)], ev[-1], ops, gbytes, plan))
            elif kind == "gemm":
                e0, e1, e2 = (torch.cuda.Event(enable_timing=True) for _ in range(3))
                e0.record()
                qx, sx = _int8.quantize_activation(x, layer.group)
                e1.record()
                layer.matmul_quantized(qx, sx, x.dtype)
                e2.record()
                qbytes = x.numel() * x.element_size() + x.numel() + 4 * x.shape[0]
                M, K, N = x.shape[0], x.shape[1], layer.out_features
                gbytes = M * K + N * K + 4 * (M + N) + (2 * N) + 2 * M * N
                recs.append(("quant", e0, e1, 0, qbytes, None))
                recs.append(("gemm", e1, e2, ops, gbytes, plan))
            else:
                e0, e1 = (torch.cuda.Event(enable_timing=True) for _ in range(2))
                e0.record()
                attention_bhld(q, k, v, "int8_turing")
                e1.record()
                recs.append(("attn", e0, e1, ops, 0, None))


def summarize(recs):
    """Per-kernel totals over recorded events; GEMM launches are also totalled
    per kernel plan (``gemm_<plan>``, from dc_w8a8_gemm_plan)."""
    out = {}
    for kind, a, b, ops, nbytes, plan in recs:
        for key in (kind, f"gemm_{plan}") if plan else (kind,):
            d = out.setdefault(key, {"ms": 0.0, "ops": 0, "bytes": 0, "launches": 0})
            d["ms"] += a.elapsed_time(b)
            d["ops"] += ops
            d["bytes"] += nbytes
            d["launches"] += 1
    return out


def time_steps(fn, steps, warmup):
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def copy_calibration(mib: int = 1024, reps: int = 5):
    """A plain device copy of ``mib`` MiB, ``reps`` times: the known-size
    kernel that scales rocprofv3's FETCH_SIZE / WRITE_SIZE counters."""
    src = torch.ones(mib << 18, device="cuda", dtype=torch.float32)
    dst = torch.empty_like(src)
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes_each_way": mib << 20, "reps": reps}), flush=True)


# ---------------------------------------------------------------- CPU baseline

def mfma_ceiling(iters: int = 100000) -> dict:
    """Measured MFMA throughput of this device (dc_mfma_probe): back-to-back
    independent MFMAs with nothing else in the loop, one workgroup per CU,
    1 or 2 waves per SIMD, constant or changing operands. The published
    peaks (int8 5.0 POP/s, bf16 2.5 PFLOP/s) assume the peak engine clock;
    under this load the chip runs at its power limit, lower with operands that
    change from one MFMA to the next (as real data does)."""
    from diffucore_amd import _lib
    L = _lib.require()
    units = L.dc_mfma_probe_units()
    sink = torch.empty(units * 8, dtype=torch.int32, device="cuda")
    stream = torch.cuda.current_stream()
    out = {"units": units, "iters": iters, "what": "TOP/s (int8) and TFLOP/s (bf16) of back-to-back independent "
           "MFMAs, one workgroup per CU; 'vary' = operands change every MFMA (per-lane hashed int8 codes / bf16 "
           "values of magnitude 0.5-2), 'const' = one operand pair reused"}
    for kind, name, per in ((0, "int8_32x32x32", 65536), (1, "bf16_32x32x16", 32768)):
        for vary in (0, 1):
            for waves in (1, 2):
                def launch(n):
                    rc = L.dc_mfma_probe(kind, vary, waves, n, ctypes.c_void_p(sink.data_ptr()),
                                         ctypes.c_void_p(stream.cuda_stream))
                    if rc:
                        raise RuntimeError(L.dc_last_error().decode())
                launch(iters // 10)
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                launch(iters)
                e1.record()
                torch.cuda.synchronize()
                s = e0.elapsed_time(e1) * 1e-3
                rate = units * 4 * waves * iters * 8 * per / s / 1e12
                out[f"{name}_{'vary' if vary else 'const'}_{waves}w"] = round(rate, 1)
    return out


def cpu_baseline(shape, budget_s: float = 12.0, rows: int = 256):
    """The reference's CPU path (oracle/cpu_path.py) on a row sample of one
    double + one single block: W8A8 linears on ``rows`` activation rows and
    attention for ``rows`` queries over all 4608 keys and 24 heads, repeated
    until ``budget_s`` has elapsed."""
    from oracle import cpu_path as C
    torch.set_num_threads(os.cpu_count() or 1)
    g = torch.Generator().manual_seed(0)
    h, m, H, D = shape.hidden, shape.mlp, shape.heads, shape.head_dim
    L = shape.img_hw[0] * shape.img_hw[1] + shape.txt_len
    lin_shapes = [(3 * h, h)] * 2 + [(h, h)] * 2 + [(m, h), (h, m)] * 2 + [(3 * h + m, h), (h, h + m)]
    weights = []
    for n, k in lin_shapes:
        w = torch.randn(n, k, generator=g) * 0.02
        q, s = C.quantize_rows(C.rotate(w, 256))
        x = torch.randn(rows, k, generator=g).to(torch.bfloat16)
        weights.append((x, q, s, (torch.randn(n, generator=g) * 0.02).to(torch.bfloat16)))
    qa = torch.randn(1, H, rows, D, generator=g)
    ka = torch.randn(1, H, L, D, generator=g)
    va = torch.randn(1, H, L, D, generator=g)
    ops_per = sum(2 * rows * n * k for n, k in lin_shapes) + 2 * 4 * H * rows * L * D
    done, t0 = 0, time.perf_counter()
    while True:
        for x, q, s, b in weights:
            C.w8a8_linear(x, q, s, b, 256)
        for _ in range(2):
            C.attention_bhld(qa, ka, va)
        done += 1
        el = time.perf_counter() - t0
        if el >= budget_s:
            break
    tops = done * ops_per / el / 1e12
    cfg1 = cpu_cfg1()
    cpu = platform.processor() or "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {
        "value": round(tops, 4), "unit": "TOPS", "cores": torch.get_num_threads(), "kind": "port",
        "sample": (f"reference CPU path (torch ops: rotate+quantize_rows, torch._int_mm, rescale; fp32 SDPA) on "
                   f"one double + one single FLUX block with {rows} activation rows per linear and {rows} "
                   f"queries x {L} keys x {H} heads per attention, {done} repetitions in {el:.1f} s; "
                   f"cpu '{cpu}', os.cpu_count()={os.cpu_count()}"),
        "cfg1": cfg1,
    }


def gemm_source_sha256() -> str:
    return hashlib.sha256((ROOT / "diffucore_amd" / "csrc" / "gemm.hip").read_bytes()).hexdigest()


def traffic_summary(root: Path) -> None:
    """Per-dispatch HBM traffic from rocprofv3 --pmc runs (one counter each):
    root/copy_FETCH_SIZE, root/copy_WRITE_SIZE (a 1 GiB device copy, from
    --copy-calibration) calibrate the counters; root/step_FETCH_SIZE,
    root/step_WRITE_SIZE (one hot-path step) are averaged per kernel and
    scaled. Writes profiles/gemm_flux_step_traffic.json, stamped with the GEMM
    source's hash so bench runs on other sources leave `traffic` null."""
    import csv
    import glob

    def per_kernel(d):
        acc = {}
        for f in glob.glob(str(root / d / "**" / "*counter_collection.csv"), recursive=True):
            for r in csv.DictReader(open(f)):
                a = acc.setdefault(r["Kernel_Name"], [0.0, 0])
                a[0] += float(r["Counter_Value"])
                a[1] += 1
        return {k: (v[0] / v[1], v[1]) for k, v in acc.items()}

    cf, cw = per_kernel("copy_FETCH_SIZE"), per_kernel("copy_WRITE_SIZE")
    copy_k = next(k for k in cf if "copyBuffer" in k)
    copy_bytes = 1024 << 20
    fetch_scale = copy_bytes / (cf[copy_k][0] * 1024)
    write_scale = copy_bytes / (cw[copy_k][0] * 1024)
    sf, sw = per_kernel("step_FETCH_SIZE"), per_kernel("step_WRITE_SIZE")
    kernels = {}
    for k in sf:
        if "dc::" not in k:
            continue
        name = k.split("(")[0].replace("void ", "")
        kernels[name] = {"dispatches": sf[k][1], "fetch_bytes": int(sf[k][0] * 1024 * fetch_scale),
                         "write_bytes": int(sw.get(k, (0, 0))[0] * 1024 * write_scale)}
    dma = next(v for k, v in kernels.items() if "w8a8_gemm_dma_kernel" in k)
    out = {"kernel": next(k for k in kernels if "w8a8_gemm_dma_kernel" in k),
           "hbm_bytes_per_launch": dma["fetch_bytes"] + dma["write_bytes"],
           "fetch_bytes_per_launch": dma["fetch_bytes"], "write_bytes_per_launch": dma["write_bytes"],
           "fetch_scale": round(fetch_scale, 4), "write_scale": round(write_scale, 4),
           "calibration": f"1 GiB device copy: FETCH_SIZE {cf[copy_k][0]:.1f} KiB, WRITE_SIZE {cw[copy_k][0]:.1f} "
                          f"KiB per dispatch",
           "kernel_source_sha256": gemm_source_sha256(), "per_kernel": kernels}
    (ROOT / "profiles" / "gemm_flux_step_traffic.json").write_text(json.dumps(out, indent=1) + "\n")
    print(json.dumps({k: out[k] for k in ("kernel", "hbm_bytes_per_launch", "fetch_scale", "write_scale")}))


def cpu_cfg1(budget_s: float = 4.0):
    """Benchmark config 1 on the reference's CPU path: W8A8 linear on x fp32
    [8192, 320] ~N(0, 1) with 2 of 320 channels (0.5%) scaled x20 as outliers,
    W [1280, 320] ~N(0, 0.02), per-token int8 activations, per-channel int8
    weights, group 0, int32 accumulate, fp32 out, seed 0 (generator draws:
    x, outlier channels, W). Timed over ``budget_s`` on all host threads."""
    from oracle import cpu_path as C
    torch.set_num_threads(os.cpu_count() or 1)
    g = torch.Generator().manual_seed(0)
    x = torch.randn(8192, 320, generator=g)
    x[:, torch.randperm(320, generator=g)[:2]] *= 20
    w = torch.randn(1280, 320, generator=g) * 0.02
    q, s = C.quantize_rows(w)
    C.w8a8_linear(x, q, s, None, 0)
    n, t0 = 0, time.perf_counter()
    while True:
        C.w8a8_linear(x, q, s, None, 0)
        n += 1
        el = time.perf_counter() - t0
        if el >= budget_s:
            break
    ms = el / n * 1e3
    return {"what": "W8A8 linear x fp32 [8192,320] (0.5% outlier channels x20), W [1280,320], group 0, fp32 out: "
                    "quantize_rows -> torch._int_mm -> rescale on the CPU",
            "ms_per_call": round(ms, 3), "TOPS": round(2 * 8192 * 1280 * 320 / (ms * 1e-3) / 1e12, 4),
            "cores": torch.get_num_threads(), "calls": n}


def cpu_configs(budget_s: float = 2.0) -> None:
    """The reference's CPU path (oracle/cpu_path.py: the W8A8 linear as
    quantize_rows(rotate(x)) -> torch._int_mm -> rescale; attention as fp32
    SDPA, where the int8 backend falls through on CPU) at each benchmark config
    shape, on all host threads. Each shape runs on a sample of its rows or
    queries (all keys, all heads) for about ``budget_s`` and is scaled to the
    full call by its share of the work; one JSON line per shape."""
    from oracle import cpu_path as C
    torch.set_num_threads(os.cpu_count() or 1)
    g = torch.Generator().manual_seed(0)

    def timed(fn):
        fn()
        n, t0 = 0, time.perf_counter()
        while True:
            fn()
            n += 1
            el = time.perf_counter() - t0
            if el >= budget_s:
                return el / n

    def attn(name, B, H, Sq, Skv, D, rows):
        rows = min(rows, Sq)
        q = torch.randn(B, H, rows, D, generator=g)
        k = torch.randn(B, H, Skv, D, generator=g)
        v = torch.randn(B, H, Skv, D, generator=g)
        t = timed(lambda: C.attention_bhld(q, k, v)) * Sq / rows
        print(json.dumps({"kind": "cpu_attention", "shape": name, "B": B, "H": H, "Sq": Sq, "Skv": Skv, "D": D,
                          "sample_queries": rows, "ms_per_call": round(t * 1e3, 3),
                          "TOPS": round(4 * B * H * Sq * Skv * D / t / 1e12, 4), "cores": torch.get_num_threads()}),
              flush=True)

    def lin(name, M, K, N, group, dtype, rows):
        rows = min(rows, M)
        w = torch.randn(N, K, generator=g) * 0.02
        w8, sw = C.quantize_rows(C.rotate(w, group) if group else w)
        x = torch.randn(rows, K, generator=g).to(dtype)
        b = (torch.randn(N, generator=g) * 0.02).to(dtype)
        t = timed(lambda: C.w8a8_linear(x, w8, sw, b, group)) * M / rows
        print(json.dumps({"kind": "cpu_w8a8_linear", "shape": name, "M": M, "K": K, "N": N, "group": group,
                          "sample_rows": rows, "ms_per_call": round(t * 1e3, 3),
                          "TOPS": round(2 * M * N * K / t / 1e12, 4), "cores": torch.get_num_threads()}),
              flush=True)

    cfg1 = cpu_cfg1(budget_s)
    print(json.dumps({"kind": "cpu_w8a8_linear", "shape": "cfg1_sd15_ff", "M": 8192, "K": 320, "N": 1280, "group": 0,
                      "sample_rows": 8192, **{k: cfg1[k] for k in ("ms_per_call", "TOPS", "cores")}}), flush=True)
    for name, B, H, Sq, Skv, D, _dt, _off in ATTN_SHAPES:
        attn(name, B, H, Sq, Skv, D, 256 if Skv > 1000 else Sq)
    for name, M, K, N, dt in LIN_SHAPES:
        lin(name, M, K, N, 256 if K % 256 == 0 else 0, dt, 256)


# ---------------------------------------------------------------- per-shape report

ATTN_SHAPES = [
    # name, B, H, Sq, Skv, D, dtype, per-channel K offset std (UNet recipe) or 0
    ("sd15_self", 2, 8, 4096, 4096, 40, torch.float16, 2.0),
    ("sd15_cross", 2, 8, 4096, 77, 40, torch.float16, 2.0),
    ("sdxl_self_4096", 2, 10, 4096, 4096, 64, torch.float16, 2.0),
    ("sdxl_self_1024", 2, 20, 1024, 1024, 64, torch.float16, 2.0),
    ("sdxl_cross_4096", 2, 10, 4096, 77, 64, torch.float16, 2.0),
    ("sdxl_cross_1024", 2, 20, 1024, 77, 64, torch.float16, 2.0),
    ("flux_joint", 1, 24, 4608, 4608, 128, torch.bfloat16, 0.0),
]

LIN_SHAPES = [
    # name, M, K, N, dtype (activations and output)
    ("sd15_ff", 8192, 320, 1280, torch.float32),
    ("sdxl_qkvo_4096", 8192, 640, 640, torch.float16),
    ("sdxl_qkvo_1024", 2048, 1280, 1280, torch.float16),
    ("sdxl_cross_kv_640", 154, 2048, 640, torch.float16),
    ("sdxl_cross_kv_1280", 154, 2048, 1280, torch.float16),
    ("sdxl_geglu_4096", 8192, 640, 5120, torch.float16),
    ("sdxl_ffout_4096", 8192, 2560, 640, torch.float16),
    ("sdxl_geglu_1024", 2048, 1280, 10240, torch.float16),
    ("sdxl_ffout_1024", 2048, 5120, 1280, torch.float16),
    ("flux_img_qkv", 4096, 3072, 9216, torch.bfloat16),
    ("flux_img_proj", 4096, 3072, 3072, torch.bfloat16),
    ("flux_img_mlp_up", 4096, 3072, 12288, torch.bfloat16),
    ("flux_img_mlp_down", 4096, 12288, 3072, torch.bfloat16),
    ("flux_txt_qkv", 512, 3072, 9216, torch.bfloat16),
    ("flux_txt_mlp_down", 512, 12288, 3072, torch.bfloat16),
    ("flux_single_linear1", 4608, 3072, 21504, torch.bfloat16),
    ("flux_single_linear2", 4608, 15360, 3072, torch.bfloat16),
]


def per_call_ms(fn, reps: int = 20) -> float:
    """Median of ``reps`` calls, each bracketed by HIP events on the current stream."""
    for _ in range(3):
        fn()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
    for a, b in ev:
        a.record()
        fn()
        b.record()
    torch.cuda.synchronize()
    t = sorted(a.elapsed_time(b) for a, b in ev)
    return t[reps // 2]


def unet_compiled(dev):
    """The UNet transformer block (unet_block.py) at SD1.5 / SDXL shapes:
    fp16 eager, the fp16 block under torch.compile (inductor; compile time
    excluded) and the W8A8 + INT8 block, per call (HIP events around each
    call, launch cost included) and as device time (the block captured in a
    HIP graph; None where capture fails). One JSON line per level."""
    import copy
    import unet_block as UB
    for lv in UB.LEVELS:
        blk = UB.build(lv, dev)
        x, ctx = UB.inputs(lv, dev)
        with torch.no_grad():
            qb = UB.to_int8(copy.deepcopy(blk), dev)
            cb = torch.compile(blk)
            t0 = time.perf_counter()
            cb(x, ctx)
            torch.cuda.synchronize()
            compile_s = time.perf_counter() - t0
            log(f"unet block {lv.name}: compiled in {compile_s:.0f} s")
            ref, out_c = blk(x, ctx) - x, cb(x, ctx) - x
            row = {"kind": "unet_block_compiled", "shape": lv.name, "dtype": "float16",
                   "compile_s": round(compile_s, 1)}
            for name, fn in (("fp16_eager", lambda: blk(x, ctx)), ("fp16_compiled", lambda: cb(x, ctx)),
                             ("int8", lambda: qb(x, ctx))):
                row[f"{name}_ms"] = round(per_call_ms(fn), 4)
                try:
                    row[f"{name}_graph_ms"] = round(graph_call_ms(fn, reps=5), 4)
                except RuntimeError as e:
                    print(f"[bench] unet block {lv.name} {name}: graph capture failed: {e}", file=sys.stderr,
                          flush=True)
                    row[f"{name}_graph_ms"] = None
            row["compiled_vs_eager"] = _cmp(out_c, ref)
        print(json.dumps(row), flush=True)
        del blk, qb, cb, x, ctx
        torch._dynamo.reset()


GEMM_AB_SHAPES = [
    # FLUX's W8A8 linears: name, M, K, N (bf16 activations and output, bias, ConvRot 256)
    ("flux_img_qkv", 4096, 3072, 9216),
    ("flux_img_proj", 4096, 3072, 3072),
    ("flux_img_mlp_up", 4096, 3072, 12288),
    ("flux_img_mlp_down", 4096, 12288, 3072),
    ("flux_single_linear1", 4608, 3072, 21504),
    ("flux_single_linear2", 4608, 15360, 3072),
    ("flux_txt_mlp_up", 512, 3072, 12288),
]


def gemm_vendor_ab(dev):
    """Same process, same ConvRot codes: the reference's ROCm int_mm (torch._int_mm
    on the transposed weight view, _int8.py:200-207, which runs hipBLASLt) alone
    and followed by rescale's torch ops (_int8.py:322-323), against this
    library's int32 GEMM and its fused-epilogue GEMM, each timed as GPU time
    per call over a captured graph of back-to-back calls. One JSON line per
    shape."""
    from diffucore_amd import Int8Linear, int_mm, quantize_activation
    dt = torch.bfloat16
    g = torch.Generator(device=dev)
    for name, M, K, N in GEMM_AB_SHAPES:
        g.manual_seed(0)
        x = torch.randn(M, K, generator=g, device=dev).to(dt)
        lin = torch.nn.Linear(K, N, device=dev)
        lin.weight.normal_(0, 0.02, generator=g)
        lin.bias.normal_(0, 0.02, generator=g)
        m = Int8Linear.from_linear(lin, 256)
        m.bias.data = m.bias.data.to(dt)
        qx, sx = quantize_activation(x, 256)
        wt = m.weight.t()
        sw = m.scale

        def vendor_rescale():
            acc = torch._int_mm(qx, wt)
            return (acc.float() * (sx[:, None] * sw[None, :])).to(dt) + m.bias

        ms_v = graph_call_ms(lambda: torch._int_mm(qx, wt))
        ms_vr = graph_call_ms(vendor_rescale)
        ms_i = graph_call_ms(lambda: int_mm(qx, m.weight))
        ms_f = graph_call_ms(lambda: m.matmul_quantized(qx, sx, dt))
        same_acc = bool(torch.equal(torch._int_mm(qx, wt), int_mm(qx, m.weight)))
        same_out = bool(torch.equal(vendor_rescale(), m.matmul_quantized(qx, sx, dt)))
        ops = 2 * M * N * K

        def tops(ms):
            return round(ops / (ms * 1e-3) / 1e12, 1)

        print(json.dumps({"kind": "gemm_vs_vendor", "shape": name, "M": M, "K": K, "N": N,
                          "plan": __import__("diffucore_amd")._int8.gemm_plan(M, N, K),
                          "torch_int_mm_ms": round(ms_v, 4), "torch_int_mm_TOPS": tops(ms_v),
                          "torch_int_mm_rescale_ms": round(ms_vr, 4),
                          "dc_int32_ms": round(ms_i, 4), "dc_int32_TOPS": tops(ms_i),
                          "dc_fused_bf16_ms": round(ms_f, 4), "dc_fused_bf16_TOPS": tops(ms_f),
                          "fused_vs_int_mm": round(ms_v / ms_f, 3),
                          "int32_equal": same_acc, "fused_equals_int_mm_rescale": same_out}), flush=True)
        del x, lin, m, qx, sx, wt


def graph_call_ms(fn, reps: int = 20) -> float:
    """GPU time per call of ``fn`` with no host launch cost: ``reps`` back-to-back
    calls captured in one HIP graph, the median of 7 replays divided by
    ``reps`` (a call's launches, and the gaps between them, included)."""
    fn()
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(reps):
            fn()
    g.replay()
    torch.cuda.synchronize()
    ts = []
    for _ in range(7):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        g.replay()
        b.record()
        torch.cuda.synchronize()
        ts.append(a.elapsed_time(b) / reps)
    return sorted(ts)[3]


def _cmp(y, ref):
    a, b = y.float().flatten(), ref.float().flatten()
    return {"max_abs": float((a - b).abs().max()), "rel_l2": float((a - b).norm() / b.norm()),
            "cos": float(a @ b / (a.norm() * b.norm()))}


def attn_calls(dev, calls: int = 5):
    """``calls`` INT8 attention calls at each benchmark config self-attention
    shape (the shapes report's tensors, no graphs, no timing): a short driver
    for rocprofv3 counter runs."""
    from diffucore_amd import attention_bhld
    from diffucore_amd._attention import SHORT_KEYS
    g = torch.Generator(device=dev)
    for name, B, H, S, Skv, D, dt, koff in ATTN_SHAPES:
        if Skv <= SHORT_KEYS:
            continue
        g.manual_seed(0)
        q = torch.randn(B, S, H * D, generator=g, device=dev).to(dt).view(B, S, H, D).transpose(1, 2)
        k = torch.randn(B, Skv, H, D, generator=g, device=dev)
        if koff:
            k = k + torch.randn(H, D, generator=g, device=dev) * koff
        k = k.to(dt).reshape(B, Skv, H * D).view(B, Skv, H, D).transpose(1, 2)
        v = torch.randn(B, Skv, H * D, generator=g, device=dev).to(dt).view(B, Skv, H, D).transpose(1, 2)
        for _ in range(calls):
            attention_bhld(q, k, v, "int8_turing")
        torch.cuda.synchronize()
        log(f"attention {name}: {calls} calls")


def shapes_report(dev):
    """One JSON line per benchmark config shape: time, TOPS, % of peak, accuracy."""
    import torch.nn.functional as F
    from diffucore_amd import Int8Linear, attention_bhld, quantize_activation
    from diffucore_amd._attention import SHORT_KEYS
    mixed_peak = 2.0 / (1.0 / INT8_PEAK_TOPS + 1.0 / 2500.0)
    g = torch.Generator(device=dev)
    for name, B, H, S, Skv, D, dt, koff in ATTN_SHAPES:
        g.manual_seed(0)
        # the UNet recipe: [B, S, H*D] tensors viewed (B, H, S, D) without a copy
        q = torch.randn(B, S, H * D, generator=g, device=dev).to(dt).view(B, S, H, D).transpose(1, 2)
        k = torch.randn(B, Skv, H, D, generator=g, device=dev)
        if koff:
            k = k + torch.randn(H, D, generator=g, device=dev) * koff
        k = k.to(dt).reshape(B, Skv, H * D).view(B, Skv, H, D).transpose(1, 2)
        v = torch.randn(B, Skv, H * D, generator=g, device=dev).to(dt).view(B, Skv, H, D).transpose(1, 2)
        ms = per_call_ms(lambda: attention_bhld(q, k, v, "int8_turing"))
        ms_gpu = graph_call_ms(lambda: attention_bhld(q, k, v, "int8_turing"))
        ms_sdpa = per_call_ms(lambda: F.scaled_dot_product_attention(q, k, v))
        # the reference's SDPA backend with the same (B, Sq, H*D) output
        ms_sdpa_path = per_call_ms(lambda: attention_bhld(q, k, v, "sdpa"))
        out = attention_bhld(q, k, v, "int8_turing")
        route = "sdpa (short key range)" if Skv <= SHORT_KEYS else "int8"
        ref = F.scaled_dot_product_attention(q.float(), k.float(), v.float()).transpose(1, 2).reshape(B, S, H * D)
        ops = 4 * B * H * S * Skv * D
        tops = ops / (ms_gpu * 1e-3) / 1e12
        print(json.dumps({"kind": "attention", "shape": name, "B": B, "H": H, "Sq": S, "Skv": Skv, "D": D,
                          "dtype": str(dt)[6:], "ms": round(ms, 4), "gpu_ms": round(ms_gpu, 4),
                          "TOPS": round(tops, 1),
                          "pct_int8_peak": round(100 * tops / INT8_PEAK_TOPS, 2),
                          "pct_mixed_ceiling": round(100 * tops / mixed_peak, 2),
                          "sdpa_ms": round(ms_sdpa, 4), "sdpa_backend_ms": round(ms_sdpa_path, 4), "route": route,
                          "vs_fp32_sdpa": _cmp(out, ref)}),
              flush=True)
        del q, k, v, out, ref
    for name, M, K, N, dt in LIN_SHAPES:
        g.manual_seed(0)
        x = torch.randn(M, K, generator=g, device=dev)
        idx = torch.randperm(K, generator=g, device=dev)[: max(1, round(K * 0.005))]
        x[:, idx] *= 20
        x = x.to(dt)
        lin = torch.nn.Linear(K, N, device=dev)
        with torch.no_grad():
            lin.weight.normal_(0, 0.02, generator=g)
            lin.bias.normal_(0, 0.02, generator=g)
        group = 256 if K % 256 == 0 else 0
        m = Int8Linear.from_linear(lin, group)
        if dt != torch.float32:
            m.bias.data = m.bias.data.to(dt)
        ms_q = per_call_ms(lambda: quantize_activation(x, group))
        qx, sx = quantize_activation(x, group)
        ms_g = per_call_ms(lambda: m.matmul_quantized(qx, sx, dt))
        # GPU time alone (no host launch cost), for the rates and % of HBM
        ms_qg = graph_call_ms(lambda: quantize_activation(x, group))
        ms_gg = graph_call_ms(lambda: m.matmul_quantized(qx, sx, dt))
        y = m.matmul_quantized(qx, sx, dt)
        # the reference's unfused int8 path on the same codes: exact int32 sums
        # (float64 holds them), then rescale's torch ops (_int8.py:322-323)
        acc = (qx.double() @ m.weight.double().T)
        ref = (acc.float() * (sx[:, None] * m.scale[None, :])).to(dt)
        ref = ref + m.bias.to(dt)
        yf = F.linear(x.float(), lin.weight.float(), lin.bias.float())
        ops = 2 * M * N * K
        qbytes = M * K * x.element_size() + M * K + 4 * M
        # the GEMM's algorithmic bytes: int8 operands, scales, bias, output
        gbytes = M * K + N * K + 4 * (M + N) + N * m.bias.element_size() + M * N * x.element_size()
        tops = ops / (ms_gg * 1e-3) / 1e12
        print(json.dumps({"kind": "w8a8_linear", "shape": name, "M": M, "K": K, "N": N, "group": group,
                          "dtype": str(dt)[6:], "plan": __import__("diffucore_amd")._int8.gemm_plan(M, N, K),
                          "gemm_ms": round(ms_g, 4), "gemm_gpu_ms": round(ms_gg, 4), "TOPS": round(tops, 1),
                          "pct_int8_peak": round(100 * tops / INT8_PEAK_TOPS, 2),
                          "gemm_bytes": gbytes, "gemm_GBps": round(gbytes / (ms_gg * 1e-3) / 1e9, 1),
                          "gemm_pct_hbm": round(100 * gbytes / (ms_gg * 1e-3) / 1e9 / HBM_PEAK_GBS, 2),
                          "quant_ms": round(ms_q, 4), "quant_gpu_ms": round(ms_qg, 4),
                          "quant_GBps": round(qbytes / (ms_qg * 1e-3) / 1e9, 1),
                          "quant_pct_hbm": round(100 * qbytes / (ms_qg * 1e-3) / 1e9 / HBM_PEAK_GBS, 2),
                          "vs_int_mm_rescale": _cmp(y, ref), "vs_float_linear": _cmp(y, yf)}), flush=True)
        del x, lin, m, qx, sx, y, acc, ref, yf
    # UNet self-attention q/k/v: separate layers, one shared quantization (the
    # reference's Anima pattern), and one GEMM over stacked weights
    from diffucore_amd import fuse_linears, shared_qkv
    for name, M, K in (("sdxl_qkv_4096", 8192, 640), ("sdxl_qkv_1024", 2048, 1280)):
        g.manual_seed(0)
        x = torch.randn(M, K, generator=g, device=dev).to(torch.float16)
        projs = []
        for _ in range(3):
            lin = torch.nn.Linear(K, K, bias=False, device=dev)
            with torch.no_grad():
                lin.weight.normal_(0, 0.02, generator=g)
            projs.append(Int8Linear.from_linear(lin, 256 if K % 256 == 0 else 0))
        fused = fuse_linears(projs)
        ms_sep = per_call_ms(lambda: [p(x) for p in projs])
        ms_shared = per_call_ms(lambda: shared_qkv(x, projs))
        ms_fused = per_call_ms(lambda: fused(x).split(K, -1))
        exact = all(torch.equal(a, b) for a, b in zip(fused(x).split(K, -1), shared_qkv(x, projs)))
        print(json.dumps({"kind": "qkv_projection", "shape": name, "M": M, "K": K, "N": 3 * K, "dtype": "float16",
                          "separate_ms": round(ms_sep, 4), "shared_quant_ms": round(ms_shared, 4),
                          "fused_gemm_ms": round(ms_fused, 4), "fused_equals_shared": exact}), flush=True)
        del x, projs, fused
    # fused MLP middle (dc_act_quantize_rows) against the ops it replaces, at FLUX shapes
    from diffucore_amd import act_quantize
    for name, M, K1, K2 in (("flux_img_mlp_middle", 4096, 0, 12288), ("flux_single_linear2_input", 4608, 3072, 12288)):
        g.manual_seed(0)
        h = (torch.randn(M, K2, generator=g, device=dev) * 2).to(torch.bfloat16)
        pre = torch.randn(M, K1, generator=g, device=dev).to(torch.bfloat16) if K1 else None

        def unfused():
            a = F.gelu(h, approximate="tanh")
            return quantize_activation(torch.cat((pre, a), 1) if K1 else a, 256)

        ms_u = per_call_ms(unfused)
        ms_f = per_call_ms(lambda: act_quantize(h, 256, "gelu_tanh", prefix=pre))
        nbytes = M * (K1 + K2) * 2 + M * (K1 + K2) + 4 * M   # read the 16-bit rows once, write codes + scales
        print(json.dumps({"kind": "fused_mlp_middle", "shape": name, "M": M, "K1": K1, "K2": K2, "dtype": "bfloat16",
                          "act": "gelu_tanh", "unfused_ms": round(ms_u, 4), "fused_ms": round(ms_f, 4),
                          "speedup": round(ms_u / ms_f, 2), "fused_GBps": round(nbytes / (ms_f * 1e-3) / 1e9, 1)}),
              flush=True)
        del h, pre
    # GEGLU middle (DC_ACT_GEGLU) against the unfused ops, at SDXL's feed-forward shapes
    for name, M, N in (("sdxl_geglu_middle_4096", 8192, 5120), ("sdxl_geglu_middle_1024", 2048, 10240)):
        g.manual_seed(0)
        h = (torch.randn(M, 2 * N, generator=g, device=dev) * 2).to(torch.float16)

        def unfused_geglu():
            a, gate = h.chunk(2, dim=-1)
            return quantize_activation(a * F.gelu(gate), 256)

        ms_u = per_call_ms(unfused_geglu)
        ms_f = per_call_ms(lambda: act_quantize(h, 256, "geglu"))
        nbytes = M * 2 * N * 2 + M * N + 4 * M
        print(json.dumps({"kind": "fused_geglu_middle", "shape": name, "M": M, "N": N, "dtype": "float16",
                          "unfused_ms": round(ms_u, 4), "fused_ms": round(ms_f, 4),
                          "speedup": round(ms_u / ms_f, 2), "fused_GBps": round(nbytes / (ms_f * 1e-3) / 1e9, 1)}),
              flush=True)
        del h
    # the UNet transformer block (unet_block.py) at SD1.5 / SDXL shapes: fp16 eager against W8A8 + INT8
    import copy
    import unet_block as UB
    for lv in UB.LEVELS:
        blk = UB.build(lv, dev)
        x, ctx = UB.inputs(lv, dev)
        with torch.no_grad():
            ms_e = per_call_ms(lambda: blk(x, ctx))
            ref = blk(x, ctx) - x
            qb = UB.to_int8(copy.deepcopy(blk), dev)
            ms_q = per_call_ms(lambda: qb(x, ctx))
            out = qb(x, ctx) - x
            # device time without the modules' Python and launch cost: the block captured in a HIP graph
            # (None if a module's ops cannot be captured)
            try:
                gms_e = graph_call_ms(lambda: blk(x, ctx), reps=5)
                gms_q = graph_call_ms(lambda: qb(x, ctx), reps=5)
            except RuntimeError as e:
                print(f"[bench] unet block {lv.name}: graph capture failed: {e}", file=sys.stderr, flush=True)
                gms_e = gms_q = None
        print(json.dumps({"kind": "unet_block", "shape": lv.name, "B": lv.batch, "tokens": lv.tokens, "dim": lv.dim,
                          "heads": lv.heads, "ctx": [lv.ctx_len, lv.ctx_dim], "dtype": "float16",
                          "fp16_eager_ms": round(ms_e, 4), "int8_ms": round(ms_q, 4),
                          "speedup": round(ms_e / ms_q, 2),
                          "fp16_graph_ms": round(gms_e, 4) if gms_e else None,
                          "int8_graph_ms": round(gms_q, 4) if gms_q else None,
                          "graph_speedup": round(gms_e / gms_q, 2) if gms_e and gms_q else None,
                          "update_vs_fp16": _cmp(out, ref)}), flush=True)
        del blk, qb, x, ctx, ref, out
    # QK RMSNorm + rotary (dc_qk_norm_rope) against FLUX's eager ops, at the FLUX double-block shape:
    # txt (512) and img (4096) q/k/v views of the two qkv projections -> joint (B, H, L, D) q, k, v
    import flux_step as FS
    from diffucore_amd import flux_qk_norm_rope
    H, D, Lt, Li = 24, 128, 512, 4096
    g.manual_seed(0)
    tqkv = torch.randn(1, Lt, 3 * H * D, generator=g, device=dev).to(torch.bfloat16)
    iqkv = torch.randn(1, Li, 3 * H * D, generator=g, device=dev).to(torch.bfloat16)
    sc = [torch.rand(D, generator=g, device=dev).add(0.5).to(torch.bfloat16) for _ in range(4)]
    pe = FS.position_embedding(FS.FluxShape(), dev)
    qn = [FS.RMSNorm(D).to(dev, torch.bfloat16) for _ in range(4)]
    for n, s_ in zip(qn, sc):
        n.scale.data.copy_(s_)

    def eager():
        iq, ik, iv = FS._split_heads(iqkv, H)
        tq, tk, tv = FS._split_heads(tqkv, H)
        iq, ik = qn[0](iq).to(iv), qn[1](ik).to(iv)
        tq, tk = qn[2](tq).to(tv), qn[3](tk).to(tv)
        q, k = FS.apply_rope(torch.cat((tq, iq), 2), torch.cat((tk, ik), 2), pe)
        return q, k, torch.cat((tv, iv), 2)

    bufs = [torch.empty(1, Lt + Li, H, D, device=dev, dtype=torch.bfloat16) for _ in range(3)]

    def fused():
        for x, a, b, sl in ((tqkv, qn[2], qn[3], slice(0, Lt)), (iqkv, qn[0], qn[1], slice(Lt, Lt + Li))):
            x5 = x.unflatten(-1, (3, H, D))
            flux_qk_norm_rope(x5[:, :, 0], x5[:, :, 1], a.scale, b.scale, pe[:, :, sl], v=x5[:, :, 2],
                              out=tuple(t[:, sl] for t in bufs))
        return bufs

    ms_e, ms_f = per_call_ms(eager), per_call_ms(fused)
    eq = eager()
    fused()
    same = [float((a.transpose(1, 2) == b).float().mean()) for a, b in zip(eq, bufs)]
    nbytes = 3 * 2 * (Lt + Li) * H * D * 2    # q, k, v: 16-bit rows read once and written once
    print(json.dumps({"kind": "qk_norm_rope", "shape": "flux_double_block", "L": Lt + Li, "H": H, "D": D,
                      "dtype": "bfloat16", "eager_ms": round(ms_e, 4), "fused_ms": round(ms_f, 4),
                      "speedup": round(ms_e / ms_f, 2), "fused_GBps": round(nbytes / (ms_f * 1e-3) / 1e9, 1),
                      "bit_equal_fraction_q_k_v": [round(x, 5) for x in same]}), flush=True)


# ---------------------------------------------------------------- main

def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-full", action="store_true", help="skip the full FLUX step vs bf16 comparison")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--compiled-bf16", action="store_true",
                    help="also time the bf16 step under torch.compile (inductor; compile time excluded)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a 1 GiB device copy (scales the rocprofv3 byte counters) and exit")
    ap.add_argument("--shapes", action="store_true",
                    help="only print the per-shape report (every benchmark config shape) and exit")
    ap.add_argument("--gemm-ab", action="store_true",
                    help="only print the same-process GEMM A/B against torch._int_mm (hipBLASLt) at FLUX's "
                         "linear shapes and exit")
    ap.add_argument("--attn-calls", action="store_true",
                    help="only make 5 INT8 attention calls at each benchmark config self-attention shape and exit "
                         "(a driver for rocprofv3 counter runs)")
    ap.add_argument("--unet-compiled", action="store_true",
                    help="only time the UNet transformer block fp16 eager, fp16 under torch.compile and W8A8 + "
                         "INT8 at SD1.5 / SDXL shapes and exit")
    ap.add_argument("--mfma-ceiling", action="store_true",
                    help="only measure the MFMA-only throughput of the device (int8 and bf16, 1 and 2 waves per "
                         "SIMD, constant and changing operands) and exit")
    ap.add_argument("--cpu-configs", action="store_true",
                    help="only time the reference's CPU path at every benchmark config shape (bounded row / query "
                         "samples scaled to a full call, all host threads) and exit (no GPU)")
    ap.add_argument("--traffic-from", metavar="DIR",
                    help="only summarize rocprofv3 FETCH_SIZE / WRITE_SIZE runs under DIR (copy_* and step_*) "
                         "into profiles/gemm_flux_step_traffic.json and exit (no GPU)")
    args = ap.parse_args()
    if args.traffic_from:
        traffic_summary(Path(args.traffic_from))
        return
    if args.cpu_configs:
        cpu_configs()
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (each box has one MI355X); "
              "run it with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    if args.copy_calibration:
        copy_calibration()
        return
    if args.mfma_ceiling:
        torch.cuda.set_device(0)
        print(json.dumps({"mfma_ceiling": mfma_ceiling()}), flush=True)
        return
    if args.attn_calls:
        from diffucore_amd import _lib
        _lib.require()
        torch.cuda.set_device(0)
        with torch.no_grad():
            attn_calls(torch.device("cuda", 0))
        return
    if args.unet_compiled:
        from diffucore_amd import _lib
        _lib.require()
        torch.cuda.set_device(0)
        unet_compiled(torch.device("cuda", 0))
        return
    if args.shapes or args.gemm_ab:
        from diffucore_amd import _lib
        _lib.require()
        torch.cuda.set_device(0)
        with torch.no_grad():
            if args.shapes:
                shapes_report(torch.device("cuda", 0))
            gemm_vendor_ab(torch.device("cuda", 0))
        return

    import flux_step as FS
    from diffucore_amd import _lib, quantize_linears, set_attention_backend, set_fused_glue

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    _lib.require()
    shape = FS.FluxShape()
    log("building the synthetic FLUX.1-schnell model (bf16, random N(0,0.02))")
    model = FS.build(shape, dev, torch.bfloat16, seed=0)
    extra = {}
    x0, txt, y, pe = FS.inputs(shape, dev)
    sigmas = FS.schnell_sigmas(4, dev)
    if not args.no_full:
        log("full step, bf16 SDPA + bf16 linears")
        with torch.no_grad():
            bf16_ms = time_steps(lambda: model(x0, txt, sigmas[:1].to(x0.dtype), y, pe), 3, 1)
            lat_bf16 = FS.denoise(model, x0, txt, y, pe, sigmas)
        log("full step, bf16 SDPA + bf16 linears + fused QK norm/rotary glue")
        set_fused_glue(model, True)
        with torch.no_grad():
            bf16_glue_ms = time_steps(lambda: model(x0, txt, sigmas[:1].to(x0.dtype), y, pe), 3, 1)
        set_fused_glue(model, False)
        if args.compiled_bf16:
            # the strongest bf16 baseline this image builds: the same eager ops
            # fused by inductor's generated kernels
            log("full step, bf16 under torch.compile: compiling")
            compiled = torch.compile(model)
            with torch.no_grad():
                t0 = time.perf_counter()
                compiled(x0, txt, sigmas[:1].to(x0.dtype), y, pe)
                torch.cuda.synchronize()
                log(f"full step, bf16 under torch.compile: compiled in {time.perf_counter() - t0:.0f} s; timing")
                bf16_compiled_ms = time_steps(lambda: compiled(x0, txt, sigmas[:1].to(x0.dtype), y, pe), 3, 1)
            del compiled
            torch._dynamo.reset()
    log("quantizing block linears to W8A8 (ConvRot group 256), stamping int8_turing")
    names = FS.block_linear_names(model)
    quantize_linears(model, names, dev, 256)
    set_attention_backend(model, "int8_turing")
    set_fused_glue(model, True)
    torch.cuda.empty_cache()
    if not args.no_full:
        log("full step, INT8 attention + W8A8 linears")
        with torch.no_grad():
            int8_ms = time_steps(lambda: model(x0, txt, sigmas[:1].to(x0.dtype), y, pe), 3, 1)
            lat_int8 = FS.denoise(model, x0, txt, y, pe, sigmas)
        a, b = lat_int8.float().flatten(), lat_bf16.float().flatten()
        extra["denoise_step"] = {
            "int8_ms": round(int8_ms, 3), "bf16_ms": round(bf16_ms, 3), "speedup": round(bf16_ms / int8_ms, 3),
            "bf16_fused_glue_ms": round(bf16_glue_ms, 3),
            **({"bf16_compiled_ms": round(bf16_compiled_ms, 3), "speedup_vs_compiled": round(bf16_compiled_ms / int8_ms, 3)}
               if args.compiled_bf16 else {}),
            "latent_rel_l2_vs_bf16": round(float((a - b).norm() / b.norm()), 5),
            "latent_cos_vs_bf16": round(float(a @ b / (a.norm() * b.norm())), 6),
            "what": "full synthetic FLUX.1-schnell forward + euler update at 1024^2 (flux_step.py), "
                    "4-step final latent compared; int8 = W8A8 linears + INT8 attention + fused glue "
                    "(LayerNorm-modulate/GELU quantize passes, QK norm + rotary, gate + residual in the GEMM "
                    "epilogue); bf16 = the reference's "
                    "eager ops, bf16_fused_glue = bf16 with only the QK norm + rotary pass fused"
                    + (", bf16_compiled = the eager bf16 model under torch.compile (inductor)" if args.compiled_bf16
                       else ""),
        }
        log(f"full step: int8 {int8_ms:.2f} ms vs bf16 {bf16_ms:.2f} ms")

    hp = HotPath(model, shape, dev)
    log(f"hot path: {len(hp.ops)} calls, {hp.total_ops / 1e12:.2f} TOP per step; timing {args.steps} steps")
    recs = []
    with torch.no_grad():
        for _ in range(args.warmup):
            hp.run()
        # per-kernel attribution: HIP events around every call, its own pass
        torch.cuda.synchronize()
        for _ in range(args.steps):
            hp.run(recs)
        torch.cuda.synchronize()
        # the timed steps: the calls issued one by one, with no events between
        ms = time_steps(hp.run, args.steps, 1)
    attr = summarize(recs)
    tops = hp.total_ops / (ms * 1e-3) / 1e12
    log(f"hot path: {ms:.3f} ms/step, {tops:.1f} TOPS ({100 * tops / INT8_PEAK_TOPS:.1f}% of int8 peak)")

    kernels = {}
    for kind, d in attr.items():
        per = {"ms_per_step": round(d["ms"] / args.steps, 3), "launches_per_step": d["launches"] // args.steps,
               "avg_launch_us": round(1e3 * d["ms"] / d["launches"], 2)}
        if d["ops"]:
            per["TOPS"] = round(d["ops"] / (d["ms"] * 1e-3) / 1e12, 1)
        if d["bytes"]:
            per["GBps"] = round(d["bytes"] / (d["ms"] * 1e-3) / 1e9, 1)
        kernels[kind] = per
    g = attr["gemm_dma_256x256"]
    ops_per_launch = g["ops"] / g["launches"]
    bytes_per_launch = g["bytes"] / g["launches"]
    launch_s = g["ms"] / g["launches"] * 1e-3
    achieved = ops_per_launch / launch_s / 1e12
    # HBM bytes per launch from the committed counter summary, used only when it
    # was measured on the GEMM source this run executes
    traffic, traffic_src = None, {"profile": "profiles/gemm_flux_step_traffic.json"}
    tfile = ROOT / "profiles" / "gemm_flux_step_traffic.json"
    if tfile.exists():
        tj = json.loads(tfile.read_text())
        traffic_src["kernel_source_sha256"] = tj.get("kernel_source_sha256")
        traffic_src["matches_current_source"] = tj.get("kernel_source_sha256") == gemm_source_sha256()
        if traffic_src["matches_current_source"]:
            traffic = tj.get("hbm_bytes_per_launch")
    roofline = {"kernel": "w8a8_gemm_dma_kernel (256x256 tiles, 4 waves, operands loaded straight into LDS): the "
                          f"{g['launches'] // args.steps} FLUX-step launches it runs (img MLP up; the double blocks' "
                          "img + txt qkv, proj and MLP down, each pair as one grouped launch; single linear1 and "
                          "linear2)",
                "bound": "mfma", "achieved": round(achieved, 1), "peak": INT8_PEAK_TOPS, "unit": "TOP/s",
                "frac": round(achieved / INT8_PEAK_TOPS, 4), "traffic": traffic, "traffic_source": traffic_src,
                "algorithmic_ops_per_launch": int(ops_per_launch),
                "algorithmic_bytes_per_launch": int(bytes_per_launch),
                "avg_launch_us": round(1e6 * launch_s, 2),
                "launches_timed": g["launches"]}
    # the MFMA-only rate this device sustains (same process, after the steps)
    ceiling = mfma_ceiling()
    best = max(ceiling["int8_32x32x32_vary_1w"], ceiling["int8_32x32x32_vary_2w"])
    roofline["measured_mfma_ceiling"] = best
    roofline["frac_of_measured_ceiling"] = round(achieved / best, 4)

    result = {
        "metric": METRIC, "value": round(tops, 2), "unit": "TOPS", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 3), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int8", "data": "synthetic",
        "config": {"workload": "FLUX.1-schnell-shaped hot path at 1024^2: 19 double + 38 single blocks, "
                               "4096 img + 512 txt tokens, H24 D128, W8A8 linears (ConvRot 256, bf16 out, bias) "
                               "+ INT8 attention (bf16 in/out), one denoise step",
                   "global_batch": 1, "seq_len": 4608, "parallelism": "none (1 GPU)",
                   "algorithmic_TOP_per_step": round(hp.total_ops / 1e12, 3)},
        "pct_int8_peak": round(100 * tops / INT8_PEAK_TOPS, 2),
        "kernels": kernels,
        "roofline": roofline,
        "mfma_ceiling": ceiling,
    }
    result.update(extra)
    if not args.no_cpu:
        log("CPU baseline (reference CPU path, bounded sample)")
        result["cpu_baseline"] = cpu_baseline(shape)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
