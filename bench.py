"""Benchmark of the quantized decode path on one MI355X.

One step = the four INT4 W4A16 decode GEMMs of the headline configuration (Qwen3-4B
down_proj: N=2560, K=9728, group 128, symmetric codes, bf16 activations) at
M = 1, 8, 32, 64 rows. `value` = algorithmic bytes of the step / its time, inputs
resident in HBM. Every launch reads its own copy of the weights (copies rotate over
more than 512 MiB), so the 256 MiB MALL cannot serve the weights from cache.

The timed region is one replay of a HIP graph holding exactly --steps steps, bracketed by
torch.cuda.synchronize() and HIP events on the stream the kernels run on; the average
kernel duration is that time / (4 * steps) (the launches run back to back in the graph).

`roofline.traffic` (HBM bytes per headline launch) comes from two rocprofv3 counter passes
(FETCH_SIZE, then WRITE_SIZE) over a short child run of the same four launches, made before
this process touches the GPU; each counter is scaled by its reading for a reference kernel
of known size in the same child run (a 256 MiB sum for FETCH_SIZE, a 256 MiB fill for
WRITE_SIZE). Without rocprofv3 it is null.

`breakdown` reports the other configurations the same way (INT8 gate_up GEMM, FP8 prefill
GEMM, paged decode attention on FP8 / INT8 KV at the 256-token default and the configuration's
512-token partition with two KV copies alternating, INT4 MoE layer), each with a CPU number:
`cpu_baseline` times the reference formulas restated on the CPU (oracle/) on a bounded
sample of the same configuration.

Usage: python bench.py [--gpus 1] [--steps 50] [--warmup 10] [--no-cpu] [--no-traffic]
                       [--only headline]
"""
import argparse
import csv
import glob
import json
import math
import os
import shutil
import subprocess
import sys
import tempfile
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "mini-inference_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import torch  # noqa: E402

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E, published
FP8_PEAK_TFLOPS = 5000.0     # MI355X dense FP8 MFMA, published
BF16_PEAK_TFLOPS = 2500.0    # MI355X dense bf16 MFMA, published
ROTATE_BYTES = 600 * 2 ** 20  # > 2 x MALL
METRIC = "quantized decode GEMM GB/s (% HBM peak) at M=1..64; FP8-KV attn µs/step"
MS = (1, 8, 32, 64)
PROBE_BYTES = 256 * 2 ** 20   # size of the counter-calibration sum / fill


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def gen(seed):
    return torch.Generator().manual_seed(seed)


def copies_for(nbytes, minimum):
    return max(minimum, math.ceil(ROTATE_BYTES / nbytes))


def time_graph(fn_list, reps=1):
    """Capture the callables in one graph, replay `reps` times; return seconds per replay."""
    stream = torch.cuda.current_stream()
    for f in fn_list[: min(len(fn_list), 8)]:
        f()  # eager warm-up: workspaces and kernel attributes exist before capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for f in fn_list:
            f()
    g.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record(stream)
    for _ in range(reps):
        g.replay()
    end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) / 1e3 / reps


_FLOOR_CACHE = {}


def stream_floor_us(nbytes, dev):
    """Time of a plain streaming read of `nbytes` (miq_stream_read: 16-byte non-temporal
    loads over 2048 workgroups), the same graph timing as the kernels, each read from a
    window of a buffer of at least 640 MiB that the previous reads did not touch (MALL
    defeated). The floor a launch of that many bytes can reach on this GPU."""
    from kernels import _lib
    nbytes = int(nbytes) // 16 * 16
    if nbytes in _FLOOR_CACHE:
        return _FLOOR_CACHE[nbytes]
    total = max(640 << 20, 3 * nbytes)
    buf = torch.empty(total, dtype=torch.uint8, device=dev)
    sink = torch.zeros(4, dtype=torch.int32, device=dev)
    lib = _lib.load()
    nwin = max(2, (total - nbytes) // max(nbytes, 1 << 20))
    step = ((total - nbytes) // nwin) // 4096 * 4096
    def rd(i):  # the stream is looked up at call time: under capture it is the capture stream
        off = (i % (nwin + 1)) * step
        return lambda: lib.miq_stream_read(buf.data_ptr() + off, nbytes, sink.data_ptr(),
                                           torch.cuda.current_stream(dev).cuda_stream)
    reps = 20
    t = min(time_graph([rd(i) for i in range(reps)]) / reps for _ in range(2))
    del buf
    _FLOOR_CACHE[nbytes] = round(t * 1e6, 2)
    return _FLOOR_CACHE[nbytes]


def with_floor(entry, nbytes, dev):
    """Adds the streaming-read floor of `nbytes` to a timing entry that has "us"."""
    f = stream_floor_us(nbytes, dev)
    entry["stream_floor_us"] = f
    entry["frac_of_stream_floor"] = round(f / entry["us"], 3)
    return entry


def host_cpu():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown CPU"


# ---------------------------------------------------------------- configurations
def int4_setup(dev, symmetric=True):
    from kernels import quant_ops as ops
    N, K, G = 2560, 9728, 128
    w = (torch.randn(N, K, generator=gen(2)) * 0.02).to(torch.bfloat16).to(dev)
    q, s, z = ops.int4_quantize(w, G, torch.bfloat16, symmetric=symmetric)
    per = q.numel() + s.numel() * 2 + (0 if z is None else z.numel() * 2)
    n = copies_for(per, 4 * len(MS))
    qs = [(q.clone(), s.clone(), None if z is None else z.clone()) for _ in range(n)]
    xs = {M: torch.randn(M, K, generator=gen(3)).to(torch.bfloat16).to(dev) for M in MS}
    return dict(N=N, K=K, G=G, copies=qs, x=xs, wbytes=per)


def int4_bytes(cfg, M):
    return cfg["wbytes"] + M * cfg["K"] * 2 + M * cfg["N"] * 2


def int4_launch(cfg, M, i):
    from kernels import quant_ops as ops
    q, s, z = cfg["copies"][i % len(cfg["copies"])]
    x = cfg["x"][M]
    return lambda: ops.w4a16_linear(x, q, s, z)


def int8_setup(dev):
    from kernels import quant_ops as ops
    N, K = 19456, 2560
    w = (torch.randn(N, K, generator=gen(1)) * 0.02).to(torch.bfloat16).to(dev)
    q, s = ops.int8_quantize(w, torch.float32)
    s = s.reshape(N)
    per = q.numel() + s.numel() * 4
    n = copies_for(per, 4)
    return dict(N=N, K=K, copies=[(q.clone(), s.clone()) for _ in range(n)], wbytes=per,
                x={M: torch.randn(M, K, generator=gen(4)).to(torch.bfloat16).to(dev) for M in MS})


def bench_headline(dev, steps, warmup):
    cfg = int4_setup(dev)
    step_bytes = sum(int4_bytes(cfg, M) for M in MS)
    launches = []
    for i in range(steps):
        for j, M in enumerate(MS):
            launches.append(int4_launch(cfg, M, 4 * i + j))
    if warmup:
        time_graph([int4_launch(cfg, M, 4 * i + j) for i in range(warmup) for j, M in enumerate(MS)])
    t = time_graph(launches)
    return cfg, step_bytes, t


def per_m(cfg, launch, nbytes, dev, reps_per_graph=40, ref_launch=None):
    """Graph timing per M; with ref_launch, the reference's own formula on the device
    (dequantize, then the library GEMM) timed the same way beside it."""
    out = {}
    for M in MS:
        t = time_graph([launch(cfg, M, i) for i in range(reps_per_graph)]) / reps_per_graph
        gbs = nbytes(cfg, M) / t / 1e9
        out[f"M={M}"] = with_floor({"us": round(t * 1e6, 2), "GB/s": round(gbs, 1),
                                    "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 1)}, nbytes(cfg, M), dev)
        if ref_launch is not None:
            n = 8
            tr = time_graph([ref_launch(cfg, M, i) for i in range(n)]) / n
            out[f"M={M}"]["reference_formula_on_device_us"] = round(tr * 1e6, 2)
    return out


def int4_ref_launch(cfg, M, i):
    """int4_wo.py:33-42 + base.py:20-24 on the device: dequantize (the HIP kernel, the
    reference's two bf16 roundings), then F.linear (hipBLASLt)."""
    from kernels import quant_ops as ops
    q, s, z = cfg["copies"][i % len(cfg["copies"])]
    x = cfg["x"][M]
    return lambda: torch.nn.functional.linear(x, ops.int4_dequantize(q, s, z).to(x.dtype))


def int8_ref_launch(cfg, M, i):
    """int8_wo.py:17-21 on the device: F.linear(x, q.to(bf16)) * s (hipBLASLt)."""
    q, s = cfg["copies"][i % len(cfg["copies"])]
    x = cfg["x"][M]
    return lambda: torch.nn.functional.linear(x, q.to(x.dtype)) * s.to(x.dtype)


def bench_int8(dev):
    from kernels import quant_ops as ops
    cfg = int8_setup(dev)

    def launch(c, M, i):
        q, s = c["copies"][i % len(c["copies"])]
        x = c["x"][M]
        return lambda: ops.w8a16_linear(x, q, s)

    nbytes = lambda c, M: c["wbytes"] + M * c["K"] * 2 + M * c["N"] * 2  # noqa: E731
    res = per_m(cfg, launch, nbytes, dev, reps_per_graph=24, ref_launch=int8_ref_launch)
    del cfg
    return res


def bench_int4_asym(dev):
    cfg = int4_setup(dev, symmetric=False)
    res = per_m(cfg, int4_launch, int4_bytes, dev)
    del cfg
    return res


def bench_wo_prefill(dev):
    """Weight-only GEMMs on prefill-sized M (libmiq's planner picks the wide kernel where its
    128 x 128 MT tiles fill the GPU, the prefill kernel below that), against the
    library route the reference itself takes for every M (dequantize to bf16, then
    F.linear on hipBLASLt: int4_wo.py:33-42 + base.py:20-24, int8_wo.py:17-21)."""
    import torch.nn.functional as F
    from kernels import quant_ops as ops
    out = {}
    reps = 10
    for name, N, K in (("int4_down_proj_2560x9728", 2560, 9728), ("int8_gate_up_19456x2560", 19456, 2560)):
        w = (torch.randn(N, K, generator=gen(11)) * 0.02).to(torch.bfloat16).to(dev)
        if name.startswith("int4"):
            q, s, z = ops.int4_quantize(w, 128, torch.bfloat16, symmetric=True)
            fused = lambda x: ops.w4a16_linear(x, q, s, z)  # noqa: E731
            lib = lambda x: F.linear(x, ops.int4_dequantize(q, s, z))  # noqa: E731
        else:
            q, s = ops.int8_quantize(w, torch.float32)
            fused = lambda x: ops.w8a16_linear(x, q, s)  # noqa: E731
            lib = lambda x: F.linear(x, q.to(torch.bfloat16)) * s.reshape(-1).to(torch.bfloat16)  # noqa: E731
        del w
        rows = {}
        for M in (256, 1024, 2048):
            x = torch.randn(M, K, generator=gen(12)).to(torch.bfloat16).to(dev)
            t = min(time_graph([lambda: fused(x)] * reps) / reps for _ in range(2))
            t_lib = min(time_graph([lambda: lib(x)] * reps) / reps for _ in range(2))
            tf = 2.0 * M * N * K / t / 1e12
            rows[str(M)] = {"us": round(t * 1e6, 1), "TFLOP/s": round(tf, 1),
                            "pct_bf16_peak": round(100 * tf / BF16_PEAK_TFLOPS, 1),
                            "dequant_plus_hipblaslt_us": round(t_lib * 1e6, 1)}
        out[name] = rows
        del q, s
        torch.cuda.empty_cache()
    return out


def bench_fp8(dev):
    from kernels import quant_ops as ops
    M, N, K = 2048, 6144, 2560
    w = (torch.randn(N, K, generator=gen(5)) * 0.02).to(torch.bfloat16).to(dev)
    wq, ws = ops.fp8_quantize_rows(w)
    x = torch.randn(M, K, generator=gen(6)).to(torch.bfloat16).to(dev)
    xq, xs = ops.fp8_quantize_rows(x)
    flops = 2.0 * M * N * K
    reps = 20
    t_gemm = time_graph([lambda: ops.fp8_gemm(xq, xs, wq, ws)] * reps) / reps
    t_quant = time_graph([lambda: ops.fp8_quantize_rows(x)] * reps) / reps
    tf = flops / t_gemm / 1e12
    tf_all = flops / (t_gemm + t_quant) / 1e12
    # the library GEMM the reference calls (fp8.py:55-61: torch._scaled_mm with row-wise
    # scales), on the same operands, in the same graph timing
    sa, sb = xs.reshape(-1, 1), ws.reshape(1, -1)
    t_lib = time_graph([lambda: torch._scaled_mm(xq, wq.t(), scale_a=sa, scale_b=sb, out_dtype=torch.bfloat16)]
                       * reps) / reps
    return {"gemm_us": round(t_gemm * 1e6, 2), "gemm_TFLOP/s": round(tf, 1),
            "pct_fp8_peak": round(100 * tf / FP8_PEAK_TFLOPS, 1),
            "act_quant_us": round(t_quant * 1e6, 2),
            "quant+gemm_TFLOP/s": round(tf_all, 1), "peak_used_TFLOP/s": FP8_PEAK_TFLOPS,
            "hipblaslt_rowwise_scaled_mm_us": round(t_lib * 1e6, 2)}


def attention_tables(B=64, page=16, seed=7):
    """Context lengths U[512, 8192] and a shuffled block table over all pages (seeded)."""
    g = gen(seed)
    lens = torch.randint(512, 8193, (B,), generator=g)
    pages = [-(-int(n) // page) for n in lens]
    total = sum(pages)
    perm = torch.randperm(total, generator=g)
    table = torch.zeros(B, max(pages), dtype=torch.int32)
    i = 0
    for b, n in enumerate(pages):
        table[b, :n] = perm[i:i + n].to(torch.int32)
        i += n
    return g, lens, pages, table


def attention_inputs(dev, kind, B=64, H=32, KV=8, D=128, page=16, seed=7, copies=2):
    """Config 4: `copies` independent KV caches (> 2 x the MALL together) so consecutive
    calls never read a cache the previous call left in the MALL."""
    g, lens, pages, table = attention_tables(B, page, seed)
    slots = sum(pages) * page
    caches = []
    for c in range(copies):
        # K/V ~ N(0,1) generated on the device from a seeded generator (570 MB of codes)
        dg = torch.Generator(device=dev).manual_seed(seed + 100 * c)
        k = torch.randn(slots, KV, D, generator=dg, device=dev)
        v = torch.randn(slots, KV, D, generator=dg, device=dev)
        if kind == "fp8":
            s = torch.tensor(4.0 / 448.0, device=dev)
            kc = (k / s).clamp(-448, 448).to(torch.float8_e4m3fn)
            vc = (v / s).clamp(-448, 448).to(torch.float8_e4m3fn)
            ks = s.reshape(1, 1).expand(slots, KV)
            vs = ks
        else:
            from engine.core.kv_cache import kv_quant_write
            kc = torch.empty(slots, KV, D, dtype=torch.int8, device=dev)
            vc = torch.empty_like(kc)
            ks = torch.empty(slots, KV, dtype=torch.float32, device=dev)
            vs = torch.empty_like(ks)
            idx = torch.arange(slots, device=dev)
            kv_quant_write(kc, ks, idx, k)
            kv_quant_write(vc, vs, idx, v)
        del k, v
        caches.append((kc, vc, ks, vs))
    scale_bytes = 0 if kind == "fp8" else int(lens.sum()) * KV * 2 * 4
    q = torch.randn(B, H, D, generator=g).to(torch.bfloat16).to(dev)
    ntok = int(lens.sum())
    nbytes = ntok * KV * D * 2 + scale_bytes + sum(pages) * 4 + B * H * D * 2 * 2 + B * 4
    return dict(q=q, caches=caches, table=table.to(dev), lens=lens.to(torch.int32).to(dev),
                max_len=int(lens.max()), page=page, bytes=nbytes, tokens=ntok)


def bench_attention(dev, kind):
    from kernels.paged_attention import paged_decode_attention
    a = attention_inputs(dev, kind)

    def call(i, partition):
        kc, vc, ks, vs = a["caches"][i % len(a["caches"])]
        return lambda: paged_decode_attention(a["q"], kc, vc, a["table"], a["lens"], a["page"], 128 ** -0.5,
                                              a["max_len"], k_scale=ks, v_scale=vs, partition=partition)
    reps = 20
    res = {"context_tokens": a["tokens"], "MB_per_call": round(a["bytes"] / 1e6, 1), "kv_copies": len(a["caches"])}
    for partition in (256, 512):
        t = time_graph([call(i, partition) for i in range(reps)]) / reps
        gbs = a["bytes"] / t / 1e9
        e = {"us_per_step": round(t * 1e6, 2), "GB/s": round(gbs, 1),
             "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 1)}
        e["stream_floor_us"] = stream_floor_us(a["bytes"], dev)
        e["frac_of_stream_floor"] = round(e["stream_floor_us"] / e["us_per_step"], 3)
        res[f"partition_{partition}"] = e
    from kernels.paged_attention.decode import choose_partition
    kc = a["caches"][0][0]
    res["default_partition"] = choose_partition(a["max_len"], None, kc.dtype)
    del a
    return res


def moe_routing(T=64, H=2048, E=64, k=8, seed=8):
    """bench/micro/bench_moe.py:113-117: softmax over a bf16 router, top-k, no renorm."""
    g = gen(seed)
    hidden = torch.randn(T, H, generator=g).to(torch.bfloat16)
    router = (torch.randn(E, H, generator=g) * 0.02).to(torch.bfloat16)
    probs = torch.softmax(hidden.float() @ router.float().t(), dim=-1)
    w, idx = torch.topk(probs, k, dim=-1)
    return hidden, w.to(torch.bfloat16), idx


def moe_setup(dev, copies=None):
    from kernels import quant_ops as ops
    T, H, inter, E, k = 64, 2048, 1024, 64, 8
    hidden, w, idx = moe_routing(T, H, E, k)
    hidden, w, idx = hidden.to(dev), w.to(dev), idx.to(dev)
    dg = torch.Generator(device=dev).manual_seed(9)
    wgu = (torch.randn(E, 2 * inter, H, generator=dg, device=dev) * 0.02).to(torch.bfloat16)
    wdn = (torch.randn(E, H, inter, generator=dg, device=dev) * 0.02).to(torch.bfloat16)
    gu = ops.int4_quantize(wgu, 128, torch.bfloat16, symmetric=True)
    dn = ops.int4_quantize(wdn, 128, torch.bfloat16, symmetric=True)
    del wgu, wdn
    touched = int(idx.unique().numel())
    per_expert = (2 * inter * H // 2 + H * inter // 2) + (2 * inter * H // 128 + H * inter // 128) * 2
    nbytes = touched * per_expert + T * H * 2 * 2 + T * k * 6
    total = E * per_expert
    n = copies or copies_for(total, 2)
    sets = [(tuple(t.clone() for t in gu[:2]), tuple(t.clone() for t in dn[:2])) for _ in range(n)]
    return dict(hidden=hidden, w=w, idx=idx, sets=sets, bytes=nbytes, touched=touched, T=T, H=H, I=inter, E=E, k=k)


def bench_moe(dev):
    from kernels.fused_moe import fused_moe_int4
    c = moe_setup(dev)

    def launch(i):
        (gq, gs), (dq, ds) = c["sets"][i % len(c["sets"])]
        return lambda: fused_moe_int4(c["hidden"], c["idx"], c["w"], gq, gs, None, dq, ds, None)
    reps = 12
    t = time_graph([launch(i) for i in range(reps)]) / reps
    gbs = c["bytes"] / t / 1e9
    from engine.quantization.int4_wo import Int4WeightOnly
    (gq, gs), (dq, ds) = c["sets"][0]
    tg = grouped_path_time(Int4WeightOnly(group_size=128), c["E"], {"qweight": gq, "scale": gs},
                           {"qweight": dq, "scale": ds}, c["hidden"], c["idx"], c["w"])
    res = {"us_per_layer": round(t * 1e6, 2), "GB/s": round(gbs, 1), "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 1),
           "experts_touched": c["touched"], "MB_per_call": round(c["bytes"] / 1e6, 1),
           "grouped_per_expert_path_us": round(tg * 1e6, 1)}
    res["stream_floor_us"] = stream_floor_us(c["bytes"], dev)
    res["frac_of_stream_floor"] = round(res["stream_floor_us"] / res["us_per_layer"], 3)
    del c
    return res


def bench_moe_int8(dev):
    """Config 5's layer with INT8 experts (per-row scales), the fused INT8 path."""
    from kernels import quant_ops as ops
    from kernels.fused_moe import fused_moe_int8
    T, H, inter, E, k = 64, 2048, 1024, 64, 8
    hidden, w, idx = moe_routing(T, H, E, k)
    hidden, w, idx = hidden.to(dev), w.to(dev), idx.to(dev)
    dg = torch.Generator(device=dev).manual_seed(9)
    wgu = (torch.randn(E, 2 * inter, H, generator=dg, device=dev) * 0.02).to(torch.bfloat16)
    wdn = (torch.randn(E, H, inter, generator=dg, device=dev) * 0.02).to(torch.bfloat16)
    gu = ops.int8_quantize(wgu, torch.bfloat16)
    dn = ops.int8_quantize(wdn, torch.bfloat16)
    del wgu, wdn
    touched = int(idx.unique().numel())
    per_expert = 2 * inter * H + H * inter + (2 * inter + H) * 2
    nbytes = touched * per_expert + T * H * 2 * 2 + T * k * 6
    n = copies_for(E * per_expert, 2)
    sets = [(gu[0].clone(), gu[1].clone(), dn[0].clone(), dn[1].clone()) for _ in range(n)]

    def launch(i):
        gq, gs, dq, ds = sets[i % len(sets)]
        return lambda: fused_moe_int8(hidden, idx, w, gq, gs, dq, ds)
    reps = 8
    t = time_graph([launch(i) for i in range(reps)]) / reps
    gbs = nbytes / t / 1e9
    from engine.quantization.int8_wo import Int8WeightOnly
    gq, gs, dq, ds = sets[0]
    tg = grouped_path_time(Int8WeightOnly(), E, {"qweight": gq, "scale": gs}, {"qweight": dq, "scale": ds},
                           hidden, idx, w)
    floor = stream_floor_us(nbytes, dev)
    return {"us_per_layer": round(t * 1e6, 2), "GB/s": round(gbs, 1), "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 1),
            "experts_touched": touched, "MB_per_call": round(nbytes / 1e6, 1),
            "grouped_per_expert_path_us": round(tg * 1e6, 1), "stream_floor_us": floor,
            "frac_of_stream_floor": round(floor / (t * 1e6), 3)}


def grouped_path_time(method, E, gate_up, down, hidden, idx, w, reps=5):
    """Seconds per call of QuantExperts' grouped path: the reference loop's structure
    (modules.py:55-75: one sort, then method.linear per hit expert) on the device. It syncs
    with the host inside (the expert list), so it is timed eagerly, not in a graph."""
    from engine.quantization.modules import QuantExperts
    qe = QuantExperts.__new__(QuantExperts)
    torch.nn.Module.__init__(qe)
    qe.method, qe.num_experts, qe.act_fn = method, E, torch.nn.SiLU()
    qe._store("gate_up_", gate_up)
    qe._store("down_", down)
    for _ in range(2):
        qe._grouped(hidden, idx, w)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        qe._grouped(hidden, idx, w)
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / reps


def bench_moe_fp8(dev):
    """Config 5's layer with FP8 experts (e4m3fn codes, fp32 per-row scales): the fused FP8
    path, and the grouped per-expert path it replaces (one sort, then FP8WeightAct.linear
    per hit expert) timed eagerly beside it."""
    from kernels import quant_ops as ops
    from kernels.fused_moe import fused_moe_fp8
    T, H, inter, E, k = 64, 2048, 1024, 64, 8
    hidden, w, idx = moe_routing(T, H, E, k)
    hidden, w, idx = hidden.to(dev), w.to(dev), idx.to(dev)
    dg = torch.Generator(device=dev).manual_seed(9)
    wgu = (torch.randn(E, 2 * inter, H, generator=dg, device=dev) * 0.02).to(torch.bfloat16)
    wdn = (torch.randn(E, H, inter, generator=dg, device=dev) * 0.02).to(torch.bfloat16)
    gu = ops.fp8_quantize_rows(wgu)
    dn = ops.fp8_quantize_rows(wdn)
    del wgu, wdn
    touched = int(idx.unique().numel())
    per_expert = 2 * inter * H + H * inter + (2 * inter + H) * 4
    nbytes = touched * per_expert + T * H * 2 * 2 + T * k * 6
    n = copies_for(E * per_expert, 2)
    sets = [(gu[0].clone(), gu[1].clone(), dn[0].clone(), dn[1].clone()) for _ in range(n)]

    def launch(i):
        gq, gs, dq, ds = sets[i % len(sets)]
        return lambda: fused_moe_fp8(hidden, idx, w, gq, gs, dq, ds)
    reps = 8
    t = time_graph([launch(i) for i in range(reps)]) / reps
    gbs = nbytes / t / 1e9
    from engine.quantization.fp8 import FP8WeightAct
    gq, gs, dq, ds = sets[0]
    tg = grouped_path_time(FP8WeightAct(device=dev), E, {"qweight": gq, "scale": gs}, {"qweight": dq, "scale": ds},
                           hidden, idx, w)
    floor = stream_floor_us(nbytes, dev)
    return {"us_per_layer": round(t * 1e6, 2), "GB/s": round(gbs, 1), "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 1),
            "experts_touched": touched, "MB_per_call": round(nbytes / 1e6, 1),
            "grouped_per_expert_path_us": round(tg * 1e6, 1), "stream_floor_us": floor,
            "frac_of_stream_floor": round(floor / (t * 1e6), 3)}


# ---------------------------------------------------------------- CPU baselines (oracle)
# The reference's CPU path restated in oracle/ (plain PyTorch), on the host cores of the
# GPU box, at each configuration's shape; a bounded sample: whole calls until about
# `budget` seconds have passed (at least one), median time. Same units as the GPU lines.
def _cpu_time(fn, budget):
    fn()  # warm-up
    times, t_start = [], time.perf_counter()
    while True:
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
        if time.perf_counter() - t_start > budget or len(times) >= 10:
            break
    times.sort()
    return times[len(times) // 2], len(times)


def _cpu_line(value, unit, n, what):
    return {"value": value, "unit": unit, "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"{n} {what}; median; oracle/ restatement of the reference's CPU path; {host_cpu()}; "
                      f"torch {torch.__version__}"}


def cpu_int4_headline(budget=6.0):
    """Int4WeightOnly.linear = dequantize (int4_wo.py:33-42) + F.linear (base.py:20-24)."""
    from oracle import quant as O
    N, K = 2560, 9728
    w = (torch.randn(N, K, generator=gen(2)) * 0.02).to(torch.bfloat16)
    q = O.int4_quantize_symmetric(w, 128)
    xs = {M: torch.randn(M, K, generator=gen(3)).to(torch.bfloat16) for M in MS}
    wbytes = q["qweight"].numel() + q["scale"].numel() * 2
    step_bytes = sum(wbytes + M * K * 2 + M * N * 2 for M in MS)
    t, n = _cpu_time(lambda: [O.int4_linear(xs[M], **q) for M in MS], budget)
    return _cpu_line(round(step_bytes / t / 1e9, 3), "GB/s", n,
                     f"whole steps (4 INT4 linears, M=1/8/32/64, N=2560 K=9728), {t * 1e3:.1f} ms/step")


def cpu_int8(budget=6.0):
    """Int8WeightOnly.linear (int8_wo.py:17-21) at the gate_up shape, M=1/8/32/64."""
    from oracle import quant as O
    N, K = 19456, 2560
    w = (torch.randn(N, K, generator=gen(1)) * 0.02).to(torch.bfloat16)
    q = O.int8_quantize(w, torch.float32)
    xs = {M: torch.randn(M, K, generator=gen(4)).to(torch.bfloat16) for M in MS}
    step_bytes = sum(N * K + N * 4 + M * K * 2 + M * N * 2 for M in MS)
    t, n = _cpu_time(lambda: [O.int8_linear(xs[M], **q) for M in MS], budget)
    return _cpu_line(round(step_bytes / t / 1e9, 3), "GB/s", n,
                     f"steps of 4 INT8 linears (M=1/8/32/64, N=19456 K=2560), {t * 1e3:.1f} ms/step")


def cpu_fp8(budget=6.0):
    """FP8WeightAct.linear on the CPU: activation quantize + the emulated matmul
    (fp8.py:41-46, 69-73), what the reference runs without native FP8."""
    from oracle import quant as O
    M, N, K = 2048, 6144, 2560
    w = (torch.randn(N, K, generator=gen(5)) * 0.02).to(torch.bfloat16)
    q = O.fp8_quantize(w)
    x = torch.randn(M, K, generator=gen(6)).to(torch.bfloat16)
    t, n = _cpu_time(lambda: O.fp8_linear_emulated(x, **q), budget)
    return _cpu_line(round(2.0 * M * N * K / t / 1e12, 4), "TFLOP/s", n,
                     f"calls at 2048x6144x2560 (activation quant + emulated GEMM), {t * 1e3:.1f} ms/call")


def cpu_attention(kind, budget=6.0, requests=16):
    """The per-request fp32 loop of paged_attention/reference.py:10-28 over the config-4
    cache; sample: the first `requests` requests of the batch."""
    from oracle import attention as A
    from oracle import quant as O
    KV, D, H, page = 8, 128, 32, 16
    g, lens, pages, table = attention_tables(64, page, 7)
    lens, table = lens[:requests], table[:requests]
    slots = (int(table.max()) + 1) * page
    kg = torch.Generator().manual_seed(107)
    k = torch.randn(slots, KV, D, generator=kg)
    v = torch.randn(slots, KV, D, generator=kg)
    if kind == "fp8":
        s = torch.tensor(4.0 / 448.0)
        kc = (k / s).clamp(-448, 448).to(torch.float8_e4m3fn)
        vc = (v / s).clamp(-448, 448).to(torch.float8_e4m3fn)
        ks = s.reshape(1, 1).expand(slots, KV)
        vs = ks
    else:
        kc, ks = O.kv_quantize(k, "int8", torch.float32)
        vc, vs = O.kv_quantize(v, "int8", torch.float32)
    del k, v
    q = torch.randn(requests, H, D, generator=g).to(torch.bfloat16)
    ntok = int(lens.sum())
    nbytes = ntok * KV * D * 2 + (0 if kind == "fp8" else ntok * KV * 2 * 4) + ntok // page * 4 + requests * H * D * 4
    t, n = _cpu_time(lambda: A.paged_decode_reference(q, kc, vc, table, lens, page, D ** -0.5, k_scale=ks,
                                                      v_scale=vs), budget)
    return _cpu_line(round(nbytes / t / 1e9, 3), "GB/s", n,
                     f"calls over {requests} of the 64 requests ({ntok} context tokens), {t * 1e3:.1f} ms/call")


def cpu_moe(budget=6.0):
    """QuantExperts.forward's per-expert loop (modules.py:55-75) with the INT4 method's
    dequantize + F.linear, at config 5."""
    from oracle import moe as MO
    from oracle import quant as O
    T, H, inter, E, k = 64, 2048, 1024, 64, 8
    hidden, w, idx = moe_routing(T, H, E, k)
    g = gen(9)
    gu = O.int4_quantize_symmetric((torch.randn(E, 2 * inter, H, generator=g) * 0.02).to(torch.bfloat16), 128)
    dn = O.int4_quantize_symmetric((torch.randn(E, H, inter, generator=g) * 0.02).to(torch.bfloat16), 128)
    touched = int(idx.unique().numel())
    per_expert = (2 * inter * H // 2 + H * inter // 2) + (2 * inter * H // 128 + H * inter // 128) * 2
    nbytes = touched * per_expert + T * H * 2 * 2 + T * k * 6
    t, n = _cpu_time(lambda: MO.quant_experts_loop(hidden, O.int4_linear, gu, dn, idx, w, E), budget)
    return _cpu_line(round(nbytes / t / 1e9, 3), "GB/s", n, f"layer calls (64 tokens, top-8 of 64 experts), "
                     f"{t * 1e3:.1f} ms/call")


# ---------------------------------------------------------------- HBM traffic (counters)
# The phases of the counter child after the headline, in order: (breakdown entry, key)
TRAFFIC_PHASES = [("int8_w8a16_gate_up_per_M", "M=1"), ("int8_w8a16_gate_up_per_M", "M=8"),
                  ("int8_w8a16_gate_up_per_M", "M=32"), ("int8_w8a16_gate_up_per_M", "M=64"),
                  ("fp8_prefill_gemm", None), ("paged_decode_fp8_kv", None), ("moe_int4_layer", None)]
TRAFFIC_CALLS = 2  # calls per phase


def traffic_child():
    """The run the counter passes watch: four headline launches per round, eagerly; then
    TRAFFIC_CALLS calls of each TRAFFIC_PHASES configuration (INT8 gate_up at every M,
    the FP8 GEMM, FP8-KV paged decode at the default partition, the INT4 MoE layer); then
    the two calibration kernels (a 256 MiB fill, and a sum over a 256 MiB buffer that a
    second fill has evicted from the MALL). A tiny miq_stream_read launch ends each phase,
    so the parent can split the dispatches."""
    from kernels import _lib
    from kernels import quant_ops as ops
    lib = _lib.load()
    dev = torch.device("cuda:0")
    mark_buf = torch.zeros(4096, dtype=torch.uint8, device=dev)
    sink = torch.zeros(4, dtype=torch.int32, device=dev)

    def marker():
        torch.cuda.synchronize()
        lib.miq_stream_read(mark_buf.data_ptr(), 4096, sink.data_ptr(), torch.cuda.current_stream(dev).cuda_stream)
        torch.cuda.synchronize()

    cfg = int4_setup(dev)
    for i in range(3):
        for j, M in enumerate(MS):
            int4_launch(cfg, M, 4 * i + j)()
    del cfg
    marker()
    c8 = int8_setup(dev)
    for M in (1, 8, 32, 64):
        for i in range(TRAFFIC_CALLS):
            q, sc = c8["copies"][i % len(c8["copies"])]
            ops.w8a16_linear(c8["x"][M], q, sc)
        marker()
    del c8
    M, N, K = 2048, 6144, 2560
    w = (torch.randn(N, K, generator=gen(5)) * 0.02).to(torch.bfloat16).to(dev)
    wq, ws = ops.fp8_quantize_rows(w)
    xq, xs = ops.fp8_quantize_rows(torch.randn(M, K, generator=gen(6)).to(torch.bfloat16).to(dev))
    torch.cuda.synchronize()
    marker()
    for _ in range(TRAFFIC_CALLS):
        ops.fp8_gemm(xq, xs, wq, ws)
    marker()
    del w, wq, ws, xq, xs
    from kernels.paged_attention import paged_decode_attention
    a = attention_inputs(dev, "fp8")
    for i in range(TRAFFIC_CALLS):
        kc, vc, ks, vs = a["caches"][i % len(a["caches"])]
        paged_decode_attention(a["q"], kc, vc, a["table"], a["lens"], a["page"], 128 ** -0.5, a["max_len"],
                               k_scale=ks, v_scale=vs)
    marker()
    del a
    from kernels.fused_moe import fused_moe_int4
    c = moe_setup(dev, copies=TRAFFIC_CALLS)
    for i in range(TRAFFIC_CALLS):
        (gq, gs), (dq, ds) = c["sets"][i]
        fused_moe_int4(c["hidden"], c["idx"], c["w"], gq, gs, None, dq, ds, None)
    marker()
    del c
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    a = torch.empty(PROBE_BYTES // 4, dtype=torch.float32, device=dev).fill_(1.0)
    b = torch.empty_like(a).fill_(2.0)
    a.sum()
    torch.cuda.synchronize()
    del a, b


def _pmc_pass(counter, outdir):
    cmd = ["rocprofv3", "--pmc", counter, "--output-format", "csv", "-d", outdir, "-o", "run", "--",
           sys.executable, os.path.abspath(__file__), "--traffic-child"]
    env = dict(os.environ, TMPDIR="/tmp")
    subprocess.run(["timeout", "-s", "KILL", "150"] + cmd, cwd="/tmp", env=env, check=True,
                   stdout=subprocess.DEVNULL, stderr=subprocess.DEVNULL)
    rows = []
    for path in glob.glob(os.path.join(outdir, "**", "*counter_collection.csv"), recursive=True):
        with open(path, newline="") as f:
            rows += [r for r in csv.DictReader(f) if r["Counter_Name"] == counter]
    rows.sort(key=lambda r: int(r["Dispatch_Id"]))
    return rows


def measure_traffic():
    """Per-launch HBM bytes from FETCH_SIZE and WRITE_SIZE passes: the headline kernels per
    M, and per call every TRAFFIC_PHASES configuration. Returns (dict, None) or
    (None, reason)."""
    if shutil.which("rocprofv3") is None:
        return None, "rocprofv3 not found"
    tmp = tempfile.mkdtemp(prefix="miq_traffic_", dir="/tmp")
    try:
        fetch = _pmc_pass("FETCH_SIZE", os.path.join(tmp, "fetch"))
        write = _pmc_pass("WRITE_SIZE", os.path.join(tmp, "write"))
    except (subprocess.CalledProcessError, OSError) as err:
        return None, f"counter pass failed: {err}"
    finally:
        shutil.rmtree(tmp, ignore_errors=True)

    def phases(rows):
        """Dispatches split at the marker launches (stream_read_kernel)."""
        out, cur = [], []
        for r in rows:
            if "stream_read" in r["Kernel_Name"]:
                out.append(cur)
                cur = []
            else:
                cur.append(r)
        out.append(cur)
        return out

    def probe(rows, key):
        hits = [float(r["Counter_Value"]) for r in rows if key(r["Kernel_Name"].lower())]
        return max(hits) if hits else None
    f_probe = probe(fetch, lambda n: "reduce" in n)   # the 256 MiB sum reads 256 MiB
    w_probe = probe(write, lambda n: "fill" in n)     # the 256 MiB fill writes 256 MiB
    fp, wp = phases(fetch), phases(write)
    # phases: headline, int8 M=1, 8, 32, 64, (fp8 operands), fp8 GEMM, attention, MoE, calibration
    if len(fp) != 10 or len(wp) != 10 or not f_probe or not w_probe:
        return None, "phases or calibration dispatches missing from the counter output"
    f_scale = PROBE_BYTES / 1024 / f_probe
    w_scale = PROBE_BYTES / 1024 / w_probe

    def ours(rows):
        return [r for r in rows if "wo_" in r["Kernel_Name"] and "_kernel" in r["Kernel_Name"]]
    fk, wk = ours(fp[0]), ours(wp[0])
    if not fk or len(fk) != len(wk):
        return None, "headline dispatches missing from the counter output"
    per_m = {}
    for i, (fr, wr) in enumerate(zip(fk, wk)):
        M = MS[i % len(MS)]
        per_m.setdefault(M, []).append((float(fr["Counter_Value"]) * f_scale + float(wr["Counter_Value"]) * w_scale) * 1024)
    means = {M: sum(v) / len(v) for M, v in per_m.items()}

    def call_bytes(fr, wr):
        tot = sum(float(r["Counter_Value"]) for r in fr) * f_scale + sum(float(r["Counter_Value"]) for r in wr) * w_scale
        return round(tot * 1024 / TRAFFIC_CALLS)
    # the kernels of each phase's calls (the phase also holds its setup: quantize, fills)
    wo = lambda n: "wo_" in n  # noqa: E731
    keep = [wo, wo, wo, wo, lambda n: "fp8_gemm" in n, lambda n: "paged_decode" in n,
            lambda n: "moe" in n and "quantize" not in n]
    sections = {}
    for (name, key), sel, i in zip(TRAFFIC_PHASES, keep, (1, 2, 3, 4, 6, 7, 8)):
        b = call_bytes([r for r in fp[i] if sel(r["Kernel_Name"])], [r for r in wp[i] if sel(r["Kernel_Name"])])
        if key is None:
            sections[name] = b
        else:
            sections.setdefault(name, {})[key] = b
    return {"bytes_per_launch": round(sum(means.values()) / len(means)),
            "per_M_bytes": {f"M={M}": round(v) for M, v in sorted(means.items())},
            "sections": sections,
            "fetch_scale": round(f_scale, 4), "write_scale": round(w_scale, 4),
            "dispatches": len(fk)}, None


def attach_traffic(breakdown, sections):
    """Adds each configuration's measured HBM bytes per call (counter passes of this run)
    beside its algorithmic bytes."""
    def put(entry, traffic, algorithmic):
        entry["traffic_bytes_per_call"] = traffic
        entry["algorithmic_bytes_per_call"] = round(algorithmic)
        entry["traffic_over_algorithmic"] = round(traffic / algorithmic, 3)
    N8, K8 = 19456, 2560
    for key, b in sections.get("int8_w8a16_gate_up_per_M", {}).items():
        M = int(key.split("=")[1])
        if key in breakdown.get("int8_w8a16_gate_up_per_M", {}):
            put(breakdown["int8_w8a16_gate_up_per_M"][key], b, N8 * K8 + N8 * 4 + M * K8 * 2 + M * N8 * 2)
    if "fp8_prefill_gemm" in sections and "fp8_prefill_gemm" in breakdown:
        M, N, K = 2048, 6144, 2560
        put(breakdown["fp8_prefill_gemm"], sections["fp8_prefill_gemm"], M * K + N * K + 4 * (M + N) + M * N * 2)
    if "paged_decode_fp8_kv" in sections and "paged_decode_fp8_kv" in breakdown:
        e = breakdown["paged_decode_fp8_kv"]
        put(e, sections["paged_decode_fp8_kv"], e["MB_per_call"] * 1e6)
        e["traffic_partition"] = e.get("default_partition")
    if "moe_int4_layer" in sections and "moe_int4_layer" in breakdown:
        e = breakdown["moe_int4_layer"]
        put(e, sections["moe_int4_layer"], e["MB_per_call"] * 1e6)


SECTIONS = {
    "int4_w4a16_sym_per_M": lambda dev: per_m(int4_setup(dev), int4_launch, int4_bytes, dev,
                                              ref_launch=int4_ref_launch),
    "int4_w4a16_zero_point_per_M": bench_int4_asym,
    "int8_w8a16_gate_up_per_M": bench_int8,
    "fp8_prefill_gemm": bench_fp8,
    "wo_prefill_large_M": bench_wo_prefill,
    "paged_decode_fp8_kv": lambda dev: bench_attention(dev, "fp8"),
    "paged_decode_int8_kv": lambda dev: bench_attention(dev, "int8"),
    "moe_int4_layer": bench_moe,
    "moe_int8_layer": bench_moe_int8,
    "moe_fp8_layer": bench_moe_fp8,
}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-traffic", action="store_true", help="skip the rocprofv3 counter passes")
    ap.add_argument("--traffic-child", action="store_true", help=argparse.SUPPRESS)
    ap.add_argument("--only", choices=["headline", "all"] + list(SECTIONS), default="all",
                    help="headline: the headline line only; a section name: that configuration alone "
                         "(for profiling runs; prints its breakdown entry)")
    args = ap.parse_args()
    if args.traffic_child:
        traffic_child()
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the quantized path has no multi-GPU code (every GPU box "
              "here has one GPU); run it with --gpus 1", file=sys.stderr)
        sys.exit(2)
    # the counter passes run as child processes before this process initialises the GPU
    traffic, traffic_note = (None, "skipped (--no-traffic)")
    if not args.no_traffic:
        log("[bench] HBM traffic: rocprofv3 FETCH_SIZE / WRITE_SIZE passes")
        traffic, traffic_note = measure_traffic()
        log(f"[bench]   {traffic or traffic_note}")
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        sys.exit(2)
    from kernels import _lib
    _lib.load()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.only in SECTIONS:
        print(json.dumps({args.only: SECTIONS[args.only](dev)}), flush=True)
        return

    log("[bench] headline: INT4 W4A16 decode GEMM sweep")
    cfg, step_bytes, t = bench_headline(dev, args.steps, args.warmup)
    launch_bytes = [int4_bytes(cfg, M) for M in MS]
    del cfg
    torch.cuda.empty_cache()
    floor_step_us = round(sum(stream_floor_us(nb, dev) for nb in launch_bytes), 2)
    ms_per_step = t / args.steps * 1e3
    value = step_bytes * args.steps / t / 1e9
    avg_kernel_us = t / (4 * args.steps) * 1e6
    breakdown = {}
    cpu_fns = {"int4_w4a16_sym_per_M": None, "int8_w8a16_gate_up_per_M": cpu_int8, "fp8_prefill_gemm": cpu_fp8,
               "paged_decode_fp8_kv": lambda: cpu_attention("fp8"), "paged_decode_int8_kv": lambda: cpu_attention("int8"),
               "moe_int4_layer": cpu_moe}
    if args.only == "all":
        for name, fn in SECTIONS.items():
            fn = (lambda f: (lambda: f(dev)))(fn)
            log(f"[bench] {name}")
            breakdown[name] = fn()
            torch.cuda.empty_cache()
            log(f"[bench]   {breakdown[name]}")
    if traffic and args.only == "all":
        attach_traffic(breakdown, traffic["sections"])
    cpu = None
    if not args.no_cpu:
        torch.set_num_threads(len(os.sched_getaffinity(0)))
        log("[bench] cpu baseline (headline)")
        cpu = cpu_int4_headline()
        log(f"[bench]   {cpu}")
        if args.only == "all":
            for name, fn in cpu_fns.items():
                if fn is None:
                    breakdown[name]["cpu_baseline"] = cpu
                    continue
                log(f"[bench] cpu baseline ({name})")
                breakdown[name]["cpu_baseline"] = fn()
                log(f"[bench]   {breakdown[name]['cpu_baseline']}")
    roofline = {"bound": "hbm", "achieved": round(value, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(value / HBM_PEAK_GBS, 4),
                "traffic": traffic["bytes_per_launch"] if traffic else None,
                "traffic_unit": "bytes per launch (HBM, rocprofv3 FETCH_SIZE + WRITE_SIZE, calibrated)",
                "algorithmic_bytes_per_launch": round(step_bytes / 4),
                "kernel": "wo_gemv_kernel<int4> (M=1), wo_tile_kernel<int4> (M=8) and wo_panel_kernel<int4> (M=32, 64)",
                "avg_kernel_us": round(avg_kernel_us, 3),
                "stream_floor_us_per_step": floor_step_us,
                "frac_of_stream_floor": round(floor_step_us / (t / args.steps * 1e6), 3),
                "stream_floor_note": "miq_stream_read of each launch's algorithmic bytes, same graph timing; "
                                     "includes the per-launch cost a graph node has on this GPU"}
    if traffic:
        roofline["traffic_per_M"] = traffic["per_M_bytes"]
        roofline["traffic_calibration"] = {"fetch_scale": traffic["fetch_scale"], "write_scale": traffic["write_scale"]}
    else:
        roofline["traffic_note"] = traffic_note
    line = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,0.02) weights quantized on the device, N(0,1) activations)",
        "config": {"workload": "INT4 W4A16 decode GEMM, Qwen3-4B down_proj N=2560 K=9728, group 128 symmetric, "
                               "one step = M in {1,8,32,64}", "global_batch": list(MS), "parallelism": "none (1 GPU)"},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "breakdown": breakdown,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
