"""Benchmark of the quantized decode path on one MI355X.

One step = the four INT4 W4A16 decode GEMMs of the headline configuration (Qwen3-4B
down_proj: N=2560, K=9728, group 128, symmetric codes, bf16 activations) at
M = 1, 8, 32, 64 rows. `value` = algorithmic bytes of the step / its time, inputs
resident in HBM. Every launch reads its own copy of the weights (copies rotate over
more than 512 MiB), so the 256 MiB MALL cannot serve the weights from cache.

The timed region is one replay of a HIP graph holding exactly --steps steps, bracketed by
torch.cuda.synchronize() and HIP events on the stream the kernels run on; the average
kernel duration is that time / (4 * steps) (the launches run back to back in the graph).

`breakdown` reports the other configurations the same way (INT8 gate_up GEMM, FP8
prefill GEMM, paged decode attention on FP8 / INT8 KV, INT4 MoE layer); `cpu_baseline`
times the reference formulas restated on the CPU (oracle/) on a bounded sample.

Usage: python bench.py [--gpus 1] [--steps 50] [--warmup 10] [--no-cpu] [--only headline]
"""
import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "mini-inference_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import torch  # noqa: E402

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E, published
FP8_PEAK_TFLOPS = 5000.0     # MI355X dense FP8 MFMA, published
ROTATE_BYTES = 600 * 2 ** 20  # > 2 x MALL
METRIC = "quantized decode GEMM GB/s (% HBM peak) at M=1..64; FP8-KV attn µs/step"
MS = (1, 8, 32, 64)
# HBM bytes per headline launch (mean over M = 1, 8, 32, 64), from rocprofv3 FETCH_SIZE /
# WRITE_SIZE passes of `bench.py --only headline --copy-probe`, scaled by the counters'
# readings for a 256 MiB sum and fill (profiles/wo_int4_headline_traffic.md).
# Re-measure when the kernel changes.
HEADLINE_TRAFFIC_BYTES = 21_413_092


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


def per_m(cfg, launch, nbytes, dev, reps_per_graph=40):
    out = {}
    for M in MS:
        t = time_graph([launch(cfg, M, i) for i in range(reps_per_graph)]) / reps_per_graph
        gbs = nbytes(cfg, M) / t / 1e9
        out[f"M={M}"] = {"us": round(t * 1e6, 2), "GB/s": round(gbs, 1), "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 1)}
    return out


def bench_int8(dev):
    from kernels import quant_ops as ops
    cfg = int8_setup(dev)

    def launch(c, M, i):
        q, s = c["copies"][i % len(c["copies"])]
        x = c["x"][M]
        return lambda: ops.w8a16_linear(x, q, s)

    nbytes = lambda c, M: c["wbytes"] + M * c["K"] * 2 + M * c["N"] * 2  # noqa: E731
    res = per_m(cfg, launch, nbytes, dev, reps_per_graph=24)
    del cfg
    return res


def bench_int4_asym(dev):
    cfg = int4_setup(dev, symmetric=False)
    res = per_m(cfg, int4_launch, int4_bytes, dev)
    del cfg
    return res


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
    return {"gemm_us": round(t_gemm * 1e6, 2), "gemm_TFLOP/s": round(tf, 1),
            "pct_fp8_peak": round(100 * tf / FP8_PEAK_TFLOPS, 1),
            "act_quant_us": round(t_quant * 1e6, 2),
            "quant+gemm_TFLOP/s": round(tf_all, 1), "peak_used_TFLOP/s": FP8_PEAK_TFLOPS}


def attention_inputs(dev, kind, B=64, H=32, KV=8, D=128, page=16, seed=7):
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
    slots = total * page
    # K/V ~ N(0,1) generated on the device from a seeded generator (570 MB of codes)
    dg = torch.Generator(device=dev).manual_seed(seed)
    k = torch.randn(slots, KV, D, generator=dg, device=dev)
    v = torch.randn(slots, KV, D, generator=dg, device=dev)
    if kind == "fp8":
        s = torch.tensor(4.0 / 448.0, device=dev)
        kc = (k / s).clamp(-448, 448).to(torch.float8_e4m3fn)
        vc = (v / s).clamp(-448, 448).to(torch.float8_e4m3fn)
        ks = s.reshape(1, 1).expand(slots, KV)
        vs = ks
        scale_bytes = 0
    else:
        from engine.core.kv_cache import kv_quant_write
        kc = torch.empty(slots, KV, D, dtype=torch.int8, device=dev)
        vc = torch.empty_like(kc)
        ks = torch.empty(slots, KV, dtype=torch.float32, device=dev)
        vs = torch.empty_like(ks)
        idx = torch.arange(slots, device=dev)
        kv_quant_write(kc, ks, idx, k)
        kv_quant_write(vc, vs, idx, v)
        scale_bytes = int(lens.sum()) * KV * 2 * 4
    del k, v
    q = torch.randn(B, H, D, generator=g).to(torch.bfloat16).to(dev)
    ntok = int(lens.sum())
    nbytes = ntok * KV * D * 2 + scale_bytes + sum(pages) * 4 + B * H * D * 2 * 2 + B * 4
    return dict(q=q, k=kc, v=vc, ks=ks, vs=vs, table=table.to(dev), lens=lens.to(torch.int32).to(dev),
                max_len=int(lens.max()), page=page, bytes=nbytes, tokens=ntok)


def bench_attention(dev, kind):
    from kernels.paged_attention import paged_decode_attention
    a = attention_inputs(dev, kind)

    def f():
        return paged_decode_attention(a["q"], a["k"], a["v"], a["table"], a["lens"], a["page"], 128 ** -0.5,
                                      8192, k_scale=a["ks"], v_scale=a["vs"])
    reps = 20
    t = time_graph([f] * reps) / reps
    gbs = a["bytes"] / t / 1e9
    res = {"us_per_step": round(t * 1e6, 2), "GB/s": round(gbs, 1), "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 1),
           "context_tokens": a["tokens"], "MB_per_call": round(a["bytes"] / 1e6, 1)}
    del a
    return res


def moe_setup(dev, copies=None):
    from kernels import quant_ops as ops
    T, H, inter, E, k = 64, 2048, 1024, 64, 8
    g = gen(8)
    hidden = torch.randn(T, H, generator=g).to(torch.bfloat16).to(dev)
    router = (torch.randn(E, H, generator=g) * 0.02).to(torch.bfloat16).to(dev)
    probs = torch.softmax(hidden.float() @ router.float().t(), dim=-1)
    w, idx = torch.topk(probs, k, dim=-1)
    w = w.to(torch.bfloat16)
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
    res = {"us_per_layer": round(t * 1e6, 2), "GB/s": round(gbs, 1), "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 1),
           "experts_touched": c["touched"], "MB_per_call": round(c["bytes"] / 1e6, 1)}
    del c
    return res


# ---------------------------------------------------------------- CPU baseline (oracle)
def cpu_baseline_headline(budget_s=20.0):
    """The reference's CPU path for the headline step: Int4WeightOnly.linear =
    dequantize (int4_wo.py:33-42) + F.linear (base.py:20-24), restated in oracle/quant.py,
    at the four M values; bounded: as many whole steps as fit in ~budget_s (at least one)."""
    from oracle import quant as O
    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    N, K = 2560, 9728
    w = (torch.randn(N, K, generator=gen(2)) * 0.02).to(torch.bfloat16)
    q = O.int4_quantize_symmetric(w, 128)
    xs = {M: torch.randn(M, K, generator=gen(3)).to(torch.bfloat16) for M in MS}
    O.int4_linear(xs[1], **q)  # warm-up
    wbytes = q["qweight"].numel() + q["scale"].numel() * 2
    step_bytes = sum(wbytes + M * K * 2 + M * N * 2 for M in MS)
    times = []
    t_start = time.perf_counter()
    while True:
        t0 = time.perf_counter()
        for M in MS:
            O.int4_linear(xs[M], **q)
        times.append(time.perf_counter() - t0)
        if time.perf_counter() - t_start > budget_s or len(times) >= 10:
            break
    times.sort()
    t = times[len(times) // 2]
    cpu = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"value": round(step_bytes / t / 1e9, 3), "unit": "GB/s", "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"{len(times)} whole steps (4 INT4 linears, M=1/8/32/64, N=2560 K=9728), median "
                      f"{t * 1e3:.1f} ms/step; oracle int4 dequantize + F.linear in bf16; {cpu}; torch {torch.__version__}"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--only", choices=["headline", "all"], default="all")
    ap.add_argument("--copy-probe", action="store_true",
                    help="also run a 256 MiB fill and a 256 MiB sum (the reference kernels for scaling "
                         "rocprofv3 WRITE_SIZE / FETCH_SIZE readings to bytes)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the quantized path has no multi-GPU code (every GPU box "
              "here has one GPU); run it with --gpus 1", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        sys.exit(2)
    from kernels import _lib
    _lib.load()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)

    log("[bench] headline: INT4 W4A16 decode GEMM sweep")
    cfg, step_bytes, t = bench_headline(dev, args.steps, args.warmup)
    del cfg
    torch.cuda.empty_cache()
    if args.copy_probe:
        # known-size reference kernels: a 256 MiB fill (writes 256 MiB) and a sum over it
        # (reads 256 MiB); the buffer is 256 MiB, the same as the MALL, so a second 256 MiB
        # fill in between evicts it before the sum
        a = torch.empty(64 * 2 ** 20, dtype=torch.float32, device=dev).fill_(1.0)
        b = torch.empty_like(a).fill_(2.0)
        a.sum()
        torch.cuda.synchronize()
        del a, b
    ms_per_step = t / args.steps * 1e3
    value = step_bytes * args.steps / t / 1e9
    avg_kernel_us = t / (4 * args.steps) * 1e6
    breakdown = {}
    if args.only == "all":
        for name, fn in (("int4_w4a16_sym_per_M", lambda: per_m(int4_setup(dev), int4_launch, int4_bytes, dev)),
                         ("int4_w4a16_zero_point_per_M", lambda: bench_int4_asym(dev)),
                         ("int8_w8a16_gate_up_per_M", lambda: bench_int8(dev)),
                         ("fp8_prefill_gemm", lambda: bench_fp8(dev)),
                         ("paged_decode_fp8_kv", lambda: bench_attention(dev, "fp8")),
                         ("paged_decode_int8_kv", lambda: bench_attention(dev, "int8")),
                         ("moe_int4_layer", lambda: bench_moe(dev))):
            log(f"[bench] {name}")
            breakdown[name] = fn()
            torch.cuda.empty_cache()
            log(f"[bench]   {breakdown[name]}")
    cpu = None
    if not args.no_cpu:
        log("[bench] cpu baseline")
        cpu = cpu_baseline_headline()
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
        "roofline": {"bound": "hbm", "achieved": round(value, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(value / HBM_PEAK_GBS, 4), "traffic": HEADLINE_TRAFFIC_BYTES,
                     "traffic_unit": "bytes per launch", "algorithmic_bytes_per_launch": round(step_bytes / 4),
                     "kernel": "wo_tile_kernel<KIND_INT4> (M=1, 8) and wo_stream_kernel<KIND_INT4> (M=32, 64)",
                     "avg_kernel_us": round(avg_kernel_us, 3)},
        "cpu_baseline": cpu,
        "breakdown": breakdown,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
