#!/usr/bin/env python3
"""Benchmark of the paged-attention hot path on one MI355X.

Default workload (the headline metric): paged decode at the GQA
Qwen2.5-7B shape - 128 sequences, 28 query / 4 kv heads, head_dim 128,
block 16, bf16, context lengths uniform in [256, 8192] (seeded per
sequence), pool sized to the tokens + 10 %, blocks scattered at random.
A step is one decode pass over the batch (balanced stream decode + LSE merge).
Inputs are resident in HBM before the timed region.

Prints one JSON line (stdout) with the whole-job throughput in GB/s of
algorithmic bytes (K/V read once per kv head + q + out + block tables),
tokens/s, a roofline entry for the dominant kernel timed with HIP events on
its own stream, and the CPU baseline: this repository's restatement of the
reference CpuAttentionBackend (the oracle) timed on the host cores over the
same sequences.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config qwen7b]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import platform
import sys
import time

METRIC = "decode-attn HBM GB/s (% of ~8 TB/s peak) + tokens/sec at GQA-7B shape, 1 GPU"
PEAK_HBM_GBS = 8000.0        # MI355X HBM3E
PEAK_BF16_TFLOPS = 2500.0    # MI355X dense bf16/fp16 MFMA

DECODE_CONFIGS = {
    # name: (num_seqs, hq, hkv, head_dim, dtype, context spec, value scale, seed, partition)
    "opt125m": dict(num_seqs=8, hq=12, hkv=12, d=64, dtype="float32", ctx=("fixed", 128),
                    vscale=1.0, seed=1001, partition=None,
                    workload="paged decode, OPT-125m shape: 8 seqs, 12 heads, head_dim 64, "
                             "block 16, fp32, context 128"),
    "llama7b": dict(num_seqs=64, hq=32, hkv=32, d=128, dtype="float16", ctx=("fixed", 2048),
                    vscale=0.5, seed=1002, partition=None,
                    workload="paged decode, MHA Llama-7B shape: 64 seqs, 32 heads, head_dim 128, "
                             "block 16, fp16, context 2048"),
    "qwen7b": dict(num_seqs=128, hq=28, hkv=4, d=128, dtype="bfloat16", ctx=("uniform", 256, 8192),
                   vscale=1.0, seed=1003, partition=None,
                   workload="paged decode, GQA Qwen2.5-7B shape: 128 seqs, 28 q / 4 kv heads, "
                            "head_dim 128, block 16, bf16, context U[256,8192] seeded per sequence"),
    # The same batch over fp32 pools: the reference's default resident KV
    # dtype and what its CPU dense nodes hand over (src/core/nodes.py:21-24).
    "qwen7b_fp32": dict(num_seqs=128, hq=28, hkv=4, d=128, dtype="float32",
                        ctx=("uniform", 256, 8192), vscale=1.0, seed=1003, partition=None,
                        workload="paged decode, GQA Qwen2.5-7B shape over fp32 pools: 128 seqs, "
                                 "28 q / 4 kv heads, head_dim 128, block 16, fp32, context "
                                 "U[256,8192] seeded per sequence"),
    "long32k": dict(num_seqs=16, hq=32, hkv=8, d=128, dtype="float16", ctx=("fixed", 32768),
                    vscale=1.0, seed=1004, partition=512,
                    workload="split-K paged decode: 16 seqs, 32 q / 8 kv heads, head_dim 128, "
                             "block 16, fp16, context 32768, partition 512"),
}


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def context_lengths(cfg) -> list[int]:
    import torch

    kind = cfg["ctx"][0]
    if kind == "fixed":
        return [cfg["ctx"][1]] * cfg["num_seqs"]
    lo, hi = cfg["ctx"][1], cfg["ctx"][2]
    return [int(torch.randint(lo, hi + 1, (1,),
                              generator=torch.Generator().manual_seed(cfg["seed"] * 1000 + i)))
            for i in range(cfg["num_seqs"])]


def decode_workload(cfg, dev):
    """Seeded paged pools, block tables and queries on the device."""
    import torch

    dtype = getattr(torch, cfg["dtype"])
    bs = 16
    ctx = context_lengths(cfg)
    need = [max(1, math.ceil(c / bs)) for c in ctx]
    nb = math.ceil(1.1 * sum(need)) if cfg["ctx"][0] == "uniform" else sum(need)
    g = torch.Generator().manual_seed(cfg["seed"])
    perm = torch.randperm(nb, generator=g)
    width = max(need)
    table = torch.full((len(ctx), width), -1, dtype=torch.int32)
    pos = 0
    for i, n in enumerate(need):
        table[i, :n] = perm[pos:pos + n].to(torch.int32)
        pos += n
    gd = torch.Generator(device=dev).manual_seed(cfg["seed"])
    shape = (nb, bs, cfg["hkv"], cfg["d"])
    k = (torch.randn(shape, generator=gd, device=dev, dtype=torch.float32) * cfg["vscale"]).to(dtype)
    v = (torch.randn(shape, generator=gd, device=dev, dtype=torch.float32) * cfg["vscale"]).to(dtype)
    q = (torch.randn((len(ctx), cfg["hq"], cfg["d"]), generator=gd, device=dev,
                     dtype=torch.float32) * cfg["vscale"]).to(dtype)
    eb = torch.finfo(dtype).bits // 8
    kv_bytes = sum(ctx) * cfg["hkv"] * cfg["d"] * eb * 2
    qo_bytes = len(ctx) * cfg["hq"] * cfg["d"] * eb * 2
    tbl_bytes = sum(math.ceil(c / bs) for c in ctx) * 4 + len(ctx) * 4
    return dict(ctx=ctx, bs=bs, k=k, v=v, q=q, table=table.to(dev),
                ctx_dev=torch.tensor(ctx, dtype=torch.int32, device=dev),
                table_host=table, algo_bytes=kv_bytes + qo_bytes + tbl_bytes,
                flops=4 * sum(ctx) * cfg["hq"] * cfg["d"], dtype=dtype, scale=cfg["d"] ** -0.5)


def _event_us(ev, a: int, b: int):
    """Mean and median, in microseconds, of the intervals between events a and
    b of every timed step (the mean is what the roofline divides by)."""
    d = sorted(e[a].elapsed_time(e[b]) * 1e3 for e in ev)
    n = len(d)
    med = d[n // 2] if n % 2 else 0.5 * (d[n // 2 - 1] + d[n // 2])
    return sum(d) / n, med


def cpu_baseline(cfg, w, budget_s: float):
    """The oracle's restatement of CpuAttentionBackend (fp32 upcast, grouped
    einsum, softmax, einsum) over the batch's sequences on the host cores."""
    import torch
    from oracle import attention as oa

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    bs = w["bs"]
    kc, vc, q = w["k"].cpu(), w["v"].cpu(), w["q"].cpu()
    seqs = []
    for i, c in enumerate(w["ctx"]):
        kk, vv = oa.gather_context(kc, vc, w["table_host"][i].tolist(), c)
        seqs.append((q[i], kk.contiguous(), vv.contiguous()))
    del kc, vc
    # Whole passes over the batch (one decode step per sequence) until the
    # budget is spent; a pass that would not fit the budget stops at the
    # sequence where the budget runs out (at least one sequence).
    eb = torch.finfo(w["dtype"]).bits // 8
    t0 = time.perf_counter()
    passes, done, nbytes, tokens = 0, 0, 0, 0
    while True:
        for qi, kk, vv in seqs:
            oa.attend(qi, kk, vv, w["scale"]).to(w["dtype"])
            done += 1
            nbytes += kk.numel() * eb * 2 + qi.numel() * eb * 2
            tokens += 1
            if time.perf_counter() - t0 > budget_s:
                break
        else:
            passes += 1
            continue
        break
    dt = time.perf_counter() - t0
    # One pass (or the part done above) with the reference's torch.cat append
    # in front of each step.
    t1 = time.perf_counter()
    cat_bytes = 0
    for qi, kk, vv in seqs[:done]:
        k2 = torch.cat([kk, kk[-1:]], dim=0)
        v2 = torch.cat([vv, vv[-1:]], dim=0)
        oa.attend(qi, k2, v2, w["scale"]).to(w["dtype"])
        cat_bytes += kk.numel() * eb * 2 + qi.numel() * eb * 2
    dt_cat = time.perf_counter() - t1
    cpu_model = platform.processor() or "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu_model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {
        "value": nbytes / dt / 1e9,
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": f"{done} decode steps = {passes} whole passes over the {len(seqs)} sequences of the "
                  f"same batch + {done - passes * len(seqs)} more, one step per sequence "
                  f"(fp32 upcast + einsum + softmax + einsum, as CpuAttentionBackend.decode_layer)",
        "seconds": dt,
        "tokens_per_s": tokens / dt,
        "with_cat_append_gbs": cat_bytes / dt_cat / 1e9,
        "cpu_model": cpu_model,
    }


def bench_decode(args, cfg):
    import torch
    from cloverinfer_amd import kernels

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    log(f"building workload {args.config}")
    w = decode_workload(cfg, dev)
    out = torch.empty_like(w["q"])
    max_ctx = max(w["ctx"])
    # A pool smaller than 512 MiB would be served from the 256 MB Infinity
    # Cache after the first step: such workloads rotate over enough copies of
    # the pools to stream at least 512 MiB between two visits of one copy.
    pool_bytes = 2 * w["k"].numel() * w["k"].element_size()
    copies = max(1, math.ceil((512 << 20) / pool_bytes))
    pools = [(w["k"], w["v"])] + [(w["k"].clone(), w["v"].clone()) for _ in range(copies - 1)]
    args_list = [kernels.decode_args(out, w["q"], kc, vc, w["table"], w["ctx_dev"], w["bs"],
                                     max_ctx, scale=w["scale"]) for kc, vc in pools]
    a = args_list[0]
    part = args.partition if args.partition is not None else cfg["partition"]
    if part is not None and part < 0:  # explicit request for the automatic schedule
        part = None
    if part is None:
        if kernels.balanced_supported(a):
            mode = "balanced"
        else:
            hq, hkv = cfg["hq"], cfg["hkv"]
            part = kernels.choose_partition(len(w["ctx"]), hkv, hq // hkv, max_ctx,
                                            kernels.num_compute_units(dev))
            mode = "split" if part > 0 and max_ctx > part else "single"
    else:
        mode = "split" if part > 0 and max_ctx > part else "single"
    stream = torch.cuda.current_stream(dev)
    lib = kernels._native.load()
    waves = args.waves
    if mode == "balanced":
        ws = kernels.splitk_workspace(dev, kernels.balanced_workspace_bytes(a, waves))
    elif mode == "split":
        ws = kernels.splitk_workspace(dev, kernels.workspace_bytes(a, part))
    else:
        ws = None

    def first_half(i=0):
        a = args_list[i % copies]
        if mode == "balanced":
            kernels.balanced_partials(a, waves, ws, stream.cuda_stream)
        elif mode == "split":
            kernels.paged_decode_partials(a, part, ws, stream.cuda_stream)
        else:
            kernels._native.check(lib.clv_paged_decode(a, stream.cuda_stream), "clv_paged_decode")

    def second_half(i=0):
        a = args_list[i % copies]
        if mode == "balanced":
            kernels.balanced_reduce(a, waves, ws, stream.cuda_stream)
        elif mode == "split":
            kernels.splitk_reduce(a, part, ws, stream.cuda_stream)

    def step(i=0):
        first_half(i)
        second_half(i)

    log(f"warmup {args.warmup} (mode {mode}, partition {part if mode == 'split' else 0}, "
        f"{copies} pool copies)")
    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    log(f"timing {args.steps} steps")
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(args.warmup + i)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = wall / args.steps * 1e3

    # Per-kernel durations: HIP events on the stream the kernels run on. A
    # leading device-side sleep keeps the GPU busy while every launch is
    # queued, so host launch gaps stay out of the event intervals.
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(args.steps)]
    torch.cuda._sleep(50_000_000)
    for i, e in enumerate(ev):
        e[0].record(stream)
        first_half(i)
        e[1].record(stream)
        second_half(i)
        e[2].record(stream)
    torch.cuda.synchronize()
    dec_us, dec_med = _event_us(ev, 0, 1)
    red_us, red_med = _event_us(ev, 1, 2)
    log(f"step {ms:.4f} ms, decode kernel {dec_us:.1f} us, reduce {red_us:.1f} us")

    value = w["algo_bytes"] / (ms * 1e-3) / 1e9
    achieved = w["algo_bytes"] / (dec_us * 1e-6) / 1e9
    traffic = None
    tpath = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                         f"traffic_{args.config}.json")
    if os.path.exists(tpath):
        traffic = json.load(open(tpath)).get("hbm_bytes_per_launch")
    result = {
        "metric": METRIC,
        "value": value,
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": {"float32": "f32", "float16": "f16", "bfloat16": "bf16"}[cfg["dtype"]],
        "data": "synthetic N(0,1) q/K/V, random init, seeded; no model weights",
        "config": {
            "workload": cfg["workload"],
            "num_seqs": len(w["ctx"]),
            "num_heads": cfg["hq"],
            "num_kv_heads": cfg["hkv"],
            "head_dim": cfg["d"],
            "block_size": w["bs"],
            "total_context_tokens": sum(w["ctx"]),
            "max_context_len": max_ctx,
            "schedule": mode,
            "partition_size": part if mode == "split" else 0,
            "kv_pool_copies": copies,
            "algorithmic_bytes_per_step": w["algo_bytes"],
            "seed": cfg["seed"],
        },
        "tokens_per_s": len(w["ctx"]) / (ms * 1e-3),
        "hbm_frac_of_peak": value / PEAK_HBM_GBS,
        "kernels_us": {"paged_decode": dec_us, "merge": red_us},
        "kernels_us_median": {"paged_decode": dec_med, "merge": red_med},
        "roofline": {
            "bound": "hbm",
            "kernel": {"balanced": "paged_decode_stream", "split": "paged_decode_mfma",
                       "single": "paged_decode_mfma"}[mode] if cfg["d"] in (64, 128)
                      else "paged_decode_valu",
            "achieved": achieved,
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": achieved / PEAK_HBM_GBS,
            "traffic": traffic,
        },
    }
    if not args.no_cpu:
        log("cpu baseline")
        result["cpu_baseline"] = cpu_baseline(cfg, w, args.cpu_budget)
    return result


def bench_decode_fp8(args):
    """The GQA Qwen2.5-7B decode batch with fp8 (OCP e4m3) pools: K/V are
    the same seeded N(0,1) data stored as e4m3 with scale 1 per kv head; q
    and out stay bf16. A step is one clv_paged_decode_fp8 call (stream decode
    + merge)."""
    import torch
    from cloverinfer_amd import kernels

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    cfg = DECODE_CONFIGS["qwen7b"]
    log("building workload qwen7b_fp8")
    w = decode_workload(cfg, dev)
    k8 = w["k"].float().clamp(-448, 448).to(kernels.FP8)
    v8 = w["v"].float().clamp(-448, 448).to(kernels.FP8)
    del w["k"], w["v"]
    ones = torch.ones(cfg["hkv"], dtype=torch.float32, device=dev)
    out = torch.empty_like(w["q"])
    max_ctx = max(w["ctx"])
    a = kernels.decode_args(out, w["q"], k8, v8, w["table"], w["ctx_dev"], w["bs"], max_ctx,
                            scale=w["scale"])
    lib = kernels._native.load()
    stream = torch.cuda.current_stream(dev)
    waves = args.waves or lib.clv_default_num_waves_fp8()
    ws = kernels.splitk_workspace(dev, kernels.balanced_workspace_bytes(a, waves))

    def step():
        kernels._native.check(lib.clv_paged_decode_fp8(a, ones.data_ptr(), ones.data_ptr(),
                                                       waves, ws.data_ptr(), ws.numel(),
                                                       stream.cuda_stream), "clv_paged_decode_fp8")

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) / args.steps * 1e3
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(2)] for _ in range(args.steps)]
    torch.cuda._sleep(50_000_000)
    for e in ev:
        e[0].record(stream)
        step()
        e[1].record(stream)
    torch.cuda.synchronize()
    call_us, call_med = _event_us(ev, 0, 1)
    ctx = w["ctx"]
    kv_bytes = sum(ctx) * cfg["hkv"] * cfg["d"] * 1 * 2
    qo_bytes = len(ctx) * cfg["hq"] * cfg["d"] * 2 * 2
    tbl_bytes = sum(math.ceil(c / w["bs"]) for c in ctx) * 4 + len(ctx) * 4
    algo = kv_bytes + qo_bytes + tbl_bytes
    log(f"step {ms:.4f} ms, decode + merge {call_us:.1f} us")
    return {
        "metric": "decode-attn HBM GB/s, fp8 KV pools, GQA-7B shape, 1 GPU",
        "value": algo / (ms * 1e-3) / 1e9, "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": ms, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "fp8-kv/bf16",
        "data": "synthetic N(0,1) q/K/V, random init, seeded; K/V stored as e4m3, scale 1",
        "config": {"workload": "paged decode over fp8 (e4m3) pools, GQA Qwen2.5-7B shape: 128 seqs, "
                               "28 q / 4 kv heads, head_dim 128, block 16, q/out bf16, "
                               "context U[256,8192] seeded per sequence",
                   "total_context_tokens": sum(ctx), "algorithmic_bytes_per_step": algo,
                   "seed": cfg["seed"]},
        "tokens_per_s": len(ctx) / (ms * 1e-3),
        "kernels_us": {"paged_decode_fp8_with_merge": call_us},
        "kernels_us_median": {"paged_decode_fp8_with_merge": call_med},
        "roofline": {"bound": "hbm", "kernel": "paged_decode_stream (fp8) + merge",
                     "achieved": algo / (call_us * 1e-6) / 1e9, "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": algo / (call_us * 1e-6) / 1e9 / PEAK_HBM_GBS,
                     "traffic": None},
    }


def bench_prefill(args):
    """Chunked prefill, 8 sequences x (4096 cached + 512 new), 32 q / 8 kv
    heads, head_dim 128, bf16: a step appends the 512 new K/V rows of every
    sequence (reshape_and_cache) and runs the causal chunk attention."""
    import torch
    from cloverinfer_amd import kernels

    dev = torch.device("cuda", 0)
    S, cached, new, hq, hkv, d, bs = 8, 4096, 512, 32, 8, 128, 16
    seed = 1005
    ctx = [cached + new] * S
    need = [math.ceil(c / bs) for c in ctx]
    nb = sum(need)
    g = torch.Generator().manual_seed(seed)
    perm = torch.randperm(nb, generator=g)
    table = perm.view(S, -1).to(torch.int32).to(dev)
    gd = torch.Generator(device=dev).manual_seed(seed)
    k = torch.randn((nb, bs, hkv, d), generator=gd, device=dev).to(torch.bfloat16)
    v = torch.randn((nb, bs, hkv, d), generator=gd, device=dev).to(torch.bfloat16)
    q = torch.randn((S * new, hq, d), generator=gd, device=dev).to(torch.bfloat16)
    kn = torch.randn((S * new, hkv, d), generator=gd, device=dev).to(torch.bfloat16)
    vn = torch.randn((S * new, hkv, d), generator=gd, device=dev).to(torch.bfloat16)
    pos = torch.arange(cached, cached + new)
    slots = torch.cat([table[s].long().cpu()[pos // bs] * bs + pos % bs for s in range(S)]).to(dev)
    ctx_dev = torch.tensor(ctx, dtype=torch.int32, device=dev)
    qsl = torch.arange(0, S * new + 1, new, dtype=torch.int32, device=dev)
    out = torch.empty_like(q)
    scale = d ** -0.5

    def append():
        kernels.reshape_and_cache(kn, vn, k, v, slots)

    def attend():
        kernels.chunked_prefill(out, q, k, v, table, ctx_dev, qsl, new, scale=scale)

    for _ in range(args.warmup):
        append()
        attend()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        append()
        attend()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) / args.steps * 1e3
    stream = torch.cuda.current_stream(dev)
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(args.steps)]
    for e in ev:
        e[0].record(stream)
        append()
        e[1].record(stream)
        attend()
        e[2].record(stream)
    torch.cuda.synchronize()
    app_us, app_med = _event_us(ev, 0, 1)
    att_us, att_med = _event_us(ev, 1, 2)
    flops = 4 * d * hq * S * sum(cached + i + 1 for i in range(new))
    achieved = flops / (att_us * 1e-6) / 1e12
    return {
        "metric": "chunked-prefill MFMA TFLOP/s (causal-masked flops)",
        "value": flops / (ms * 1e-3) / 1e12,
        "unit": "TFLOP/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": ms,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic N(0,1), seeded",
        "config": {"workload": "chunked prefill: 8 seqs x (4096 cached + 512 new), 32 q / 8 kv "
                               "heads, head_dim 128, block 16, bf16, causal in chunk",
                   "flops_per_step": flops},
        "tokens_per_s": S * new / (ms * 1e-3),
        "kernels_us": {"reshape_and_cache": app_us, "chunked_prefill": att_us},
        "kernels_us_median": {"reshape_and_cache": app_med, "chunked_prefill": att_med},
        "roofline": {"bound": "mfma", "kernel": "chunked_prefill", "achieved": achieved,
                     "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": achieved / PEAK_BF16_TFLOPS, "traffic": None},
    }


def bench_copy(args):
    """Calibration workload: a plain device copy of a known number of bytes
    (2 GiB read + 2 GiB written per step), used to scale HBM byte counters."""
    import torch

    dev = torch.device("cuda", 0)
    n = 1 << 31
    src = torch.empty(n, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    for _ in range(args.warmup):
        dst.copy_(src)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        dst.copy_(src)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) / args.steps * 1e3
    return {"metric": "device copy GB/s (read + write)", "value": 2 * n / (ms * 1e-3) / 1e9,
            "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "ms_per_step": ms, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
            "dtype": "u8", "data": "constant bytes",
            "config": {"workload": "calibration copy, 2 GiB read + 2 GiB write per step",
                       "bytes_read_per_step": n, "bytes_written_per_step": n}}


def bench_node(args, dtype_name="bfloat16", packed=False):
    """The "gpu" AttentionNode backend end to end: one decode_layer_batch of
    the GQA Qwen2.5-7B shape batch (128 requests, 28 q / 4 kv heads, head_dim
    128, contexts U[256, 8192]) with the query/key/value rows on the host, as
    the node receives them; wall time per call, host work included. bf16, or
    fp32 (what the reference's CPU dense nodes send, src/core/nodes.py:21-24;
    the pools then default to fp32). packed: the same batch through
    decode_layer_packed, the payloads stacked as [128, heads, 128] host tensors."""
    import torch
    from cloverinfer_amd.attention_backend import GpuAttentionBackend

    cfg = DECODE_CONFIGS["qwen7b"]
    dev = torch.device("cuda", 0)
    ctx = context_lengths(cfg)
    S, hq, hkv, d, bs = cfg["num_seqs"], cfg["hq"], cfg["hkv"], cfg["d"], 16
    steps_total = args.warmup + args.steps
    nb = sum(math.ceil((c + steps_total + 1) / bs) for c in ctx) + 16
    be = GpuAttentionBackend(num_blocks=nb, block_size=bs, device="cuda")
    g = torch.Generator(device=dev).manual_seed(cfg["seed"])
    dt = getattr(torch, dtype_name)
    for i, c in enumerate(ctx):
        k = torch.randn((c, hkv, d), generator=g, device=dev).to(dt)
        v = torch.randn((c, hkv, d), generator=g, device=dev).to(dt)
        be.init_request(f"r{i}", [{"key": k, "value": v}], decode_reserve_tokens=steps_total + 1)
    gh = torch.Generator().manual_seed(cfg["seed"] + 1)
    items = [{"request_id": f"r{i}", "layer_idx": 0,
              "query": torch.randn((1, hq, d), generator=gh).to(dt),
              "key": torch.randn((1, hkv, d), generator=gh).to(dt),
              "value": torch.randn((1, hkv, d), generator=gh).to(dt),
              "score_scale": d ** -0.5} for i in range(S)]
    if packed:
        rids = [it["request_id"] for it in items]
        qkv = [torch.cat([it[n] for it in items]) for n in ("query", "key", "value")]

        def call():
            return be.decode_layer_packed(rids, 0, *qkv, d ** -0.5)
    else:
        def call():
            return be.decode_layer_batch(items)
    for _ in range(args.warmup):
        call()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        call()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) / args.steps * 1e3
    api = "decode_layer_packed" if packed else "decode_layer_batch"
    return {"metric": f"gpu AttentionNode backend: {api} wall time per layer",
            "value": ms, "unit": "ms", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "ms_per_step": ms, "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
            "dtype": {"bfloat16": "bf16", "float32": "f32"}[dtype_name],
            "data": "synthetic N(0,1), seeded; q/k/v rows on the host",
            "config": {"workload": f"{api} of 128 requests, GQA Qwen2.5-7B shape, "
                                   "contexts U[256,8192], one layer, host-side q/k/v"},
            "requests_per_s": S / (ms * 1e-3)}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    # The GPU clock ramps up over the first tens of milliseconds of a run:
    # 200 untimed steps (about 40 ms of decode) reach the steady clock.
    ap.add_argument("--steps", type=int, default=500)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--config", default="qwen7b",
                    choices=sorted(DECODE_CONFIGS) + ["qwen7b_fp8", "prefill", "copy", "node",
                                                      "node_fp32", "node_packed"])
    ap.add_argument("--partition", type=int, default=None,
                    help="split-K partition size (0 = single pass, -1 or default: automatic)")
    ap.add_argument("--waves", type=int, default=0,
                    help="waves of the balanced decode (0 = device default)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-budget", type=float, default=15.0,
                    help="seconds of CPU baseline work (a bounded sample)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}): the paged-attention "
              "kernels run on a single device and this build has no multi-GPU path.",
              file=sys.stderr)
        return 2
    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        return 1
    if args.config == "qwen7b_fp8":
        result = bench_decode_fp8(args)
    elif args.config == "prefill":
        result = bench_prefill(args)
    elif args.config == "copy":
        result = bench_copy(args)
    elif args.config == "node":
        result = bench_node(args)
    elif args.config == "node_fp32":
        result = bench_node(args, "float32")
    elif args.config == "node_packed":
        result = bench_node(args, packed=True)
    else:
        result = bench_decode(args, DECODE_CONFIGS[args.config])
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
