#!/usr/bin/env python3
"""Benchmark of the paged-attention hot path on one MI355X.

The default run measures all five workloads of the hot path, each on the
GPU and, for comparison, on the host cores:

  opt125m   paged decode, 8 seqs, 12 heads, head_dim 64, fp32, context 128,
            a step = 1-token append (reshape_and_cache) + decode
  llama7b   paged decode, 64 seqs, 32 heads, head_dim 128, fp16, context 2048
  long32k   split-K paged decode, 16 seqs, 32 q / 8 kv heads, fp16, context
            32768, partition 512 + the log-sum-exp reduce
  prefill   chunked prefill, 8 seqs x (4096 cached + 512 new), 32 q / 8 kv
            heads, bf16, a step = append of the 4096 new rows + causal prefill
  qwen7b    (headline) paged decode, 128 seqs, 28 q / 4 kv heads, head_dim
            128, bf16, context U[256, 8192] seeded per sequence

The JSON line's top-level fields are the headline (qwen7b): whole-job GB/s of
algorithmic bytes (K/V read once per kv head + q + out + block tables) per
step, tokens/s, a roofline entry for the decode kernel timed with HIP events
on the stream it runs on, and the CPU baseline (this repository's
restatement of the reference CpuAttentionBackend, timed on the host cores
over a bounded sample of the same batch). "configs" holds the same fields
for every workload. Inputs are resident in HBM before any timed region.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config all|NAME]
"""
from __future__ import annotations

import argparse
import glob
import hashlib
import json
import math
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
METRIC = "decode-attn HBM GB/s (% of ~8 TB/s peak) + tokens/sec at GQA-7B shape, 1 GPU"
PEAK_HBM_GBS = 8000.0        # MI355X HBM3E
PEAK_BF16_TFLOPS = 2500.0    # MI355X dense bf16/fp16 MFMA

DECODE_CONFIGS = {
    # name: shape, dtype, context spec, value scale, seed, schedule
    "opt125m": dict(num_seqs=8, hq=12, hkv=12, d=64, dtype="float32", ctx=("fixed", 128),
                    vscale=1.0, seed=1001, partition=None, append=True,
                    workload="paged decode, OPT-125m shape: 8 seqs, 12 heads, head_dim 64, "
                             "block 16, fp32, context 128; a step appends 1 token per sequence "
                             "(reshape_and_cache) and decodes"),
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
                             "block 16, fp16, context 32768, partition 512 + LSE reduce"),
}

# The default run: every workload, the headline last (earlier ones bring the
# GPU clock up); CPU baselines after all GPU measurements.
ALL = ["opt125m", "llama7b", "long32k", "prefill", "qwen7b"]
CPU_BUDGET_S = {"opt125m": 5.0, "llama7b": 8.0, "long32k": 8.0, "prefill": 10.0, "qwen7b": 10.0}

DTYPE_TAG = {"float32": "f32", "float16": "f16", "bfloat16": "bf16"}


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def sources_sha256() -> str:
    """Hash of the kernel sources and the C ABI: a traffic figure measured
    on other sources is stale."""
    h = hashlib.sha256()
    files = sorted(glob.glob(os.path.join(ROOT, "cloverinfer_amd", "csrc", "*")) +
                   glob.glob(os.path.join(ROOT, "include", "*.h")))
    for f in files:
        h.update(os.path.basename(f).encode())
        h.update(open(f, "rb").read())
    return h.hexdigest()


def traffic_for(name: str):
    """HBM bytes per launch of the workload's dominant kernel: calibrated
    FETCH_SIZE + WRITE_SIZE from profiles/traffic_<name>.json, or None when
    absent or measured on other kernel sources."""
    path = os.path.join(ROOT, "profiles", f"traffic_{name}.json")
    if not os.path.exists(path):
        return None, "not measured"
    rec = json.load(open(path))
    if rec.get("sources_sha256") != sources_sha256():
        return None, "stale: measured on other kernel sources"
    return rec.get("hbm_bytes_per_launch"), rec.get("measured")


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
                flops=4 * sum(ctx) * cfg["hq"] * cfg["d"], dtype=dtype, eb=eb,
                scale=cfg["d"] ** -0.5)


def _event_us(ev, a: int, b: int):
    """Mean and median, in microseconds, of the intervals between events a and
    b of every timed step (the mean is what the roofline divides by)."""
    d = sorted(e[a].elapsed_time(e[b]) * 1e3 for e in ev)
    n = len(d)
    med = d[n // 2] if n % 2 else 0.5 * (d[n // 2 - 1] + d[n // 2])
    return sum(d) / n, med


def time_steps(args, phases, solo=None):
    """After args.settle seconds of untimed steps (see below), run W untimed
    steps, then K steps timed by wall clock (synchronised on both sides), then
    K more steps with HIP events between the phases of each step. ``phases``: callables run in order as one step; each takes the step
    index. Returns (ms per step, [(mean us, median us) per phase])."""
    import torch

    def step(i):
        for ph in phases:
            ph(i)

    # GPU clock settle, untimed and before the warm-up: MI355X raises its
    # engine clock over the first tens of milliseconds of sustained work (the
    # prefill kernel took 496 us on its 5th call and 399 us on its 45th, same
    # inputs), and the workload set-up before each measurement leaves the GPU
    # idle. Steps run one at a time, synchronised, for args.settle seconds.
    t_end = time.perf_counter() + getattr(args, "settle", 0.0)
    while time.perf_counter() < t_end:
        step(0)
        torch.cuda.synchronize()
    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(args.warmup + i)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) / args.steps * 1e3
    # HIP events on the stream the kernels run on. A leading device-side
    # sleep keeps the GPU busy while every launch is queued, so host launch
    # gaps stay out of the event intervals; it is sized to the queueing time
    # (about 100K cycles, some 50 us, per step), since a long spin lets the
    # engine clock drop before the timed kernels run.
    stream = torch.cuda.current_stream()
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(len(phases) + 1)]
          for _ in range(args.steps)]
    torch.cuda._sleep(min(50_000_000, 100_000 * max(1, args.steps)))
    for i, e in enumerate(ev):
        e[0].record(stream)
        for j, ph in enumerate(phases):
            ph(args.warmup + args.steps + i)
            e[j + 1].record(stream)
    torch.cuda.synchronize()
    res = [_event_us(ev, j, j + 1) for j in range(len(phases))]
    if solo is None:
        return ms, res
    # Phase `solo` alone, K launches back to back between one pair of events:
    # for kernels of a few microseconds the per-launch event pairs above add
    # about 2 us each; this figure (which includes the gaps between launches)
    # does not.
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda._sleep(min(50_000_000, 100_000 * max(1, args.steps)))
    e0.record(stream)
    for i in range(args.steps):
        phases[solo](args.warmup + 2 * args.steps + i)
    e1.record(stream)
    torch.cuda.synchronize()
    return ms, res, e0.elapsed_time(e1) * 1e3 / max(1, args.steps)


def cpu_model() -> str:
    name = platform.processor() or "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return name


def cpu_threads() -> int:
    return len(os.sched_getaffinity(0))


def cpu_baseline_decode(host, budget_s: float):
    """The oracle's restatement of CpuAttentionBackend (fp32 upcast, grouped
    einsum, softmax, einsum, output cast to the query dtype) over the batch's
    sequences on the host cores: whole passes over the batch (one decode step
    per sequence) until the budget is spent, at least one sequence."""
    import torch
    from oracle import attention as oa

    threads = cpu_threads()
    torch.set_num_threads(threads)
    seqs = host["seqs"]
    eb = host["eb"]
    t0 = time.perf_counter()
    passes, done, nbytes = 0, 0, 0
    while True:
        for qi, kk, vv in seqs:
            oa.attend(qi, kk, vv, host["scale"]).to(host["dtype"])
            done += 1
            nbytes += kk.numel() * eb * 2 + qi.numel() * eb * 2
            if time.perf_counter() - t0 > budget_s:
                break
        else:
            passes += 1
            continue
        break
    dt = time.perf_counter() - t0
    # The sequences done above once more, each with the reference's
    # torch.cat append in front of its step (src/core/attention_backend.py:105-110).
    t1 = time.perf_counter()
    cat_bytes = 0
    for qi, kk, vv in seqs[:min(done, len(seqs))]:
        k2 = torch.cat([kk, kk[-1:]], dim=0)
        v2 = torch.cat([vv, vv[-1:]], dim=0)
        oa.attend(qi, k2, v2, host["scale"]).to(host["dtype"])
        cat_bytes += kk.numel() * eb * 2 + qi.numel() * eb * 2
    dt_cat = time.perf_counter() - t1
    return {
        "value": nbytes / dt / 1e9, "unit": "GB/s", "cores": threads, "kind": "port",
        "sample": f"{done} decode steps = {passes} whole passes over the {len(seqs)} sequences of "
                  f"the same batch + {done - passes * len(seqs)} more, one step per sequence "
                  f"(fp32 upcast + einsum + softmax + einsum, as CpuAttentionBackend.decode_layer)",
        "seconds": dt, "tokens_per_s": done / dt,
        "with_cat_append_gbs": cat_bytes / dt_cat / 1e9 if dt_cat > 0 else None,
        "cpu_model": cpu_model(),
    }


def cpu_baseline_prefill(host, budget_s: float):
    """Chunked prefill on the host cores, two ways over the same sequences:
    (1) successive append-then-attend decode steps (the oracle's
    CpuAttentionBackend restatement, one query token at a time, as the
    reference backend would serve a prompt), a bounded sample of tokens from
    the start of each sequence's chunk; (2) the equivalent causal-masked fp32
    contraction per kv head (one batched matmul form), whole sequences.
    Both in TFLOP/s of causal-masked flops (4 D Hq per visible key)."""
    import torch
    from oracle import attention as oa

    threads = cpu_threads()
    torch.set_num_threads(threads)
    q, ks, vs, n_new, scale = host["q"], host["keys"], host["values"], host["new"], host["scale"]
    hq, d = q.shape[2], q.shape[3]
    S = q.shape[0]
    # (1) successive decode steps: token i of every sequence in turn until
    # half the budget is spent.
    t0 = time.perf_counter()
    flops, tokens = 0, 0
    i = 0
    while i < n_new and time.perf_counter() - t0 < budget_s / 2:
        for s in range(S):
            lim = ks[s].shape[0] - n_new + i + 1
            oa.attend(q[s, i], ks[s][:lim], vs[s][:lim], scale).to(host["dtype"])
            flops += 4 * d * hq * lim
            tokens += 1
        i += 1
    dt_steps = time.perf_counter() - t0
    # (2) the causal-masked contraction, whole sequences until the budget.
    t1 = time.perf_counter()
    mflops, mseqs = 0, 0
    for s in range(S):
        oa.chunked_prefill_masked(q[s], ks[s], vs[s], scale).to(host["dtype"])
        L = ks[s].shape[0]
        mflops += 4 * d * hq * sum(L - n_new + j + 1 for j in range(n_new))
        mseqs += 1
        if time.perf_counter() - t1 > budget_s / 2:
            break
    dt_masked = time.perf_counter() - t1
    return {
        "value": flops / dt_steps / 1e12, "unit": "TFLOP/s", "cores": threads, "kind": "port",
        "sample": f"{tokens} query tokens ({i} per sequence, from the start of each of the {S} "
                  f"chunks) as successive append-then-attend decode steps (fp32 upcast + einsum "
                  f"+ softmax + einsum, as CpuAttentionBackend.decode_layer)",
        "seconds": dt_steps, "tokens_per_s": tokens / dt_steps,
        "masked_contraction": {"value": mflops / dt_masked / 1e12, "unit": "TFLOP/s",
                               "sample": f"{mseqs} whole sequences (512 query tokens each) as one "
                                         f"causal-masked fp32 contraction per kv head",
                               "seconds": dt_masked,
                               "tokens_per_s": mseqs * n_new / dt_masked},
        "cpu_model": cpu_model(),
    }


# How the roofline's kernel time is taken, for every workload: K launches of
# the dominant kernel alone, queued back to back on its stream between one
# pair of HIP events, total / K (time_steps' ``solo`` figure). It agrees with
# rocprofv3's per-dispatch average; per-launch event pairs add a launch gap
# to every launch and are reported beside it, never used for ``frac``.
ROOFLINE_TIMING = ("back-to-back mean: K launches of the kernel alone between one pair of HIP "
                   "events on its stream, total / K")


def roofline(bound: str, kernel: str, work: float, kernel_us: float, traffic, traffic_note):
    """``work``: algorithmic bytes (hbm) or flops (mfma) per launch;
    ``kernel_us``: the back-to-back mean launch time."""
    peak = PEAK_HBM_GBS if bound == "hbm" else PEAK_BF16_TFLOPS
    achieved = work / (kernel_us * 1e-6) / (1e9 if bound == "hbm" else 1e12)
    return {"bound": bound, "kernel": kernel, "achieved": achieved, "peak": peak,
            "unit": "GB/s" if bound == "hbm" else "TFLOP/s", "frac": achieved / peak,
            "kernel_us": kernel_us, "work_per_launch": work, "timing": ROOFLINE_TIMING,
            "traffic": traffic, "traffic_source": traffic_note}


# Parity bar of the attention outputs against the fp32 oracle, as in the
# tests: max-abs <= 2e-3 everywhere and max-rel <= 1e-2 where |ref| >= 0.2.
PARITY_ATOL, PARITY_RTOL, PARITY_REL_FLOOR = 2e-3, 1e-2, 0.2


def parity_record(got, ref, rows: int, what: str) -> dict:
    """Margins of a timed launch's output ``got`` against the oracle's
    ``ref`` (same shape, any float dtype) and whether they meet the bar."""
    import torch

    got = got.float()
    ref = ref.float()
    finite = bool(torch.isfinite(got).all())
    err = (got - ref).abs()
    big = ref.abs() >= PARITY_REL_FLOOR
    max_abs = float(err.max()) if err.numel() else 0.0
    max_rel = float((err[big] / ref.abs()[big]).max()) if bool(big.any()) else 0.0
    return {"what": what, "rows": rows, "elements": err.numel(), "max_abs": max_abs,
            "max_rel": max_rel, "rel_elements": int(big.sum()), "finite": finite,
            "bar": {"max_abs": PARITY_ATOL, "max_rel": PARITY_RTOL,
                    "rel_where_abs_ref_at_least": PARITY_REL_FLOOR},
            "within_bar": finite and max_abs <= PARITY_ATOL and max_rel <= PARITY_RTOL}


def decode_reference(host):
    """The oracle's fp32 decode output for every sequence of the batch."""
    import torch
    from oracle import attention as oa

    return torch.stack([oa.attend(qi, kk, vv, host["scale"]) for qi, kk, vv in host["seqs"]])


def parity_decode(host, what: str) -> dict:
    return parity_record(host["out"], decode_reference(host), len(host["seqs"]), what)


def prefill_reference(host):
    """The oracle's fp32 chunked-prefill output ``[S, new, Hq, D]`` (one
    causal-masked contraction per sequence)."""
    import torch
    from oracle import attention as oa

    return torch.stack([oa.chunked_prefill_masked(host["q"][s], host["keys"][s],
                                                  host["values"][s], host["scale"])
                        for s in range(host["q"].shape[0])])


def parity_prefill(host, what: str) -> dict:
    q = host["q"]
    return parity_record(host["out"], prefill_reference(host), q.shape[0] * q.shape[1], what)


def measure_decode(args, name):
    """One decode workload on the GPU: (entry, host data for the CPU baseline)."""
    import torch
    from cloverinfer_amd import kernels

    cfg = DECODE_CONFIGS[name]
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    log(f"{name}: building workload")
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
    waves = args.waves
    part = args.partition if args.partition is not None else cfg["partition"]
    if part is not None and part < 0:
        part = None
    if part is None:
        if waves > 0 and kernels.balanced_supported(a):
            mode, part = "balanced", 0
        else:
            mode, part = kernels.choose_schedule(a, kernels.num_compute_units(dev))
    else:
        mode = "split" if part > 0 and max_ctx > part else "single"
    stream = torch.cuda.current_stream(dev).cuda_stream
    lib = kernels._native.load()
    if mode == "balanced":
        ws = kernels.splitk_workspace(dev, kernels.balanced_workspace_bytes(a, waves))
    elif mode == "split":
        ws = kernels.splitk_workspace(dev, kernels.workspace_bytes(a, part))
    else:
        ws = None

    phases, names = [], []
    append_bytes = 0
    fused = None
    if cfg.get("append"):
        # The step's append: token ctx - 1 of every sequence (its new row)
        # through reshape_and_cache into the pool copy the step decodes.
        g = torch.Generator(device=dev).manual_seed(cfg["seed"] + 7)
        kn = torch.randn((len(w["ctx"]), cfg["hkv"], cfg["d"]), generator=g, device=dev).to(w["dtype"])
        vn = torch.randn((len(w["ctx"]), cfg["hkv"], cfg["d"]), generator=g, device=dev).to(w["dtype"])
        bs = w["bs"]
        slots = torch.tensor([int(w["table_host"][s, (c - 1) // bs]) * bs + (c - 1) % bs
                              for s, c in enumerate(w["ctx"])], dtype=torch.int64, device=dev)
        append_bytes = 2 * kn.numel() * kn.element_size() * 2 + slots.numel() * 8
        cache_list = [kernels.cache_args(kn, vn, kc, vc, slots) for kc, vc in pools]

        def append(i):
            kernels._native.check(lib.clv_reshape_and_cache(cache_list[i % copies], stream),
                                  "clv_reshape_and_cache")

        if mode == "single" and kernels.append_fusable(w["q"], w["k"], len(w["ctx"])):
            # The step as the backend runs it: one single-pass launch that
            # writes token ctx - 1 of every sequence and attends over it
            # (clv_paged_decode_append); the two-launch form (append kernel,
            # then decode) is timed beside it.
            fused = [kernels.AppendDecodeLaunch(out, w["q"], kc, vc, w["table"], w["ctx_dev"],
                                                w["bs"], max_ctx, kn, vn, scale=w["scale"])
                     for kc, vc in pools]
        else:
            phases.append(append)
            names.append("reshape_and_cache")

    def first_half(i):
        a = args_list[i % copies]
        if mode == "balanced":
            kernels.balanced_partials(a, waves, ws, stream)
        elif mode == "split":
            kernels.paged_decode_partials(a, part, ws, stream)
        else:
            kernels._native.check(lib.clv_paged_decode(a, stream), "clv_paged_decode")

    def second_half(i):
        a = args_list[i % copies]
        if mode == "balanced":
            kernels.balanced_reduce(a, waves, ws, stream)
        else:
            kernels.splitk_reduce(a, part, ws, stream)

    two_launch = None
    if fused is not None:
        log(f"{name}: two-launch form (reshape_and_cache, then the decode), {args.steps} steps")
        ms2, ev2 = time_steps(args, [append, first_half])
        two_launch = {"ms_per_step": ms2, "kernels_us": {"reshape_and_cache": ev2[0][0],
                                                         "paged_decode": ev2[1][0]}}
        calls = [f.bind() for f in fused]

        def fused_step(i):
            kernels._native.check(calls[i % copies](), "clv_paged_decode_append")

        phases.append(fused_step)
        names.append("paged_decode_append")
    else:
        phases.append(first_half)
        names.append("paged_decode")
        if mode != "single":
            phases.append(second_half)
            names.append("merge")
    log(f"{name}: warmup {args.warmup}, {args.steps} steps (schedule {mode}, partition "
        f"{part if mode == 'split' else 0}, {copies} pool copies)")
    dom = names.index("paged_decode_append" if fused is not None else "paged_decode")
    ms, ev, dec_batched = time_steps(args, phases, solo=dom)
    # Every step computes the same output from the same inputs (the pool
    # copies are equal, the append rewrites one row with the same data): the
    # last timed launch's output is what the parity leg checks.
    torch.cuda.synchronize()
    out_host = out.cpu()
    log(f"{name}: step {ms:.4f} ms, " + ", ".join(f"{n} {e[0]:.1f} us" for n, e in zip(names, ev)))
    step_bytes = w["algo_bytes"] + append_bytes
    kernel = {"balanced": "paged_decode_stream", "split": "paged_decode_stream (split-K partials)",
              "single": "paged_decode_mfma (single pass)"}[mode]
    kernel_bytes = w["algo_bytes"]
    if fused is not None:
        kernel, kernel_bytes = "paged_decode_mfma (single pass, fused append)", step_bytes
    traffic, note = traffic_for(name)
    entry = {
        "workload": cfg["workload"],
        "value": step_bytes / (ms * 1e-3) / 1e9, "unit": "GB/s",
        "ms_per_step": ms,
        "tokens_per_s": len(w["ctx"]) / (ms * 1e-3),
        "dtype": DTYPE_TAG[cfg["dtype"]],
        "num_seqs": len(w["ctx"]), "num_heads": cfg["hq"], "num_kv_heads": cfg["hkv"],
        "head_dim": cfg["d"], "block_size": w["bs"],
        "total_context_tokens": sum(w["ctx"]), "max_context_len": max_ctx,
        "schedule": mode, "partition_size": part if mode == "split" else 0,
        "kv_pool_copies": copies, "seed": cfg["seed"],
        "algorithmic_bytes_per_step": step_bytes,
        "decode_algorithmic_bytes": w["algo_bytes"],
        "kernels_us": {n: e[0] for n, e in zip(names, ev)},
        "kernels_us_median": {n: e[1] for n, e in zip(names, ev)},
        "kernel_us_back_to_back": {names[dom]: dec_batched},
        "roofline": roofline("hbm", kernel, kernel_bytes, dec_batched, traffic, note),
    }
    if two_launch is not None:
        entry["two_launch"] = two_launch
    # Host copies for the CPU baseline: each sequence's context gathered into
    # the reference backend's contiguous [L, Hkv, D] form (untimed setup).
    from oracle import attention as oa

    kc, vc, q = w["k"].cpu(), w["v"].cpu(), w["q"].cpu()
    seqs = []
    for i, c in enumerate(w["ctx"]):
        kk, vv = oa.gather_context(kc, vc, w["table_host"][i].tolist(), c)
        seqs.append((q[i], kk.contiguous(), vv.contiguous()))
    host = {"seqs": seqs, "eb": w["eb"], "dtype": w["dtype"], "scale": w["scale"],
            "out": out_host}
    del pools, args_list, w
    torch.cuda.empty_cache()
    return entry, host


def measure_prefill(args):
    """Chunked prefill, 8 sequences x (4096 cached + 512 new), 32 q / 8 kv
    heads, head_dim 128, bf16: a step appends the 512 new K/V rows of every
    sequence (reshape_and_cache) and runs the causal chunk attention."""
    import torch
    from cloverinfer_amd import kernels

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    S, cached, new, hq, hkv, d, bs = 8, 4096, 512, 32, 8, 128, 16
    seed = 1005
    log("prefill: building workload")
    ctx = [cached + new] * S
    need = [math.ceil(c / bs) for c in ctx]
    nb = sum(need)
    g = torch.Generator().manual_seed(seed)
    perm = torch.randperm(nb, generator=g)
    table_host = perm.view(S, -1).to(torch.int32)
    table = table_host.to(dev)
    gd = torch.Generator(device=dev).manual_seed(seed)
    k = torch.randn((nb, bs, hkv, d), generator=gd, device=dev).to(torch.bfloat16)
    v = torch.randn((nb, bs, hkv, d), generator=gd, device=dev).to(torch.bfloat16)
    q = torch.randn((S * new, hq, d), generator=gd, device=dev).to(torch.bfloat16)
    kn = torch.randn((S * new, hkv, d), generator=gd, device=dev).to(torch.bfloat16)
    vn = torch.randn((S * new, hkv, d), generator=gd, device=dev).to(torch.bfloat16)
    pos = torch.arange(cached, cached + new)
    slots = torch.cat([table_host[s].long()[pos // bs] * bs + pos % bs for s in range(S)]).to(dev)
    ctx_dev = torch.tensor(ctx, dtype=torch.int32, device=dev)
    qsl = torch.arange(0, S * new + 1, new, dtype=torch.int32, device=dev)
    out = torch.empty_like(q)
    scale = d ** -0.5

    lib = kernels._native.load()
    stream = torch.cuda.current_stream(dev).cuda_stream
    ca = kernels.cache_args(kn, vn, k, v, slots)

    def append(i):
        kernels._native.check(lib.clv_reshape_and_cache(ca, stream), "clv_reshape_and_cache")

    def attend(i):
        kernels.chunked_prefill(out, q, k, v, table, ctx_dev, qsl, new, scale=scale)

    log(f"prefill: warmup {args.warmup}, {args.steps} steps")
    ms, ev, att_batched = time_steps(args, [append, attend], solo=1)
    (app_us, app_med), (att_us, att_med) = ev
    torch.cuda.synchronize()
    out_host = out.cpu().view(S, new, hq, d)
    log(f"prefill: step {ms:.4f} ms, append {app_us:.1f} us, prefill {att_us:.1f} us")
    flops = 4 * d * hq * S * sum(cached + i + 1 for i in range(new))
    traffic, note = traffic_for("prefill")
    entry = {
        "workload": "chunked prefill: 8 seqs x (4096 cached + 512 new), 32 q / 8 kv heads, "
                    "head_dim 128, block 16, bf16, causal in chunk; a step appends the 4096 new "
                    "K/V rows (reshape_and_cache) and runs the prefill",
        "value": flops / (ms * 1e-3) / 1e12, "unit": "TFLOP/s",
        "ms_per_step": ms,
        "tokens_per_s": S * new / (ms * 1e-3),
        "dtype": "bf16", "seed": seed,
        "flops_per_step": flops,
        "kernels_us": {"reshape_and_cache": app_us, "chunked_prefill": att_us},
        "kernels_us_median": {"reshape_and_cache": app_med, "chunked_prefill": att_med},
        "kernel_us_back_to_back": {"chunked_prefill": att_batched},
        "roofline": roofline("mfma", "chunked_prefill_mfma", flops, att_batched, traffic, note),
    }
    # Host copies for the CPU baseline: each sequence's whole context in the
    # reference backend's contiguous form, the query rows per sequence.
    from oracle import attention as oa

    kc, vc = k.cpu(), v.cpu()
    keys, values = [], []
    for s in range(S):
        kk, vv = oa.gather_context(kc, vc, table_host[s].tolist(), ctx[s])
        keys.append(kk.contiguous())
        values.append(vv.contiguous())
    host = {"q": q.cpu().view(S, new, hq, d), "keys": keys, "values": values, "new": new,
            "scale": scale, "dtype": torch.bfloat16, "out": out_host}
    del k, v, q, kn, vn, out
    torch.cuda.empty_cache()
    return entry, host


def bench_all(args, names):
    measured = {}
    for name in names:
        if name == "prefill":
            measured[name] = measure_prefill(args)
        else:
            measured[name] = measure_decode(args, name)
    if not args.no_cpu:
        for name in names:
            log(f"{name}: cpu baseline")
            entry, host = measured[name]
            budget = args.cpu_budget if args.cpu_budget > 0 else CPU_BUDGET_S.get(name, 10.0)
            if name == "prefill":
                entry["cpu_baseline"] = cpu_baseline_prefill(host, budget)
            else:
                entry["cpu_baseline"] = cpu_baseline_decode(host, budget)
    for name in names:
        entry, host = measured[name]
        log(f"{name}: parity of the timed launch's output against the oracle")
        what = f"{name}: last timed launch, every row"
        entry["parity"] = (parity_prefill(host, what) if name == "prefill"
                           else parity_decode(host, what))
        p = entry["parity"]
        log(f"{name}: parity max-abs {p['max_abs']:.3e}, max-rel {p['max_rel']:.3e} over "
            f"{p['rows']} rows: {'within' if p['within_bar'] else 'OUTSIDE'} the bar")
    return {n: measured[n][0] for n in names}


def result_line(args, entries, head: str):
    """The contract's JSON object: the headline workload's fields at the top,
    every measured workload under "configs"."""
    e = entries[head]
    is_prefill = head == "prefill"
    metric = ("chunked-prefill MFMA TFLOP/s (causal-masked flops)" if is_prefill else
              METRIC if head == "qwen7b" else f"decode-attn HBM GB/s, {head} workload, 1 GPU")
    res = {
        "metric": metric,
        "value": e["value"], "unit": e["unit"], "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": e["ms_per_step"],
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": e["dtype"],
        "data": "synthetic N(0,1) q/K/V (x0.5 for the Llama-7B shape), random init, seeded; "
                "no model weights",
        "config": {k: v for k, v in e.items()
                   if k not in ("value", "unit", "ms_per_step", "dtype", "kernels_us",
                                "kernels_us_median", "kernel_us_back_to_back", "roofline",
                                "cpu_baseline", "tokens_per_s")},
        "tokens_per_s": e["tokens_per_s"],
        "kernels_us": e["kernels_us"],
        "kernels_us_median": e["kernels_us_median"],
        "kernel_us_back_to_back": e["kernel_us_back_to_back"],
        "roofline": e["roofline"],
    }
    if not is_prefill:
        res["hbm_frac_of_peak"] = e["value"] / PEAK_HBM_GBS
    if "cpu_baseline" in e:
        res["cpu_baseline"] = e["cpu_baseline"]
    if "parity" in e:
        res["parity"] = e["parity"]
    if len(entries) > 1:
        res["configs"] = entries
    res["gpu_clock_settle_s"] = args.settle
    res["sources_sha256"] = sources_sha256()[:16]
    return res


def bench_decode_fp8(args):
    """The GQA Qwen2.5-7B decode batch with fp8 (OCP e4m3) pools: K/V are
    the same seeded N(0,1) data stored as e4m3 with scale 1 per kv head; q
    and out stay bf16. A step is one clv_paged_decode_fp8 call (stream decode
    + merge), issued as its two halves (clv_paged_decode_fp8_partials, then
    clv_balanced_reduce) so that the roofline times the decode kernel alone."""
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

    # clv_paged_decode_fp8 is the fp8 stream kernel then the merge; issued as
    # its two halves so that each is timed on its own.
    def partials(i):
        kernels._native.check(lib.clv_paged_decode_fp8_partials(
            a, ones.data_ptr(), ones.data_ptr(), waves, ws.data_ptr(), ws.numel(),
            stream.cuda_stream), "clv_paged_decode_fp8_partials")

    def merge(i):
        kernels._native.check(lib.clv_balanced_reduce(a, waves, ws.data_ptr(), ws.numel(),
                                                      stream.cuda_stream), "clv_balanced_reduce")

    ms, ev, dec_batched = time_steps(args, [partials, merge], solo=0)
    call_us, call_med = ev[0]
    torch.cuda.synchronize()
    out_host = out.cpu()
    ctx = w["ctx"]
    kv_bytes = sum(ctx) * cfg["hkv"] * cfg["d"] * 1 * 2
    qo_bytes = len(ctx) * cfg["hq"] * cfg["d"] * 2 * 2
    tbl_bytes = sum(math.ceil(c / w["bs"]) for c in ctx) * 4 + len(ctx) * 4
    algo = kv_bytes + qo_bytes + tbl_bytes
    merge_us, merge_med = ev[1]
    log(f"step {ms:.4f} ms, decode {call_us:.1f} us, merge {merge_us:.1f} us")
    traffic, note = traffic_for("qwen7b_fp8")
    # Parity of the last timed launch: the oracle over the dequantised pools
    # (scale 1: each code's e4m3 value), every sequence.
    from oracle import attention as oa

    log("qwen7b_fp8: parity of the timed launch's output against the oracle")
    kc, vc, q = k8.cpu().float(), v8.cpu().float(), w["q"].cpu()
    seqs = []
    for i, c in enumerate(ctx):
        kk, vv = oa.gather_context(kc, vc, w["table_host"][i].tolist(), c)
        seqs.append((q[i], kk, vv))
    parity = parity_decode({"seqs": seqs, "scale": w["scale"], "out": out_host},
                           "qwen7b_fp8: last timed launch, every row")
    log(f"qwen7b_fp8: parity max-abs {parity['max_abs']:.3e}: "
        f"{'within' if parity['within_bar'] else 'OUTSIDE'} the bar")
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
        "kernels_us": {"paged_decode": call_us, "merge": merge_us},
        "kernels_us_median": {"paged_decode": call_med, "merge": merge_med},
        "kernel_us_back_to_back": {"paged_decode": dec_batched},
        "roofline": roofline("hbm", "paged_decode_stream (fp8)", algo, dec_batched, traffic, note),
        "parity": parity,
    }


def bench_copy(args):
    """Calibration workload: a plain device copy of a known number of bytes
    (``--copy-mib`` MiB read + the same written per step), used to scale HBM
    byte counters."""
    import torch

    dev = torch.device("cuda", 0)
    n = args.copy_mib << 20
    src = torch.empty(n, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    ms, _ = time_steps(args, [lambda i: dst.copy_(src)])
    return {"metric": "device copy GB/s (read + write)", "value": 2 * n / (ms * 1e-3) / 1e9,
            "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "ms_per_step": ms, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
            "dtype": "u8", "data": "constant bytes",
            "config": {"workload": f"calibration copy, {args.copy_mib} MiB read + "
                                   f"{args.copy_mib} MiB written per step",
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
    # The GPU clock ramps up over the first tens of milliseconds of a run.
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--config", default="all",
                    choices=["all"] + sorted(DECODE_CONFIGS) +
                            ["qwen7b_fp8", "prefill", "copy", "node", "node_fp32", "node_packed"])
    ap.add_argument("--partition", type=int, default=None,
                    help="split-K partition size (0 = single pass, -1 or default: automatic)")
    ap.add_argument("--waves", type=int, default=0,
                    help="waves of the balanced decode (0 = device default)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--settle", type=float, default=0.2,
                    help="seconds of untimed, synchronised steps before each workload's "
                         "warm-up, so that the GPU clock has ramped up (0: none)")
    ap.add_argument("--cpu-budget", type=float, default=0.0,
                    help="seconds of CPU baseline work per workload (0: the built-in "
                         "per-workload budgets, 5-10 s)")
    ap.add_argument("--copy-mib", type=int, default=2048, help="size of the calibration copy")
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
    if args.config == "all":
        result = result_line(args, bench_all(args, ALL), "qwen7b")
        # The fp8-pool batch and the "gpu" AttentionNode backend's calls ride
        # along under "configs" (a failure there is recorded, not raised). A
        # node call is a fraction of a millisecond of wall time, noisy over a
        # few calls: those time at least 200 (after at least 50 warm-up).
        node_args = argparse.Namespace(**{**vars(args), "steps": max(args.steps, 200),
                                          "warmup": max(args.warmup, 50)})
        for name, fn, a in (("qwen7b_fp8", bench_decode_fp8, args),
                            ("node", bench_node, node_args),
                            ("node_packed", lambda a: bench_node(a, packed=True), node_args),
                            ("node_fp32", lambda a: bench_node(a, "float32"), node_args)):
            log(f"{name}")
            try:
                result["configs"][name] = fn(a)
            except Exception as exc:  # noqa: BLE001 - reported in the JSON line
                result["configs"][name] = {"error": f"{type(exc).__name__}: {exc}"}
    elif args.config in DECODE_CONFIGS or args.config == "prefill":
        result = result_line(args, bench_all(args, [args.config]), args.config)
    elif args.config == "qwen7b_fp8":
        result = bench_decode_fp8(args)
    elif args.config == "copy":
        result = bench_copy(args)
    elif args.config == "node":
        result = bench_node(args)
    elif args.config == "node_fp32":
        result = bench_node(args, "float32")
    else:
        result = bench_node(args, packed=True)
    print(json.dumps(result), flush=True)
    # A timed launch whose output is outside the parity bar fails the run.
    bad = [n for n, e in (result.get("configs") or {"": result}).items()
           if "parity" in e and not e["parity"]["within_bar"]]
    if bad:
        print(f"bench.py: output outside the parity bar for {', '.join(bad) or result['metric']}",
              file=sys.stderr)
        return 3
    return 0


if __name__ == "__main__":
    sys.exit(main())
