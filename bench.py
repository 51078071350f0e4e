#!/usr/bin/env python3
"""PKM lookup-path benchmark on one MI355X.

Default workload ("layer"): one product-key memory layer, forward + backward,
bf16, through the drop-in module (modelos_amd.pkm.memory.HashingMemory):
x [8, 2048, 1024] (16384 tokens), 8 heads x 1024 keys per half (2^20 value
slots), k_dim 512, knn 32, value dim 1024, RMSNorm query, swilu projection,
random init (reset_parameters), N(0,1) input and upstream gradient. One step =
forward + backward (gradients of x and every parameter; no optimizer step).

"--workload eb": the standalone weighted embedding bag, forward + backward,
bf16: 16384 bags x 128 lookups into a 2^20 x 1024 table, softmax per-sample
weights, N(0,1) upstream gradient (drop-in xformers_embedding_bag).

Prints one JSON line: whole-job tokens/s (K steps timed with nothing but the
work on the stream), the roofline of the dominant HIP kernel (algorithmic
bytes or flops / its HIP-event time, from a second, instrumented pass of the
same K steps), every entry point's time (same pass), and the reference's CPU
path (op-for-op torch CPU restatement: einsum/topk/F.embedding_bag + ATen
autograd) timed on this host's cores on a bounded sample of the same workload.

The default run also reports, under extra keys, the standalone embedding bag
("eb_standalone"), the fast-weight PKM layer in float32 and bfloat16
("fwpkm"), the CPU parity configuration's forward ("cpu_parity_config"),
each with its CPU baseline, the layer step after a 512 MB cache flush
("cache_flush"), the large-memory stress shape (2^22 slots, 16 GiB table,
Zipf-skewed lookups; "stress") and a Qwen3-0.6B-shaped decoder train step
with two PKM layers (3 steps; "model_step"). "--workload model" / "stress"
time those alone.

Usage: python bench.py [--gpus 1] [--steps 10] [--warmup 3]
                       [--workload layer|eb|fwupdate|fwpkm|model|stress] [--no-cpu-baseline] [--no-extras]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, 8 TB/s
MFMA_BF16_PEAK_TFLOPS = 2516.6  # MI355X dense bf16 MFMA
METRIC = "PKM layer fwd+bwd tokens/sec at 1M slots bf16; embedding-bag HBM GB/s vs peak"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def eb_algorithmic_bytes(B, L, K, D, U, s_w=2, s_p=2, s_g=2):
    """Algorithmic HBM bytes of one embedding-bag forward / backward.
    fwd: every lookup reads its row (N*D*s_w), index + weight (N*(8+s_p)),
         output write (B*D*s_w).
    bwd: upstream grad once (B*D*s_g), each distinct row once (U*D*s_w),
         dense weight-gradient write (K*D*s_w), index + weight (N*(8+s_p)),
         weight-gradient write (N*s_p)."""
    N = B * L
    fwd = N * D * s_w + N * (8 + s_p) + B * D * s_w
    bwd = B * D * s_g + U * D * s_w + K * D * s_w + N * (8 + s_p) + N * s_p
    return fwd, bwd


def eb_rows_algorithmic_bytes(B, L, K, D, U, s_w=2, s_g=2):
    """Algorithmic HBM bytes of the backward's row-reduction kernel (after the
    sort): each distinct row of W once (U*D*s_w), the dense weight-gradient
    write (K*D*s_w), the upstream gradient once (B*D*s_g), 8 bytes of sorted
    occurrence metadata per lookup (N*8), the row offsets ((K+1)*4) and the
    float32 psw-gradients in sorted order (N*4)."""
    N = B * L
    return U * D * s_w + K * D * s_w + B * D * s_g + N * 8 + (K + 1) * 4 + N * 4


def score_flops(tokens, heads, n_keys, k_dim):
    """Sub-key scoring: 2 * tokens * heads * 2 halves * n_keys * k_dim/2."""
    return 2 * tokens * heads * 2 * n_keys * (k_dim // 2)


def cpu_model():
    """The host CPU's model name as lscpu prints it (/proc/cpuinfo if lscpu is absent)."""
    import subprocess

    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        fields = {}
        for line in out.splitlines():
            if ":" in line:
                k, v = line.split(":", 1)
                fields.setdefault(k.strip(), v.strip())
        name = fields.get("Model name")
        if name:
            if not any(ch.isdigit() for ch in name):
                # a generic name (virtualised hosts): add lscpu's family / model / stepping numbers
                ids = ", ".join(f"{k.lower()} {fields[k]}" for k in ("CPU family", "Model", "Stepping") if k in fields)
                name = f"{name} ({ids})" if ids else name
            return name
    except (OSError, subprocess.SubprocessError):
        pass
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def load_traffic():
    """HBM bytes per launch measured with rocprofv3 --pmc (FETCH_SIZE,
    WRITE_SIZE, scaled by a copy-kernel calibration), committed under
    profiles/ (not measured in this run: the counters need a profiler run of
    their own); each entry is returned with the tree it was profiled on."""
    p = ROOT / "profiles" / "hbm_traffic.json"
    if not p.exists():
        return {}
    try:
        d = json.loads(p.read_text())
    except ValueError:
        return {}
    when = d.get("_profiled_at", "see profiles/hbm_traffic.md")
    return {k: {"bytes": v, "source": "profiles/hbm_traffic.json", "profiled_at": when}
            for k, v in d.items() if not k.startswith("_")}


BAR_HBM = 0.60  # graded fraction of HBM peak for the embedding-bag kernels
BAR_MFMA = 0.50  # graded fraction of bf16 MFMA peak for the sub-key scoring


def graded_rooflines(kernels, bars, traffic_prefix=""):
    """One roofline entry per graded kernel that was timed: achieved / peak on
    its algorithmic work, its bar and frac / bar, with the calibrated HBM
    traffic per launch where profiles/hbm_traffic.json holds it (and the tree
    it was profiled on)."""
    traffic = load_traffic()
    out = []
    for name, bar in bars.items():
        v = kernels.get(name)
        if v is None or "frac" not in v:
            continue
        t = traffic.get(traffic_prefix + name)
        out.append({
            "kernel": name, "bound": v["bound"], "ms": v["ms"], "achieved": v["achieved"], "peak": v["peak"],
            "unit": v["unit"], "frac": v["frac"], "bar": bar, "frac_of_bar": round(v["frac"] / bar, 4),
            "traffic": t["bytes"] if t else None, "traffic_profiled_at": t["profiled_at"] if t else None,
        })
    return out


def headline_roofline(rooflines):
    """The graded kernel furthest below its bar (smallest frac / bar), so the
    headline names the bottleneck rather than whichever kernel took longest
    in this run."""
    if not rooflines:
        return None
    r = dict(min(rooflines, key=lambda e: e["frac_of_bar"]))
    r["selected_as"] = "graded kernel furthest below its bar (every graded kernel is listed under rooflines)"
    return r


def timed_steps(step, steps, kernel_timer=True):
    """Times `steps` calls of `step` with nothing else on the stream (the
    headline: wall clock between two synchronizations, and the median of
    per-step event pairs), then runs the same number of steps again with the
    library's call timer (event pair around every entry point) and, when
    asked, its kernel timer (event pairs around single kernels inside entry
    points) for the per-kernel breakdown. The instrumented pass is not part of
    the headline: its event records add host work to every call.
    Returns (wall ms per step, median event ms, call records, kernel timer)."""
    import torch

    from modelos_amd import _lib

    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        ev[i][0].record()
        step()
        ev[i][1].record()
    torch.cuda.synchronize()
    ms_per_step = (time.perf_counter() - t0) * 1e3 / steps
    step_ms = sorted(a.elapsed_time(b) for a, b in ev)[steps // 2]

    timer = _lib.CallTimer()
    ktimer = _lib.KernelTimer()
    if kernel_timer:
        ktimer.__enter__()
    try:
        with timer:
            for _ in range(steps):
                step()
        torch.cuda.synchronize()
    finally:
        if kernel_timer:
            ktimer.__exit__(None, None, None)
    return ms_per_step, step_ms, timer.summary(), ktimer


def timed_median(fn, budget_s=25.0, max_repeats=3):
    """1 warm-up, then up to max_repeats timed calls within the budget; median seconds."""
    t0 = time.perf_counter()
    fn()
    warm = time.perf_counter() - t0
    reps = max(1, min(max_repeats, int(budget_s / max(warm, 1e-3)) - 1))
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    times.sort()
    return times[len(times) // 2], reps


# ---------------------------------------------------------------------------
# PKM layer
# ---------------------------------------------------------------------------
LAYER = dict(B=8, T=2048, C=1024, H=8, n=1024, k=512, knn=32, D=1024)


def cpu_baseline_layer(mem, x, dout, budget_s=25.0):
    """The reference's CPU path (pkm/memory.py:190-289 ops: Linear + RMSNorm,
    einsum, topk, cartesian topk, softmax, F.embedding_bag, swilu, ATen
    autograd) on the same bf16 parameters, on a bounded token sample."""
    import torch

    from oracle import pkm_layer

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    P = {n: p.detach().cpu().requires_grad_(True) for n, p in mem.named_parameters()}
    H, knn = mem.heads, mem.knn
    xc_all, gc_all = x.detach().cpu(), dout.cpu()

    def make_step(tokens):
        xs = xc_all.reshape(-1, xc_all.shape[-1])[:tokens].reshape(1, tokens, -1).clone().requires_grad_(True)
        gs = gc_all.reshape(-1, gc_all.shape[-1])[:tokens].reshape(1, tokens, -1)

        def step():
            out, _ = pkm_layer.hashing_memory_forward(xs, P, H, knn, reference_ops=True)
            out.backward(gs)
            for p in P.values():
                p.grad = None
            xs.grad = None

        return step

    total = xc_all.shape[0] * xc_all.shape[1]
    probe = min(2048, total)
    t_probe, _ = timed_median(make_step(probe), budget_s=1e9, max_repeats=1)
    tokens = probe
    while tokens * 2 <= total and t_probe * (tokens * 2 / probe) * 4 <= budget_s:
        tokens *= 2
    t, reps = timed_median(make_step(tokens), budget_s=budget_s)
    return {
        "value": round(tokens / t, 1),
        "unit": "tokens/s",
        "cores": cores,
        "kind": "port",
        "sample": f"{tokens} of the {total} tokens (same bf16 parameters and inputs), full 2^20 x 1024 value "
        f"table, fwd+bwd; median of {reps} after 1 warm-up; torch CPU ops of the reference's path on {cores} "
        f"threads ({cpu_model()})",
        "ms_per_step": round(t * 1e3, 1),
    }


def run_layer(args, dev):
    import torch

    from modelos_amd import _lib
    from modelos_amd.pkm.memory import HashingMemory

    c = LAYER
    B, T, C, H, n, k, knn, D = c["B"], c["T"], c["C"], c["H"], c["n"], c["k"], c["knn"], c["D"]
    tokens = B * T
    torch.manual_seed(0)
    with torch.device(dev):
        mem = HashingMemory(input_dim=C, output_dim=D, mem_k_dim=k, mem_heads=H, mem_knn=knn, mem_n_keys=n)
        mem.reset_parameters()
    mem = mem.to(torch.bfloat16).train()
    gen = torch.Generator(device=dev).manual_seed(0)
    x = torch.randn((B, T, C), generator=gen, device=dev).to(torch.bfloat16).requires_grad_(True)
    dout = torch.randn((B, T, D), generator=gen, device=dev).to(torch.bfloat16)
    log(f"layer ready: tokens={tokens} heads={H} n_keys={n} (slots {n * n}) k_dim={k} knn={knn} v_dim={D}")

    def step():
        mem.zero_grad(set_to_none=True)
        x.grad = None
        out, idx = mem(x)
        out.backward(dout)
        return idx

    for i in range(args.warmup):
        idx = step()
    torch.cuda.synchronize()
    U = int(torch.unique(idx).numel())
    log(f"warmup done ({args.warmup} steps); distinct value rows U={U}")

    # headline steps bare, then the same number instrumented (per-call and
    # single-kernel event pairs) for the breakdown
    ms_per_step, step_ms, calls, ktimer = timed_steps(step, args.steps)
    for kname in ktimer.KERNELS:
        if ktimer.ms(kname):
            calls[("kernel", kname)] = ktimer.ms(kname)
    log(f"timed {args.steps} steps: {ms_per_step:.3f} ms/step (median event time {step_ms:.3f} ms)")

    L = H * knn
    a_fwd, a_bwd = eb_algorithmic_bytes(tokens, L, n * n, D, U)

    def med(key):
        v = sorted(calls.get(key, []))
        return v[len(v) // 2] if v else None

    kernels = {}

    def add(name, key, work, unit, peak, bound, note=None):
        ms = med(key)
        if ms is None:
            return
        rate = work / (ms * 1e-3) / (1e12 if unit == "TFLOP/s" else 1e9)
        kernels[name] = {
            "ms": round(ms, 4), "calls_per_step": len(calls[key]) // args.steps,
            "work": work, "achieved": round(rate, 2), "unit": unit, "peak": peak,
            "frac": round(rate / peak, 4), "bound": bound,
        }
        if note:
            kernels[name]["note"] = note

    add("pkm_score_stream_kernel (scoring + per-half top-k)", ("kernel", "score_topk"), score_flops(tokens, H, n, k),
        "TFLOP/s", MFMA_BF16_PEAK_TFLOPS, "mfma")
    add("pkm_score_topk", ("pkm_score_topk", (tokens, H, n, k // 2)), score_flops(tokens, H, n, k), "TFLOP/s",
        MFMA_BF16_PEAK_TFLOPS, "mfma", "entry point: scoring + per-half top-k kernel, then the cartesian kernel")
    add("pkm_eb_fwd (values)", ("pkm_eb_fwd", (n * n, D)), a_fwd, "GB/s", HBM_PEAK_GBS, "hbm")
    add("value backward row reduction (eb_bwd_rows_dyn_kernel + eb_bwd_long_rows_kernel)", ("kernel", "eb_bwd_rows"),
        eb_rows_algorithmic_bytes(tokens, L, n * n, D, U), "GB/s", HBM_PEAK_GBS, "hbm")
    add("pkm_eb_bwd (values)", ("pkm_eb_bwd", (n * n, D)), a_bwd, "GB/s", HBM_PEAK_GBS, "hbm",
        "entry point: sort + row reduction + psw-gradient scatter (several kernels)")

    def add_ms(name, entry, note):
        """Every call of one entry point, whatever its sizes."""
        keys = [kk for kk in calls if kk[0] == entry]
        if keys:
            per_step = sum(len(calls[kk]) for kk in keys) / args.steps
            ms = sum(med(kk) * len(calls[kk]) for kk in keys) / args.steps / per_step
            kernels[name] = {"ms": round(ms, 4), "calls_per_step": round(per_step), "note": note}

    add_ms("pkm_score_grad_sparse (score backward)", "pkm_score_grad_sparse",
           "nonzero lists + fused dq gather, dK on MFMA + ordered split reduction (several kernels)")
    add_ms("pkm_rmsnorm_fwd (query)", "pkm_rmsnorm_fwd", "query RMSNorm forward")
    add_ms("pkm_rmsnorm_bwd (query)", "pkm_rmsnorm_bwd", "query RMSNorm backward + ordered weight-gradient reduction")
    add_ms("pkm_swilu_fwd (value gate)", "pkm_swilu_fwd", "e * silu(s) of the value output")
    add_ms("pkm_swilu_bwd (value gate)", "pkm_swilu_bwd", "gradients of the value gate")
    add_ms("pkm_column_sum (Linear bias gradients, split-K sums)", "pkm_column_sum",
           "per call; per Linear one bias gradient and one sum of the weight gradient's split-K partials")
    add_ms("pkm_softmax_fwd (scores)", "pkm_softmax_fwd", "softmax of the selected scores")
    add_ms("pkm_softmax_bwd (scores)", "pkm_softmax_bwd", "its gradient")
    # single kernels timed inside an entry point are part of that entry's time
    inner = ("pkm_score_stream_kernel (scoring + per-half top-k)", "value backward row reduction (eb_bwd_rows_dyn_kernel + eb_bwd_long_rows_kernel)")
    for kk in inner:
        if kk in kernels:
            kernels[kk]["part_of"] = "pkm_score_topk" if kk.startswith("pkm_score") else "pkm_eb_bwd (values)"
    hip_ms = sum(v["ms"] * v["calls_per_step"] for kk, v in kernels.items() if kk not in inner)
    kernels["other (query/swilu/value GEMMs, glue)"] = {"ms": round(step_ms - hip_ms, 4)}

    rooflines = graded_rooflines(kernels, {
        "pkm_eb_fwd (values)": BAR_HBM,
        "value backward row reduction (eb_bwd_rows_dyn_kernel + eb_bwd_long_rows_kernel)": BAR_HBM,
        "pkm_eb_bwd (values)": BAR_HBM,
        "pkm_score_stream_kernel (scoring + per-half top-k)": BAR_MFMA,
    })
    roofline = headline_roofline(rooflines)

    # the same step with a 512 MB write between steps (caches hold none of the previous step's data)
    flush = torch.empty(512 << 20, dtype=torch.uint8, device=dev)
    fl_ms = []
    for i in range(args.steps):
        flush.fill_(i & 0xFF)
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        step()
        b.record()
        fl_ms.append((a, b))
    torch.cuda.synchronize()
    flushed_ms = sorted(a.elapsed_time(b) for a, b in fl_ms)[args.steps // 2]
    del flush
    log(f"with a 512 MB cache flush between steps: {flushed_ms:.3f} ms/step (median event time)")

    cpu = None
    if not args.no_cpu_baseline:
        log("timing the CPU baseline ...")
        cpu = cpu_baseline_layer(mem, x, dout)
        log(f"cpu baseline: {cpu['value']} tokens/s ({cpu['sample']})")

    return {
        "metric": METRIC,
        "value": round(tokens / (ms_per_step * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (N(0,1) input and upstream gradient, reset_parameters init)",
        "config": {
            "workload": "PKM layer fwd+bwd (HashingMemory: RMSNorm query, swilu projection), 2^20 value slots",
            "tokens": tokens, "batch": B, "seq_len": T, "input_dim": C, "heads": H, "n_keys": n,
            "k_dim": k, "knn": knn, "v_dim": D, "distinct_rows": U,
        },
        "roofline": roofline,
        "rooflines": rooflines,
        "kernels": kernels,
        "cache_flush": {"ms_per_step": round(flushed_ms, 4), "ms_per_step_no_flush": round(step_ms, 4),
                        "note": "median HIP-event time of a step run right after a 512 MB write; "
                                "ms_per_step_no_flush: the same median for back-to-back steps"},
        "layer_floor": layer_floor(tokens, H, n, k, knn, C, D, U, ms_per_step),
        "cpu_baseline": cpu,
    }


def layer_floor(tokens, H, n, k, knn, C, D, U, ms_per_step):
    """The layer step's lower bound from its algorithmic work at MI355X peaks:
    the value gather and the value backward at HBM bandwidth (algorithmic
    bytes as in the roofline), the sub-key scoring and the dense projections
    (query C -> H k, swilu gate C -> D, output D -> C; forward and two
    backward products each) at the bf16 MFMA peak. frac = floor / measured."""
    L = H * knn
    a_fwd, a_bwd = eb_algorithmic_bytes(tokens, L, n * n, D, U)
    proj_flops = 3 * 2 * tokens * (C * H * k + C * D + D * C)
    parts_ms = {
        "values_fwd": a_fwd / (HBM_PEAK_GBS * 1e9) * 1e3,
        "values_bwd": a_bwd / (HBM_PEAK_GBS * 1e9) * 1e3,
        "scoring": score_flops(tokens, H, n, k) / (MFMA_BF16_PEAK_TFLOPS * 1e12) * 1e3,
        "projections": proj_flops / (MFMA_BF16_PEAK_TFLOPS * 1e12) * 1e3,
    }
    floor_ms = sum(parts_ms.values())
    return {
        "ms": round(floor_ms, 4), "tokens_per_s": round(tokens / (floor_ms * 1e-3), 1),
        "frac": round(floor_ms / ms_per_step, 4), "parts_ms": {kk: round(v, 4) for kk, v in parts_ms.items()},
        "note": "value gather and backward at 8 TB/s (algorithmic bytes), scoring and projection GEMMs "
                "(fwd + 2 bwd products) at 2516.6 TFLOP/s bf16; frac = floor / measured ms_per_step",
    }


# ---------------------------------------------------------------------------
# Standalone embedding bag
# ---------------------------------------------------------------------------
def cpu_baseline_eb(W, idx, p, g, budget_s=25.0):
    """The reference's CPU path on the same inputs: F.embedding_bag + autograd
    (pkm/xformer_embeddingbag.py:436-437)."""
    import torch

    from oracle import eb as ref

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    Wc = W.detach().cpu().requires_grad_(True)
    pc = p.detach().cpu().requires_grad_(True)
    ic, gc = idx.cpu(), g.cpu()

    def step():
        out = ref.eb_forward_library(ic, Wc, pc)
        out.backward(gc)
        Wc.grad = None
        pc.grad = None

    t, reps = timed_median(step, budget_s=budget_s)
    return {
        "value": round(idx.shape[0] / t, 1),
        "unit": "tokens/s",
        "cores": cores,
        "kind": "port",
        "sample": f"full step ({idx.shape[0]} bags x {idx.shape[1]}, 2^20 x 1024 bf16 table), "
        f"median of {reps} after 1 warm-up; F.embedding_bag + ATen autograd on {cores} threads ({cpu_model()})",
        "ms_per_step": round(t * 1e3, 1),
    }


def run_eb(args, dev):
    import torch

    from modelos_amd import _lib
    from modelos_amd.pkm.xformer_embeddingbag import xformers_embedding_bag

    B, L, K, D = 16384, 128, 1 << 20, 1024
    gen = torch.Generator(device=dev).manual_seed(0)
    W = (torch.randn((K, D), generator=gen, device=dev) * 0.03).to(torch.bfloat16).requires_grad_(True)
    idx = torch.randint(0, K, (B, L), generator=gen, device=dev)
    p = torch.softmax(torch.randn((B, L), generator=gen, device=dev), -1).to(torch.bfloat16).requires_grad_(True)
    g = torch.randn((B, D), generator=gen, device=dev).to(torch.bfloat16)
    U = int(torch.unique(idx).numel())
    log(f"inputs ready: B={B} L={L} K={K} D={D} distinct rows U={U}")

    def step():
        W.grad = None
        p.grad = None
        out = xformers_embedding_bag(idx, W, p)
        out.backward(g)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    ms_per_step, _, calls, ktimer = timed_steps(step, args.steps)
    calls["rows"] = ktimer.ms("eb_bwd_rows")  # the row-reduction kernel inside the backward entry point

    def med(key):
        v = sorted(calls[key])
        return v[len(v) // 2]

    fwd_ms, bwd_ms, rows_ms = med(("pkm_eb_fwd", (K, D))), med(("pkm_eb_bwd", (K, D))), med("rows")
    log(f"timed {args.steps} steps: {ms_per_step:.3f} ms/step (fwd {fwd_ms:.3f} ms, bwd {bwd_ms:.3f} ms, "
        f"row kernel {rows_ms:.3f} ms)")
    a_fwd, a_bwd = eb_algorithmic_bytes(B, L, K, D, U)
    kernels = {
        "pkm_eb_fwd (values)": {"ms": round(fwd_ms, 4), "work": a_fwd},
        "value backward row reduction (eb_bwd_rows_dyn_kernel + eb_bwd_long_rows_kernel)": {
            "ms": round(rows_ms, 4), "work": eb_rows_algorithmic_bytes(B, L, K, D, U),
            "part_of": "pkm_eb_bwd (values)"},
        "pkm_eb_bwd (values)": {"ms": round(bwd_ms, 4), "work": a_bwd,
                                "note": "entry point: sort + row reduction + psw-gradient scatter (several kernels)"},
    }
    for v in kernels.values():
        v["achieved"] = round(v["work"] / (v["ms"] * 1e-3) / 1e9, 2)
        v["unit"], v["peak"], v["bound"] = "GB/s", HBM_PEAK_GBS, "hbm"
        v["frac"] = round(v["achieved"] / HBM_PEAK_GBS, 4)
    rooflines = graded_rooflines(kernels, {kk: BAR_HBM for kk in kernels}, traffic_prefix="eb:")
    roofline = headline_roofline(rooflines)
    cpu = None
    if not args.no_cpu_baseline:
        log("timing the CPU baseline ...")
        cpu = cpu_baseline_eb(W, idx, p, g)
    return {
        "metric": "standalone embedding-bag fwd+bwd bags/sec, bf16, 2^20 x 1024 table",
        "value": round(B / (ms_per_step * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "standalone weighted embedding-bag fwd+bwd (drop-in xformers_embedding_bag)",
            "bags": B, "bag_size": L, "num_rows": K, "dim": D, "distinct_rows": U,
        },
        "roofline": roofline,
        "rooflines": rooflines,
        "kernels": kernels,
        "cpu_baseline": cpu,
    }


def run_fwupdate(args, dev):
    """Fast-weight value update (FwPKM update_fw, values, sgd): 2^18 x 512 float32
    table (4 heads x 512 keys per half), 8192 tokens x 64 lookups, lr 0.1."""
    import torch

    from modelos_amd import _lib
    from modelos_amd.fwpkm.fwpkm import sgd_value_update
    from oracle import fw_update as ref

    K, D, N, L = 1 << 18, 512, 8192, 4 * 16
    scale, lr = N * D * 16 * 4, 0.1
    gen = torch.Generator(device=dev).manual_seed(0)
    p = (torch.randn((K, D), generator=gen, device=dev) * D**-0.5).float()
    g = torch.randn((K, D), generator=gen, device=dev) * 1e-6
    idx = torch.randint(0, K, (N, L), generator=gen, device=dev)

    def step():
        return sgd_value_update(p, g, idx, scale, lr, 0.0, False)

    def torch_step():
        return ref.sgd_value_update(p, g, idx, scale, lr, 0.0, False)

    for _ in range(args.warmup):
        step()
        torch_step()
    torch.cuda.synchronize()
    ms_per_step, _, calls, _ = timed_steps(step, args.steps, kernel_timer=False)
    t1 = time.perf_counter()
    for _ in range(args.steps):
        torch_step()
    torch.cuda.synchronize()
    torch_ms = (time.perf_counter() - t1) * 1e3 / args.steps
    v = sorted(next(c for k, c in calls.items() if k[0] == "pkm_fw_sgd_update"))
    kern_ms = v[len(v) // 2]
    work = 4 * K * D * 4 + K * 8  # read values and gradient, write both outputs; the counts
    achieved = work / (kern_ms * 1e-3) / 1e9
    log(f"timed {args.steps} steps: {ms_per_step:.3f} ms/step (kernel {kern_ms:.3f} ms), "
        f"reference op sequence on the GPU {torch_ms:.3f} ms")
    cpu = None
    if not args.no_cpu_baseline:
        log("timing the CPU baseline ...")
        pc, gc, ic = p.cpu(), g.cpu(), idx.cpu()
        t, reps = timed_median(lambda: ref.sgd_value_update(pc, gc, ic, scale, lr, 0.0, False), budget_s=10.0)
        cores = torch.get_num_threads()
        cpu = {"value": round(K / t, 1), "unit": "rows/s", "cores": cores, "kind": "port",
               "sample": f"full update ({K} x {D} float32), median of {reps} after 1 warm-up; the reference's "
               f"ATen op sequence on {cores} threads ({cpu_model()})", "ms_per_step": round(t * 1e3, 1)}
    return {
        "metric": "FwPKM fast-weight value update (bincount-normalised SGD) table rows/sec, float32",
        "value": round(K / (ms_per_step * 1e-3), 1),
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "FwPKM update_fw values step (scale, bincount division, sgd) in one pass",
                   "num_rows": K, "dim": D, "tokens": N, "lookups_per_token": L},
        "roofline": {"bound": "hbm", "kernel": "pkm_fw_sgd_update", "achieved": round(achieved, 2),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": None},
        "kernels": {"pkm_fw_sgd_update": {"ms": round(kern_ms, 4), "work": work},
                    "reference op sequence (torch, same GPU)": {"ms": round(torch_ms, 4)}},
        "cpu_baseline": cpu,
    }


FWPKM = dict(mem_k_dim=256, mem_v_dim=1024, mem_heads=4, mem_topk=16, mem_n_subkeys=512, lookahead=0,
             qk_score_type="idw", learning_rate=0.1, addr_loss="me")


MFMA_F32_PEAK_TFLOPS = 157.3  # MI355X fp32 matrix


def fwpkm_rooflines(kern, dtype_bytes, distinct_rows, bags=4096, bag_size=64, K=1 << 18, D=1024, H=4, n=512,
                    k_dim=256, chunks=2, clip=False, wd=0.0):
    """Per-call algorithmic work of the fast-weight step's library kernels,
    achieved / peak from their measured per-step times, and the step's floor
    (every library call at its roofline, the torch glue at zero: a lower
    bound). Per chunk: bags = 8 sequences x 512 tokens, bag_size = heads x
    knn lookups into K x D; psw in the table dtype.
      pkm_eb_fwd (gather):     N*D*s + N*(8 + s) + B*D*s
      pkm_eb_bwd (outer):      B*D*s + U*D*s + K*D*s + N*(8 + s) + N*s
      pkm_eb_bwd_sgd (step):   every table row read and the new one written
                               (2*K*D*s), B*D*s + N*(8 + s), 8*K; the scaled
                               gradient (K*D*s) for every step but the last
                               only under grad_clip or weight decay (the only
                               cases whose backward reads it again)
      pkm_eb_bwd2_sgd:         the double backward's A_bwd2, N*D*s + 2*B*D*s
                               + N*(8 + 2*s), plus N*D*s of scaled-gradient
                               rows under grad_clip
      pkm_eb_bwd_accumulate:   as pkm_eb_bwd, the table gradient's touched
                               rows read and written (2*U*D*s) instead of
                               every row written
      pkm_me_grad_fwd:         the sub-score matrices read twice (2 * 2*R*n*s,
                               R = tokens x heads), the <q, k> products read
                               and the coefficient rows written (2 * 2H*T*n*4)
      pkm_me_grad_hvp:         the sub-scores read twice and their gradient
                               written (3 * 2*R*n*s), <q, k> and <q, gbar>
                               read twice (4 * 2H*T*n*4), [U | lam] rows
                               written (2H*T*2n*4)
      pkm_idw_grad_coef:       the dense sub-score gradient read (2H*T*n*s),
                               <q, k> read and U written (2 * 2H*T*n*4)
      pkm_score_topk:          2 * tokens * heads * 2 * n * k_dim/2 flops on
                               the matrix peak of the dtype"""
    s = dtype_bytes
    N, B = bags * bag_size, bags
    U = distinct_rows
    T, R = bags, bags * H  # tokens per chunk, sub-score rows per half
    dense = 2 * H * T * n  # entries of a [2 heads, tokens, n] operand
    per_call = {
        "pkm_eb_fwd": N * D * s + N * (8 + s) + B * D * s,
        "pkm_eb_bwd": B * D * s + U * D * s + K * D * s + N * (8 + s) + N * s,
        "pkm_eb_bwd_accumulate": B * D * s + U * D * s + 2 * U * D * s + N * (8 + s) + N * s,
        "pkm_eb_bwd2_sgd": N * D * s * (2 if clip else 1) + 2 * B * D * s + N * (8 + 2 * s),
        "pkm_me_grad_fwd": 2 * 2 * R * n * s + 2 * dense * 4,
        "pkm_me_grad_hvp": 3 * 2 * R * n * s + 4 * dense * 4 + 2 * dense * 4,
        "pkm_idw_grad_coef": dense * s + 2 * dense * 4,
    }
    sgd_total = chunks * (2 * K * D * s + B * D * s + N * (8 + s) + 8 * K) + (chunks - 1) * K * D * s * (
        1 if (clip or wd) else 0)
    flops = score_flops(bags, H, n, k_dim)
    peak_tf = MFMA_F32_PEAK_TFLOPS if s == 4 else MFMA_BF16_PEAK_TFLOPS
    out, floor = {}, 0.0
    for name, v in kern.items():
        calls, ms = v["calls_per_step"], v["ms_per_step"]
        if name in per_call:
            work, unit, peak = per_call[name] * calls, "GB/s", HBM_PEAK_GBS
        elif name == "pkm_eb_bwd_sgd":
            work, unit, peak = sgd_total, "GB/s", HBM_PEAK_GBS
        elif name == "pkm_score_topk":
            work, unit, peak = flops * calls, "TFLOP/s", peak_tf
        else:
            continue
        achieved = work / (ms * 1e-3) / (1e9 if unit == "GB/s" else 1e12)
        floor += work / (peak * (1e9 if unit == "GB/s" else 1e12)) * 1e3
        out[name] = {"ms_per_step": ms, "work_per_step": work, "achieved": round(achieved, 2), "unit": unit,
                     "peak": peak, "frac": round(achieved / peak, 4)}
    return out, floor


def cpu_baseline_fwpkm(mem, x, target, budget_s=25.0):
    """The reference's fast-weight chain as torch CPU ops (oracle.fwpkm, pinned
    to the reference's own outputs): one sequence of 1024 tokens (two chunks
    of 512, the second reading the updated table), full 2^18 x 1024 float32
    table, outer backward."""
    import torch

    from oracle import fwpkm as ofw

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    cfg = ofw.FwConfig.from_module_kwargs(dict(FWPKM, fp32_fw=True))
    k0 = mem.keys.detach().float().cpu()
    v0 = mem.values.detach().float().cpu()
    xs, ts = x[:1].float().cpu(), target[:1].float().cpu()

    def step():
        keys, values = k0.clone().requires_grad_(True), v0.clone().requires_grad_(True)
        q = xs.clone().requires_grad_(True)
        out = ofw.forward_wo_past(q, ts, keys, values, cfg, 512)
        torch.nn.functional.mse_loss(out["output"][:, 512:], ts[:, 512:]).backward()

    t, reps = timed_median(step, budget_s=budget_s, max_repeats=2)
    return {"value": round(1024 / t, 1), "unit": "tokens/s", "cores": cores, "kind": "port",
            "sample": f"1 of the 8 sequences (1024 tokens, 2 chunks), full 2^18 x 1024 float32 table, inner update "
            f"+ outer backward; median of {reps} after 1 warm-up; torch CPU ops of the reference's chain "
            f"(oracle.fwpkm) on {cores} threads ({cpu_model()})", "ms_per_step": round(t * 1e3, 1)}


def run_fwpkm(args, dev, with_cpu=None):
    """Fast-weight PKM layer step (the drop-in FastWeightProductKeyMemory):
    x [8, 1024, 1024] as queries (4 heads x 256), targets ~ N(0,1), 512 keys
    per half (2^18 slots), knn 16, value dim 1024, chunks of 512 (the second
    chunk reads the table after one inner SGD step, lr 0.1, "me" address loss),
    outer loss the MSE of the second chunk's output: forward with the inner
    update, then the outer backward through it (the embedding bag's
    grad-of-grad). float32 (fp32_fw) and bfloat16 (fp32_fw off)."""
    import torch

    from modelos_amd import _lib
    from modelos_amd.fwpkm.fwpkm import FastWeightProductKeyMemory

    with_cpu = (not args.no_cpu_baseline) if with_cpu is None else with_cpu
    results = {}
    gen = torch.Generator(device=dev).manual_seed(0)
    x32 = torch.randn((8, 1024, 1024), generator=gen, device=dev)
    t32 = torch.randn((8, 1024, 1024), generator=gen, device=dev)
    for dtype in (torch.float32, torch.bfloat16):
        torch.manual_seed(0)
        mem = FastWeightProductKeyMemory(**FWPKM, fp32_fw=dtype == torch.float32).to(dev)
        mem.reset_parameters()
        mem = mem.to(dtype).train()
        x, target = x32.to(dtype), t32.to(dtype)

        def step():
            mem.zero_grad(set_to_none=True)
            xx = x.detach().requires_grad_(True)
            out = mem(q=xx, ref_v=target, gates=None, chunk_size=512)
            torch.nn.functional.mse_loss(out["output"][:, 512:].float(), target[:, 512:].float()).backward()

        for _ in range(args.warmup):
            step()
        torch.cuda.synchronize()
        ms, _, calls, _ = timed_steps(step, args.steps, kernel_timer=False)
        kern = {}
        for name in sorted({k[0] for k in calls}):  # every library entry point the step called
            keys = [k for k in calls if k[0] == name]
            kern[name] = {"ms_per_step": round(sum(sum(calls[k]) for k in keys) / args.steps, 4),
                          "calls_per_step": sum(len(calls[k]) for k in keys) // args.steps}
        lib_ms = sum(v["ms_per_step"] for v in kern.values())
        tag = "f32" if dtype == torch.float32 else "bf16"
        log(f"fwpkm {tag}: {ms:.3f} ms/step, library entry points {lib_ms:.3f} ms")
        # distinct rows per chunk (the outer value backward reads each once), from one more forward
        with torch.no_grad():
            idx = mem(q=x, ref_v=target, gates=None, chunk_size=512)["indices"]
        U = sum(int(torch.unique(idx[:, c:c + 512]).numel()) for c in (0, 512)) // 2
        roof, floor_ms = fwpkm_rooflines(kern, 4 if dtype == torch.float32 else 2, U)
        results[tag] = {"ms_per_step": round(ms, 4), "tokens_per_s": round(8192 / (ms * 1e-3), 1), "kernels": kern,
                        "library_ms_per_step": round(lib_ms, 4),
                        "library_frac": round(lib_ms / ms, 4),
                        "rooflines": roof,
                        "distinct_rows_per_chunk": U,
                        "floor": {"ms": round(floor_ms, 4), "frac": round(floor_ms / ms, 4),
                                  "note": "every library call at its roofline (HBM 8 TB/s on algorithmic bytes, "
                                          "scoring at the dtype's matrix peak), the torch glue at zero"},
                        "note": "library_ms_per_step: HIP-event time of every libpkm_hip entry point per step "
                                "(instrumented pass); the rest is the module's torch glue (losses, transforms, "
                                "autograd bookkeeping) and hipBLASLt products"}
        if with_cpu and dtype == torch.float32:
            log("timing the fast-weight CPU baseline ...")
            results["cpu_baseline"] = cpu_baseline_fwpkm(mem, x, target)
        del mem
    return {
        "workload": "fast-weight PKM step (FastWeightProductKeyMemory.forward_wo_past, 2 chunks of 512 per "
                    "sequence, inner update + outer backward), 8 x 1024 tokens, 4 heads x 512 keys/half, knn 16, "
                    "v_dim 1024, idw scores, lr 0.1",
        **results,
    }


def run_fwpkm_workload(args, dev):
    r = run_fwpkm(args, dev)
    f32 = r["f32"]
    return {
        "metric": "FwPKM layer step (inner update + outer backward) tokens/sec, float32",
        "value": f32["tokens_per_s"], "unit": "tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": f32["ms_per_step"], "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic (N(0,1) queries and targets, reset_parameters init)",
        "config": {"workload": r["workload"], "tokens": 8192},
        "fwpkm": r, "cpu_baseline": r.get("cpu_baseline"),
    }


def cpu_parity_config(args, dev, budget_s=20.0):
    """The CPU parity configuration: one PKM layer forward, float32, x [4, 512,
    1024], 4 heads x 256 keys per half (65,536 slots), k_dim 512, knn 32, value
    dim 1024, BatchNorm query: the reference's op sequence on the CPU
    (oracle.pkm_layer, reference_ops) and the drop-in module on the GPU."""
    import torch

    from modelos_amd.pkm.memory import HashingMemory
    from oracle import pkm_layer

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    torch.manual_seed(0)
    mem = HashingMemory(input_dim=1024, output_dim=1024, mem_k_dim=512, mem_heads=4, mem_knn=32, mem_n_keys=256,
                        mem_query_batchnorm=True, mem_query_rmsnorm=False)
    mem.reset_parameters()
    g = torch.Generator().manual_seed(0)
    with torch.no_grad():
        mem.keys.copy_((torch.rand(mem.keys.shape, generator=g) * 2 - 1) / 16)
        mem.values.weight.copy_(torch.randn(mem.values.weight.shape, generator=g) * 1024**-0.5)
    x = torch.randn((4, 512, 1024), generator=g)
    P = {n: p.detach() for n, p in mem.named_parameters()}

    def cpu_step():
        with torch.no_grad():
            pkm_layer.hashing_memory_forward(x, P, 4, 32, batchnorm=True, reference_ops=True)

    t_cpu, reps = timed_median(cpu_step, budget_s=budget_s)
    memd = mem.to(dev).train()
    xd = x.to(dev)
    with torch.no_grad():
        for _ in range(3):
            memd(xd)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            memd(xd)
        torch.cuda.synchronize()
    t_gpu = (time.perf_counter() - t0) / args.steps
    return {
        "workload": "PKM layer forward, float32, x [4, 512, 1024], 4 heads x 256 keys/half, k_dim 512, knn 32, "
                    "v_dim 1024, BatchNorm query",
        "gpu_ms": round(t_gpu * 1e3, 4), "gpu_tokens_per_s": round(2048 / t_gpu, 1),
        "cpu_baseline": {"value": round(2048 / t_cpu, 1), "unit": "tokens/s", "cores": cores, "kind": "port",
                         "sample": f"the whole forward (2048 tokens), median of {reps} after 1 warm-up; torch CPU "
                         f"ops of the reference's path on {cores} threads ({cpu_model()})",
                         "ms_per_step": round(t_cpu * 1e3, 1)},
    }


# ---------------------------------------------------------------------------
# Large-memory stress: 4,194,304 slots, 16 GiB bf16 value table, Zipf-skewed lookups
# ---------------------------------------------------------------------------
STRESS = dict(B=4, T=4096, C=2048, H=16, n=2048, k=512, knn=64, D=2048)


def run_stress(args, dev, steps=3, warmup=1):
    """HashingMemory fwd+bwd at the large-memory stress shape: x [4, 4096,
    2048] ~ N(0,1), 16 heads, 2048 keys per half (2^22 slots), k_dim 512,
    knn 64, value dim 2048 (16 GiB bf16 table), RMSNorm query, bf16. The
    sub-key scores carry a Zipf(1.1) pre-bias realised through the module's
    own parameters: in every (head, half) one query coordinate has a zero
    weight row and bias 1, and the matching key coordinate is
    -1.1 * ln(rank + 1) * 0.5 over a seeded permutation of the sub-keys, so a
    few value rows collect thousands of lookups (the backward's heavy-row
    path). Reported: step time, the gather's rate on per-lookup and on
    distinct-row bytes, the value backward's rate, the scoring's MFMA rate and
    the lookup skew. Not graded against the bars (a contention stress)."""
    import math

    import torch

    from modelos_amd import _lib
    from modelos_amd.pkm.memory import HashingMemory

    c = STRESS
    B, T, C, H, n, k, knn, D = c["B"], c["T"], c["C"], c["H"], c["n"], c["k"], c["knn"], c["D"]
    tokens, half = B * T, k // 2
    torch.manual_seed(0)
    with torch.device(dev):
        mem = HashingMemory(input_dim=C, output_dim=C, mem_k_dim=k, mem_v_dim=D, mem_heads=H, mem_knn=knn,
                            mem_n_keys=n, mem_share_values=False, mem_query_rmsnorm=True)
        mem.reset_parameters()
    gen = torch.Generator(device=dev).manual_seed(5)
    with torch.no_grad():
        lin = mem.query_proj.query_mlps[0]
        cols = torch.tensor([h * k + cc * half for h in range(H) for cc in range(2)], device=dev)
        lin.weight[cols] = 0.0
        lin.bias.zero_()
        lin.bias[cols] = 1.0
        rank = torch.argsort(torch.rand((2 * H, n), generator=gen, device=dev), dim=1).float()
        mem.keys.view(2 * H, n, half)[:, :, 0] = -1.1 * torch.log(rank + 1.0) * 0.5
    mem = mem.to(torch.bfloat16).train()
    x = torch.randn((B, T, C), generator=gen, device=dev).to(torch.bfloat16).requires_grad_(True)
    dout = torch.randn((B, T, C), generator=gen, device=dev).to(torch.bfloat16)
    log(f"stress ready: tokens={tokens} heads={H} n_keys={n} (slots {n * n}) knn={knn} v_dim={D}")

    def step():
        mem.zero_grad(set_to_none=True)
        x.grad = None
        out, idx = mem(x)
        out.backward(dout)
        return idx

    for _ in range(warmup):
        idx = step()
    torch.cuda.synchronize()
    flat = idx.reshape(-1)
    counts = torch.bincount(flat, minlength=n * n)
    U, top = int((counts > 0).sum()), int(counts.max())
    heavy = int((counts > 256).sum())
    # rows of at least max(257, bags / 16) lookups: the value backward's matrix-core products
    hot_min = max(257, tokens // 16)
    hot_rows = int((counts >= hot_min).sum())
    hot_lookups = int(counts[counts >= hot_min].sum())
    del flat, counts
    ms_per_step, step_ms, calls, ktimer = timed_steps(step, steps)

    def med(key):
        v = sorted(calls.get(key, []))
        return v[len(v) // 2] if v else None

    L = H * knn
    N = tokens * L
    a_fwd, a_bwd = eb_algorithmic_bytes(tokens, L, n * n, D, U)
    a_fwd_u = U * D * 2 + N * (8 + 2) + tokens * D * 2  # each distinct row once
    fwd_ms, bwd_ms = med(("pkm_eb_fwd", (n * n, D))), med(("pkm_eb_bwd", (n * n, D)))
    sc_ms = med(("pkm_score_topk", (tokens, H, n, half)))
    rows = ktimer.ms("eb_bwd_rows")
    rows_ms = sorted(rows)[len(rows) // 2] if rows else None
    hot = ktimer.ms("eb_bwd_hot")
    hot_ms = sorted(hot)[len(hot) // 2] if hot else None
    hot_flops = 2 * 2 * hot_rows * tokens * D  # C G and W_hot G^T, dense
    log(f"stress: {ms_per_step:.3f} ms/step; gather {fwd_ms:.3f} ms, value backward {bwd_ms:.3f} ms "
        f"(hot-row products {hot_ms if hot_ms is None else round(hot_ms, 3)} ms for {hot_rows} rows), "
        f"scoring {sc_ms:.3f} ms; U={U}, hottest row {top} lookups, {heavy} rows over 256")

    def rate(work, ms, peak):
        if ms is None:
            return None
        r = work / (ms * 1e-3) / (1e12 if peak == MFMA_BF16_PEAK_TFLOPS else 1e9)
        return {"ms": round(ms, 4), "achieved": round(r, 2), "frac": round(r / peak, 4)}

    return {
        "metric": "large-memory stress: PKM layer fwd+bwd tokens/sec, 2^22 slots, 16 GiB bf16 table, Zipf lookups",
        "value": round(tokens / (ms_per_step * 1e-3), 1), "unit": "tokens/s", "ms_per_step": round(ms_per_step, 4),
        "steps": steps, "warmup": warmup, "dtype": "bf16",
        "data": "synthetic (N(0,1) input and upstream gradient; Zipf(1.1) pre-bias through a reserved query "
                "coordinate and a log-rank key coordinate per (head, half))",
        "config": {"workload": "HashingMemory fwd+bwd (RMSNorm query, swilu), 16 GiB bf16 value table",
                   "tokens": tokens, "batch": B, "seq_len": T, "input_dim": C, "heads": H, "n_keys": n,
                   "k_dim": k, "knn": knn, "v_dim": D},
        "lookups": {"total": N, "distinct_rows": U, "hottest_row": top, "rows_over_256": heavy},
        "gather_per_lookup": dict(rate(a_fwd, fwd_ms, HBM_PEAK_GBS) or {}, unit="GB/s", work=a_fwd,
                                  note="every lookup reads its row (N*D*2 + N*10 + B*D*2 bytes)"),
        "gather_distinct_rows": dict(rate(a_fwd_u, fwd_ms, HBM_PEAK_GBS) or {}, unit="GB/s", work=a_fwd_u,
                                     note="each distinct row once (U*D*2 + N*10 + B*D*2): the HBM floor "
                                          "when the hot rows are served from the caches"),
        "value_backward": dict(rate(a_bwd, bwd_ms, HBM_PEAK_GBS) or {}, unit="GB/s", work=a_bwd,
                               row_reduction_ms=round(rows_ms, 4) if rows_ms else None,
                               note="entry point: sort, heavy-row chunk partials, row reduction, scatter"),
        "hot_rows": dict(rate(hot_flops, hot_ms, MFMA_BF16_PEAK_TFLOPS) or {}, unit="TFLOP/s", work=hot_flops,
                         rows=hot_rows, lookups=hot_lookups, threshold=hot_min,
                         note="value backward's hot rows (at least max(257, bags/16) lookups) as two dense bf16 "
                              "products, C G (table gradient) and W_hot G^T (psw-gradients): operand copies, "
                              "products and split sums, one event pair"),
        "scoring": dict(rate(score_flops(tokens, H, n, k), sc_ms, MFMA_BF16_PEAK_TFLOPS) or {}, unit="TFLOP/s",
                        work=score_flops(tokens, H, n, k),
                        note="entry point (scoring + per-half top-64 tile kernel, cartesian top-64)"),
        "cpu_baseline": None,
        "cpu_baseline_note": "not timed: the 16 GiB table and 268 M lookups per step are beyond the bounded "
                             "CPU sample; the CPU comparison is the layer benchmark's",
    }


# ---------------------------------------------------------------------------
# Model step: a Qwen3-0.6B-shaped decoder with PKM layers
# ---------------------------------------------------------------------------
def run_model(args, dev):
    """A Qwen3-0.6B-shaped decoder (hidden 1024, 28 layers, 16 query / 8 KV
    heads, head_dim 128, MLP 3072, vocab 151936; transformers' Qwen3 modules,
    random init) whose layers 8 and 20 replace the MLP with the drop-in
    HashingMemory (8 heads, 1024 keys per half, knn 32, value dim 1024, as
    modeling_qwen3pkm.py:319-329 and :700-707 wire it): one train step
    (forward, causal-LM loss, backward) on 8 x 2048 uniform token ids, bf16."""
    import torch
    from torch import nn
    from transformers import Qwen3Config, Qwen3ForCausalLM

    from modelos_amd.pkm.memory import HashingMemory

    class PkmBlock(nn.Module):
        """The decoder layer's feed-forward slot: hidden_states, _ = self.pkm(hidden_states)."""

        def __init__(self, mem):
            super().__init__()
            self.pkm = mem

        def forward(self, h):
            out, _ = self.pkm(h)
            return out

    cfg = Qwen3Config(hidden_size=1024, num_hidden_layers=28, num_attention_heads=16, num_key_value_heads=8,
                      head_dim=128, intermediate_size=3072, vocab_size=151936, max_position_embeddings=4096,
                      tie_word_embeddings=True, attn_implementation="sdpa")
    torch.manual_seed(0)
    with torch.device(dev):
        model = Qwen3ForCausalLM(cfg)
        for i in (8, 20):
            mem = HashingMemory(input_dim=1024, output_dim=1024, mem_k_dim=512, mem_v_dim=1024, mem_heads=8,
                                mem_knn=32, mem_n_keys=1024, mem_share_values=False, mem_query_rmsnorm=True)
            mem.reset_parameters()
            model.model.layers[i].mlp = PkmBlock(mem)
    model = model.to(torch.bfloat16).train()
    gen = torch.Generator(device=dev).manual_seed(0)
    ids = torch.randint(0, cfg.vocab_size, (8, 2048), generator=gen, device=dev)
    n_params = sum(p.numel() for p in model.parameters())
    log(f"model ready: {n_params / 1e6:.1f} M parameters, PKM at layers 8 and 20")

    def step():
        model.zero_grad(set_to_none=True)
        out = model(input_ids=ids, labels=ids)
        out.loss.backward()
        return out.loss.detach()

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        loss = step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / args.steps
    log(f"model step: {ms:.2f} ms, loss {float(loss):.3f}")
    return {
        "metric": "Qwen3-0.6B-shaped decoder with 2 PKM layers, train step tokens/sec, bf16",
        "value": round(16384 / (ms * 1e-3), 1), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic (uniform token ids, random init)",
        "config": {"workload": "Qwen3-0.6B-shaped decoder (28 layers, hidden 1024, 16/8 heads, MLP 3072, vocab "
                               "151936), FFN of layers 8 and 20 replaced by PKM (8 heads, 2^20 slots, knn 32, "
                               "v_dim 1024); forward + causal-LM loss + backward, no optimizer",
                   "batch": 8, "seq_len": 2048, "parameters": n_params},
        "roofline": None, "cpu_baseline": None,
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", choices=["layer", "eb", "fwupdate", "fwpkm", "model", "stress"], default="layer")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extras", action="store_true",
                    help="layer workload: skip the extra measurements (standalone embedding bag, fast-weight "
                    "layer, the CPU parity configuration)")
    ap.add_argument(
        "--copy-probe-mib", type=int, default=0,
        help="run one plain elementwise copy (torch.neg, fp32) of this many MiB first; "
        "its FETCH_SIZE / WRITE_SIZE calibrate the HBM counters of the kernels",
    )
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(
            f"bench.py measures one GPU only (got --gpus {args.gpus}, WORLD_SIZE {world}): the PKM lookup "
            "path is benchmarked at its single-GPU shape; multi-GPU sharding is design-only.",
            file=sys.stderr,
        )
        sys.exit(2)

    import torch

    dev = torch.device("cuda", 0)
    if args.copy_probe_mib:
        src = torch.ones(args.copy_probe_mib << 18, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        torch.neg(src, out=dst)
        torch.cuda.synchronize()
        del src, dst
        log(f"copy probe: {args.copy_probe_mib} MiB read + {args.copy_probe_mib} MiB written")
    runs = {"layer": run_layer, "eb": run_eb, "fwupdate": run_fwupdate, "fwpkm": run_fwpkm_workload,
            "model": run_model, "stress": lambda a, d: run_stress(a, d, a.steps, a.warmup)}
    res = runs[args.workload](args, dev)
    if args.workload == "layer" and not args.no_extras:
        # the other benchmark configurations, reported beside the headline (not part of `value`)
        torch.cuda.empty_cache()
        log("extra: standalone embedding bag ...")
        eb = run_eb(args, dev)
        res["eb_standalone"] = {k: eb[k] for k in ("metric", "value", "unit", "ms_per_step", "config", "roofline",
                                                    "rooflines", "kernels", "cpu_baseline")}
        torch.cuda.empty_cache()
        log("extra: fast-weight PKM layer ...")
        res["fwpkm"] = run_fwpkm(args, dev)
        torch.cuda.empty_cache()
        if not args.no_cpu_baseline:
            log("extra: CPU parity configuration ...")
            res["cpu_parity_config"] = cpu_parity_config(args, dev)
            torch.cuda.empty_cache()
        log("extra: large-memory stress ...")
        res["stress"] = run_stress(args, dev)
        torch.cuda.empty_cache()
        log("extra: Qwen3-0.6B-shaped model step ...")
        margs = argparse.Namespace(**{**vars(args), "steps": 3, "warmup": 1})
        m = run_model(margs, dev)
        res["model_step"] = {kk: m[kk] for kk in ("metric", "value", "unit", "ms_per_step", "steps", "warmup",
                                                   "config")}
        torch.cuda.empty_cache()
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
