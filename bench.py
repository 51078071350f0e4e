#!/usr/bin/env python3
"""PKM lookup-path benchmark on one MI355X.

Workload (default): the standalone weighted embedding bag, forward + backward,
bf16 — 16384 bags x 128 lookups into a 2^20 x 1024 table, softmax
per-sample weights, N(0,1) upstream gradient — through the drop-in autograd
API (modelos_amd.pkm.xformer_embeddingbag.xformers_embedding_bag). One step =
forward gather + backward (dense weight gradient + per-sample-weight gradient).
A "token" is one bag (one token's H*knn lookups in the PKM layer).

Prints one JSON line: whole-job tokens/s, HBM roofline of the dominant kernel
(algorithmic bytes / HIP-event time), and the reference's CPU path
(F.embedding_bag + ATen autograd, pkm/xformer_embeddingbag.py:436-437) timed
on this host's cores on the same inputs.

Usage: python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--no-cpu-baseline]
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


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def load_traffic():
    """HBM bytes per launch measured with rocprofv3 --pmc (FETCH_SIZE,
    WRITE_SIZE), committed under profiles/; None if absent."""
    p = ROOT / "profiles" / "eb_hbm_traffic.json"
    if not p.exists():
        return None
    try:
        return json.loads(p.read_text())
    except ValueError:
        return None


def cpu_baseline(W, idx, p, g, min_seconds=10.0, max_repeats=3):
    """The reference's CPU path on the same inputs: F.embedding_bag + autograd."""
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

    t0 = time.perf_counter()
    step()  # warm-up
    warm = time.perf_counter() - t0
    reps = max(1, min(max_repeats, int(min_seconds / max(warm, 1e-3))))
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        step()
        times.append(time.perf_counter() - t0)
    times.sort()
    t = times[len(times) // 2]
    return {
        "value": idx.shape[0] / t,
        "unit": "tokens/s",
        "cores": cores,
        "kind": "port",
        "sample": f"full step ({idx.shape[0]} bags x {idx.shape[1]}, 2^20 x 1024 bf16 table), "
        f"median of {reps} after 1 warm-up; F.embedding_bag + ATen autograd on {cores} threads ({cpu_model()})",
        "ms_per_step": t * 1e3,
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument(
        "--copy-probe-mib", type=int, default=0,
        help="run one plain elementwise copy (torch.neg, fp32) of this many MiB after warm-up; "
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

    from modelos_amd.pkm.xformer_embeddingbag import xformers_embedding_bag

    dev = torch.device("cuda", 0)
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
    log(f"warmup done ({args.warmup} steps)")
    if args.copy_probe_mib:
        src = torch.ones(args.copy_probe_mib << 18, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        torch.neg(src, out=dst)
        torch.cuda.synchronize()
        del src, dst
        log(f"copy probe: {args.copy_probe_mib} MiB read + {args.copy_probe_mib} MiB written")

    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True),
           torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        W.grad = None
        p.grad = None
        ev[i][0].record()
        out = xformers_embedding_bag(idx, W, p)
        ev[i][1].record()
        out.backward(g)
        ev[i][2].record()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms_per_step = (t1 - t0) * 1e3 / args.steps
    fwd_ms = sorted(a.elapsed_time(b) for a, b, _ in ev)[args.steps // 2]
    bwd_ms = sorted(b.elapsed_time(c) for _, b, c in ev)[args.steps // 2]
    log(f"timed {args.steps} steps: {ms_per_step:.3f} ms/step (fwd {fwd_ms:.3f} ms, bwd {bwd_ms:.3f} ms)")

    a_fwd, a_bwd = eb_algorithmic_bytes(B, L, K, D, U)
    traffic = load_traffic() or {}
    kernels = {
        "eb_fwd_kernel": {
            "ms": fwd_ms, "algorithmic_bytes": a_fwd,
            "achieved_gbs": a_fwd / (fwd_ms * 1e-3) / 1e9,
        },
        "pkm_eb_bwd (count+scan+3 radix passes+row reduction)": {
            "ms": bwd_ms, "algorithmic_bytes": a_bwd,
            "achieved_gbs": a_bwd / (bwd_ms * 1e-3) / 1e9,
        },
    }
    for v in kernels.values():
        v["frac"] = v["achieved_gbs"] / HBM_PEAK_GBS
    dom_name, dom = max(kernels.items(), key=lambda kv: kv[1]["ms"])
    t = traffic.get("eb_fwd_kernel" if dom_name == "eb_fwd_kernel" else "pkm_eb_bwd")
    roofline = {
        "bound": "hbm",
        "kernel": dom_name,
        "achieved": round(dom["achieved_gbs"], 1),
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(dom["frac"], 4),
        "traffic": t,
    }

    cpu = None
    if not args.no_cpu_baseline:
        log("timing the CPU baseline ...")
        cpu = cpu_baseline(W, idx, p, g)
        log(f"cpu baseline: {cpu['ms_per_step']:.1f} ms/step on {cpu['cores']} threads")

    res = {
        "metric": METRIC,
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
            "psw": "softmax(N(0,1)) bf16", "table": "N(0,0.03) bf16",
        },
        "roofline": roofline,
        "kernels": {k: {kk: (round(vv, 4) if isinstance(vv, float) else vv) for kk, vv in v.items()}
                    for k, v in kernels.items()},
        "cpu_baseline": cpu,
    }
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
