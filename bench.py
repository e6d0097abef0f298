#!/usr/bin/env python3
"""Benchmark of the fused RoPE + varlen attention path on one MI355X.

Metric: microseconds per call of the fused op on the 1344^2
Qwen2.5-VL window layer (workload ``cfg2w``: 9216 tokens in 144 windows of 64,
16 heads, head_dim 80, bf16 q/k/v, fp32 cos/sin [N, 40]), plus its fraction of
the HBM roofline.

Protocol:
* inputs are synthetic (q, k, v ~ N(0, 1), seeded) and resident in HBM;
* ``--warmup`` untimed calls, then ``--steps`` timed calls; before each timed
  call a 1 GiB buffer is read (a reduction over it), so that neither the L2s
  nor the 256 MB Infinity Cache hold the inputs and no dirty lines are left
  for the timed call to write back (the cold number is the headline); each call
  is bracketed by HIP events on the stream the kernel runs on (torch's
  current stream); ``value`` is the median;
* the warm number is the same call back to back, total time / steps;
* ``roofline.achieved`` = algorithmic bytes (window layers) or flops (full
  layers) / median call time;
* ``cpu_baseline`` times the CPU oracle (numpy fp32 port of the unfused path)
  on this host on a bounded sample of the same workload.

Prints ONE JSON line on stdout.  ``--report FILE`` additionally measures every
workload and writes the list to FILE.
"""
import argparse
import json
import os
import statistics
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

from fused_rope_attn_amd import fused_rope_attention, plan  # noqa: E402
from fused_rope_attn_amd.configs import WORKLOADS, algorithmic_bytes, algorithmic_flops, make_inputs  # noqa: E402

METRIC = "µs/call fused RoPE+varlen attn (1344² window layer); % HBM/MFMA roofline"
HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, published
MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 MFMA, published
FLUSH_BYTES = 1 << 30


def workload_cost(w, inp):
    cu = inp["cu_seqlens"].cpu()
    lens = (cu[1:] - cu[:-1]).tolist()
    n = int(cu[-1])
    cos = inp["cos"]
    nbytes = algorithmic_bytes(n, w.heads, w.head_dim, inp["q"].element_size(), cos.shape[1],
                               cos.element_size(), len(lens))
    flops = algorithmic_flops(w.heads, w.head_dim, lens)
    return n, lens, nbytes, flops


def evict(flush: torch.Tensor) -> None:
    """Read the whole flush buffer: the caches end up holding its (clean)
    lines instead of the workload's inputs."""
    torch.sum(flush, dtype=torch.int32)


def measure(inp, steps: int, warmup: int, flush: torch.Tensor) -> dict:
    q, k, v, cos, sin, cu = (inp[x] for x in ("q", "k", "v", "cos", "sin", "cu_seqlens"))
    ms = inp["max_seqlen"]
    out = torch.empty_like(q)

    def call():
        fused_rope_attention(q, k, v, cos, sin, cu, ms, out=out)

    for _ in range(warmup):
        call()
    torch.cuda.synchronize()

    stream = torch.cuda.current_stream()
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        evict(flush)
        starts[i].record(stream)
        call()
        ends[i].record(stream)
    torch.cuda.synchronize()
    wall_cold = time.perf_counter() - t0
    cold = sorted(s.elapsed_time(e) * 1000.0 for s, e in zip(starts, ends))

    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(stream)
    for _ in range(steps):
        call()
    e1.record(stream)
    torch.cuda.synchronize()
    warm = e0.elapsed_time(e1) * 1000.0 / steps

    def pct(p):
        return cold[min(len(cold) - 1, int(p * (len(cold) - 1) + 0.5))]

    return {"cold_median_us": statistics.median(cold), "cold_mean_us": sum(cold) / len(cold),
            "cold_p10_us": pct(0.1), "cold_p90_us": pct(0.9), "warm_us": warm,
            "wall_cold_s": wall_cold}


def cpu_baseline(w, inp, budget_s: float) -> dict:
    """The oracle's fp32 unfused path on the host cores, on a bounded sample,
    scaled to one full call."""
    import numpy as np

    from oracle import attention as A
    try:
        from threadpoolctl import threadpool_info
        threads = max([p.get("num_threads", 1) for p in threadpool_info() if p.get("user_api") == "blas"] or [1])
    except Exception:
        threads = os.cpu_count() or 1
    q, k, v = (inp[x].float().cpu().numpy() for x in ("q", "k", "v"))
    cos, sin = inp["cos"].float().cpu().numpy(), inp["sin"].float().cpu().numpy()
    cu = inp["cu_seqlens"].cpu().numpy()
    if w.kind == "window":
        heads, scale, sample = list(range(w.heads)), 1.0, "the full call (all windows, all heads)"
    else:
        heads, scale, sample = [0], float(w.heads), f"one head of {w.heads}, scaled by {w.heads}"
    qs, ks, vs = q[:, heads], k[:, heads], v[:, heads]
    A.fused_rope_attention(qs[:64], ks[:64], vs[:64], cos[:64], sin[:64], np.array([0, 64]))  # warm the BLAS
    times = []
    t_start = time.perf_counter()
    while True:
        t0 = time.perf_counter()
        A.fused_rope_attention(qs, ks, vs, cos, sin, cu)
        times.append(time.perf_counter() - t0)
        if time.perf_counter() - t_start > budget_s or len(times) >= 200:
            break
    per_call = statistics.median(times) * scale
    return {"value": per_call * 1e6, "unit": "µs/call", "cores": int(threads), "kind": "port",
            "sample": f"numpy fp32 oracle of the unfused path (rotate, then per-segment softmax attention), "
                      f"{sample}; median of {len(times)} runs; host has {os.cpu_count()} logical CPUs"}


def run_workload(name: str, steps: int, warmup: int, flush: torch.Tensor, dev) -> dict:
    w = WORKLOADS[name]
    inp = make_inputs(w, seed=1234 + list(WORKLOADS).index(name), device=dev)
    n, lens, nbytes, flops = workload_cost(w, inp)
    pl = plan(*(inp[x] for x in ("q", "k", "v", "cos", "sin", "cu_seqlens")), max_seqlen=inp["max_seqlen"])
    m = measure(inp, steps, warmup, flush)
    t = m["cold_median_us"] * 1e-6
    hbm = w.kind == "window"
    achieved = nbytes / t / 1e9 if hbm else flops / t / 1e12
    peak = HBM_PEAK_GBS if hbm else MFMA_BF16_PEAK_TFLOPS
    return {"workload": name, "note": w.note, "tokens": n, "segments": len(lens), "max_seqlen": max(lens),
            "heads": w.heads, "head_dim": w.head_dim, "kernel": pl["name"], "grid": pl["grid"],
            "bytes": nbytes, "flops": flops, **m,
            "roofline": {"bound": "hbm" if hbm else "mfma", "achieved": achieved, "peak": peak,
                         "unit": "GB/s" if hbm else "TFLOP/s", "frac": achieved / peak},
            "warm_achieved": (nbytes if hbm else flops) / (m["warm_us"] * 1e-6) / (1e9 if hbm else 1e12)}, inp


def profile_driver(args, flush, dev) -> int:
    """Kernel launches for rocprofv3: warmup, then ``--profile-calls`` calls of
    the workload each after a cache flush, then one copy of known size whose
    FETCH_SIZE / WRITE_SIZE calibrate the counters (it reads and writes
    exactly ``--copy-mib`` MiB)."""
    w = WORKLOADS[args.workload]
    inp = make_inputs(w, seed=1234 + list(WORKLOADS).index(args.workload), device=dev)
    q, k, v, cos, sin, cu = (inp[x] for x in ("q", "k", "v", "cos", "sin", "cu_seqlens"))
    out = torch.empty_like(q)
    for _ in range(3):
        fused_rope_attention(q, k, v, cos, sin, cu, inp["max_seqlen"], out=out)
    for i in range(args.profile_calls):
        evict(flush)
        fused_rope_attention(q, k, v, cos, sin, cu, inp["max_seqlen"], out=out)
    torch.cuda.synchronize()
    n = args.copy_mib << 20
    src = torch.ones(n // 4, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    evict(flush)
    dst.copy_(src)
    torch.cuda.synchronize()
    n_tok, lens, nbytes, flops = workload_cost(w, inp)
    print(json.dumps({"profile_driver": args.workload, "calls": args.profile_calls, "bytes": nbytes,
                      "flops": flops, "copy_bytes_each_way": n}), flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="cfg2w", choices=list(WORKLOADS))
    ap.add_argument("--report", default=None, help="measure every workload and write them to this JSON file")
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="CPU baseline time budget")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--profile-calls", type=int, default=0,
                    help="profiling driver: run this many cold calls of --workload, then a plain "
                         "device copy of --copy-mib MiB (HBM counter calibration), and exit")
    ap.add_argument("--copy-mib", type=int, default=256)
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (the op shards by head or "
              "segment with no exchange; see DESIGN.md).  Run with --gpus 1.", file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    dev = torch.device("cuda:0")
    flush = torch.ones(FLUSH_BYTES, dtype=torch.uint8, device=dev)
    if args.profile_calls:
        return profile_driver(args, flush, dev)

    torch.cuda.synchronize()
    res, inp = run_workload(args.workload, args.steps, args.warmup, flush, dev)
    w = WORKLOADS[args.workload]
    line = {
        "metric": METRIC,
        "value": round(res["cold_median_us"], 3),
        "unit": "µs/call",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(res["cold_median_us"] / 1000.0, 6),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": f"{args.workload}: {w.note}", "tokens": res["tokens"], "segments": res["segments"],
                   "max_seqlen": res["max_seqlen"], "heads": w.heads, "head_dim": w.head_dim,
                   "qkv": "bf16 [N, H, D]", "rope": f"fp32 [N, {w.head_dim // 2}]",
                   "cache": "cold: 1 GiB read before each timed call", "parallelism": "single GPU"},
        "roofline": dict(res["roofline"], traffic=None),
        "kernel": res["kernel"],
        "cold_p10_us": round(res["cold_p10_us"], 3),
        "cold_p90_us": round(res["cold_p90_us"], 3),
        "warm_us": round(res["warm_us"], 3),
        "warm_frac": round(res["warm_achieved"] / res["roofline"]["peak"], 4),
    }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(w, inp, args.cpu_seconds)
    del inp

    if args.report:
        rows = [res]
        for name in WORKLOADS:
            if name == args.workload:
                continue
            r, _ = run_workload(name, max(10, args.steps // 2), max(3, args.warmup // 2), flush, dev)
            rows.append(r)
            print(f"[bench] {name}: cold {r['cold_median_us']:.1f} us, warm {r['warm_us']:.1f} us, "
                  f"{r['roofline']['frac'] * 100:.1f}% of {r['roofline']['bound']}", file=sys.stderr, flush=True)
        with open(args.report, "w") as f:
            json.dump(rows, f, indent=1)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
