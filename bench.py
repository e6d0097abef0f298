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

from fused_rope_attn_amd import (fused_rope_attention, fused_rope_attention_bwd,  # noqa: E402
                                 fused_rope_attention_fwd, fused_rope_attention_pos, plan, plan_pos)
from fused_rope_attn_amd.configs import (WORKLOADS, algorithmic_bytes, algorithmic_bytes_bwd,  # noqa: E402
                                         algorithmic_flops, algorithmic_flops_bwd, image_order, make_inputs,
                                         positions)

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


def committed_traffic(workload: str, kernel: str):
    """HBM bytes per call of ``kernel`` on ``workload`` from the committed
    rocprofv3 summary ``profiles/<workload>_<kernel>.md`` (FETCH_SIZE and
    WRITE_SIZE, each calibrated by a device copy of known size), or None when
    no summary for this kernel is committed."""
    path = os.path.join(ROOT, "profiles", f"{workload}_{kernel}.md")
    if not os.path.exists(path):
        return None
    fields = {}
    with open(path) as f:
        for ln in f:
            if ":" in ln and ln.startswith("- `"):
                key, _, val = ln[3:].partition("`:")
                fields[key.strip()] = val.strip().strip("`")
    if fields.get("kernel") != kernel or "traffic_bytes_per_call" not in fields:
        return None
    return int(fields["traffic_bytes_per_call"])


def evict(flush: torch.Tensor) -> None:
    """Read the whole flush buffer with one reduction that converts nothing
    (int64 elements, int64 sum): the caches end up holding its clean lines
    instead of the workload's inputs, and no dirty lines are left behind."""
    flush.view(torch.int64).sum()


def measure(inp, steps: int, warmup: int, flush: torch.Tensor) -> dict:
    q, k, v, cos, sin, cu = (inp[x] for x in ("q", "k", "v", "cos", "sin", "cu_seqlens"))
    ms = inp["max_seqlen"]
    out = torch.empty_like(q)

    def call():
        fused_rope_attention(q, k, v, cos, sin, cu, ms, out=out)

    return time_calls(call, steps, warmup, flush)


def backward_call(inp):
    """A closure running one backward (``fused_rope_attention_bwd``: the
    row-dot, dq and dk/dv kernels) on the workload, with dO ~ N(0, 1) and
    the forward's out and lse computed once beforehand."""
    q, k, v, cos, sin, cu = (inp[x] for x in ("q", "k", "v", "cos", "sin", "cu_seqlens"))
    ms = inp["max_seqlen"]
    out, lse = fused_rope_attention_fwd(q, k, v, cos, sin, cu, ms)
    g = torch.Generator(device=q.device).manual_seed(99)
    dout = torch.randn(q.shape, generator=g, device=q.device).to(q.dtype)
    dq, dk, dv = (torch.empty_like(q) for _ in range(3))

    def call():
        fused_rope_attention_bwd(dout, q, k, v, cos, sin, out, lse, cu, ms, dq=dq, dk=dk, dv=dv)

    return call


def floor_call(inp):
    """A closure running the box's floor for a window layer's traffic: one
    elementwise kernel that reads the layer's q, k and v and writes an
    output of the same shape (``torch.addcmul(q, k, v)``: torch's own
    vectorised, coalesced elementwise kernel), i.e. the fused op's Q/K/V/O
    bytes with no attention, no rotation, no tables and no dependent
    round trips between the loads and the store."""
    q, k, v = inp["q"], inp["k"], inp["v"]
    o = torch.empty_like(q)

    def call():
        torch.addcmul(q, k, v, out=o)

    return call


def time_calls(call, steps: int, warmup: int, flush: torch.Tensor) -> dict:
    """Cold (1 GiB read before each call) and warm (back-to-back) timings of
    ``call`` with HIP events on torch's current stream, where the kernels run."""
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


def unfused_call(inp):
    """A closure running the unfused path on the GPU, as the reference's own
    benchmark baseline does it (bench.py:72-82 of the reference: rotate Q and
    K with separate elementwise ops in fp32, round to the input dtype, then
    varlen attention), with torch's ``varlen_attn`` in place of the CUDA-only
    flash-attn."""
    from torch.nn.attention.varlen import varlen_attn
    q, k, v, cos, sin, cu = (inp[x] for x in ("q", "k", "v", "cos", "sin", "cu_seqlens"))
    ms = inp["max_seqlen"]
    half = q.shape[2] // 2
    c, s = cos.float()[:, None, :], sin.float()[:, None, :]

    def rot(x):
        xf = x.float()
        x0, x1 = xf[..., :half], xf[..., half:]
        return torch.cat([x0 * c - x1 * s, x0 * s + x1 * c], -1).to(x.dtype)

    def call():
        return varlen_attn(rot(q), rot(k), v, cu, cu, ms, ms)

    return call


def train_step_calls(inp):
    """Closures running forward + backward through autograd (dO ~ N(0, 1)):
    the fused op, and the unfused path of ``unfused_call`` (whose rotation and
    attention get their gradients from torch)."""
    from torch.nn.attention.varlen import varlen_attn
    q, k, v, cos, sin, cu = (inp[x] for x in ("q", "k", "v", "cos", "sin", "cu_seqlens"))
    ms = inp["max_seqlen"]
    half = q.shape[2] // 2
    c, s = cos.float()[:, None, :], sin.float()[:, None, :]
    g = torch.Generator(device=q.device).manual_seed(98)
    dout = torch.randn(q.shape, generator=g, device=q.device).to(q.dtype)
    qg, kg, vg = (t.detach().clone().requires_grad_(True) for t in (q, k, v))

    def rot(x):
        xf = x.float()
        x0, x1 = xf[..., :half], xf[..., half:]
        return torch.cat([x0 * c - x1 * s, x0 * s + x1 * c], -1).to(x.dtype)

    def fused():
        qg.grad = kg.grad = vg.grad = None
        fused_rope_attention(qg, kg, vg, cos, sin, cu, ms).backward(dout)

    def unfused():
        qg.grad = kg.grad = vg.grad = None
        varlen_attn(rot(qg), rot(kg), vg, cu, cu, ms, ms).backward(dout)

    return fused, unfused


def run_comparator(name: str, steps: int, warmup: int, flush: torch.Tensor, dev) -> dict:
    """The fused op and the unfused torch path on the same inputs and GPU:
    cold medians and their ratio (context only; the reference's published
    figures are this ratio on its own hardware)."""
    w = WORKLOADS[name]
    inp = make_inputs(w, seed=1234 + list(WORKLOADS).index(name), device=dev)
    row = {"workload": name, "note": w.note}
    fused = measure(inp, steps, warmup, flush)
    row["fused_cold_us"] = fused["cold_median_us"]
    try:
        call = unfused_call(inp)
        ref = call()
        got = fused_rope_attention(inp["q"], inp["k"], inp["v"], inp["cos"], inp["sin"], inp["cu_seqlens"],
                                   inp["max_seqlen"])
        torch.cuda.synchronize()
        row["max_abs_diff"] = float((ref.float() - got.float()).abs().max())
        m = time_calls(call, steps, warmup, flush)
        row["unfused_cold_us"] = m["cold_median_us"]
        row["speedup"] = m["cold_median_us"] / fused["cold_median_us"]
        f_call, u_call = train_step_calls(inp)
        mf = time_calls(f_call, steps, warmup, flush)
        mu = time_calls(u_call, steps, warmup, flush)
        row["fused_fwd_bwd_cold_us"] = mf["cold_median_us"]
        row["unfused_fwd_bwd_cold_us"] = mu["cold_median_us"]
        row["fwd_bwd_speedup"] = mu["cold_median_us"] / mf["cold_median_us"]
    except Exception as e:  # an unsupported head_dim or backend: recorded, not fatal
        row["unfused_error"] = f"{type(e).__name__}: {e}"[:300]
    return row


def positions_call(w, inp, dev):
    """A closure running ``fused_rope_attention_pos`` on the workload: the
    same q, k, v and cu_seqlens, the rotation angles computed in the kernels
    from the tokens' (h, w) positions instead of read from cos/sin."""
    pos, inv = positions(w, dev)
    q, k, v, cu = (inp[x] for x in ("q", "k", "v", "cu_seqlens"))
    ms = inp["max_seqlen"]
    out = torch.empty_like(q)

    def call():
        fused_rope_attention_pos(q, k, v, pos, inv, cu, ms, out=out)

    return call, pos, inv


def run_positions(name: str, steps: int, warmup: int, flush: torch.Tensor, dev) -> dict:
    """The table op and the position variant on the same inputs, timed
    alternately (table, positions, table, positions): cold medians."""
    w = WORKLOADS[name]
    inp = make_inputs(w, seed=1234 + list(WORKLOADS).index(name), device=dev)
    q, k, v, cos, sin, cu = (inp[x] for x in ("q", "k", "v", "cos", "sin", "cu_seqlens"))
    ms = inp["max_seqlen"]
    out = torch.empty_like(q)

    def tab():
        fused_rope_attention(q, k, v, cos, sin, cu, ms, out=out)

    posc, pos, inv = positions_call(w, inp, dev)
    t1 = time_calls(tab, steps, warmup, flush)
    p1 = time_calls(posc, steps, warmup, flush)
    t2 = time_calls(tab, steps, warmup, flush)
    p2 = time_calls(posc, steps, warmup, flush)
    ref = fused_rope_attention(q, k, v, cos, sin, cu, ms)
    got = fused_rope_attention_pos(q, k, v, pos, inv, cu, ms)
    torch.cuda.synchronize()
    tab_us = (t1["cold_median_us"] + t2["cold_median_us"]) / 2
    pos_us = (p1["cold_median_us"] + p2["cold_median_us"]) / 2
    return {"workload": name, "note": w.note, "kernel": plan_pos(q, k, v, pos, inv, cu, ms)["name"],
            "tables_cold_us": tab_us, "positions_cold_us": pos_us, "positions_over_tables": pos_us / tab_us,
            "tables_warm_us": (t1["warm_us"] + t2["warm_us"]) / 2,
            "positions_warm_us": (p1["warm_us"] + p2["warm_us"]) / 2,
            "max_abs_diff": float((ref.float() - got.float()).abs().max())}


HIDDEN = 1280  # Qwen2.5-VL vision hidden size: the encoder shuffles [N, HIDDEN] hidden states


def run_gather(name: str, steps: int, warmup: int, flush: torch.Tensor, dev) -> dict:
    """A window layer on window-ordered tensors (the reference's route) and
    on image-ordered tensors through ``row_index`` (the shuffle fused into
    the kernel's addressing), timed alternately, beside the two gathers the
    fused form removes from an encoder pass: ``window_shuffle`` of the
    ``[N, 1280]`` bf16 hidden state before the blocks and
    ``window_unshuffle`` after them."""
    from fused_rope_attn_amd import window_shuffle, window_unshuffle, get_window_index
    w = WORKLOADS[name]
    inp = make_inputs(w, seed=1234 + list(WORKLOADS).index(name), device=dev)
    rows, cos_i, sin_i = image_order(w, dev)
    inv = torch.empty_like(rows, dtype=torch.int64)
    inv[rows.long()] = torch.arange(rows.numel(), device=dev)
    q, k, v, cos, sin, cu = (inp[x] for x in ("q", "k", "v", "cos", "sin", "cu_seqlens"))
    qi, ki, vi = q[inv], k[inv], v[inv]
    ms = inp["max_seqlen"]
    out, outi = torch.empty_like(q), torch.empty_like(q)

    def win():
        fused_rope_attention(q, k, v, cos, sin, cu, ms, out=out)

    def gat():
        fused_rope_attention(qi, ki, vi, cos_i, sin_i, cu, ms, out=outi, row_index=rows)

    hid = torch.randn(rows.numel(), HIDDEN, device=dev).to(torch.bfloat16)
    widx = rows.view(-1, 4)[:, 0].long() // 4 if len(w.groups) == 1 and w.groups[0][1] == 2 else None

    a1 = time_calls(win, steps, warmup, flush)
    g1 = time_calls(gat, steps, warmup, flush)
    a2 = time_calls(win, steps, warmup, flush)
    g2 = time_calls(gat, steps, warmup, flush)
    row = {"workload": name, "note": w.note,
           "window_order_cold_us": (a1["cold_median_us"] + a2["cold_median_us"]) / 2,
           "image_order_gather_cold_us": (g1["cold_median_us"] + g2["cold_median_us"]) / 2}
    row["gather_over_window_order"] = row["image_order_gather_cold_us"] / row["window_order_cold_us"]
    if widx is not None:
        sh = time_calls(lambda: window_shuffle(hid, widx), steps, warmup, flush)
        un = time_calls(lambda: window_unshuffle(hid, widx), steps, warmup, flush)
        row["hidden_shuffle_cold_us"] = sh["cold_median_us"]
        row["hidden_unshuffle_cold_us"] = un["cold_median_us"]
        row["window_layers_to_break_even"] = ((sh["cold_median_us"] + un["cold_median_us"])
                                              / max(1e-9, row["image_order_gather_cold_us"]
                                                    - row["window_order_cold_us"]))
    return row


def run_backward(name: str, steps: int, warmup: int, flush: torch.Tensor, dev) -> dict:
    w = WORKLOADS[name]
    inp = make_inputs(w, seed=1234 + list(WORKLOADS).index(name), device=dev)
    cu = inp["cu_seqlens"].cpu()
    lens = (cu[1:] - cu[:-1]).tolist()
    n = int(cu[-1])
    cos = inp["cos"]
    nbytes = algorithmic_bytes_bwd(n, w.heads, w.head_dim, inp["q"].element_size(), cos.shape[1],
                                   cos.element_size(), len(lens))
    flops = algorithmic_flops_bwd(w.heads, w.head_dim, lens)
    m = time_calls(backward_call(inp), steps, warmup, flush)
    t = m["cold_median_us"] * 1e-6
    hbm = w.kind == "window"
    achieved = nbytes / t / 1e9 if hbm else flops / t / 1e12
    peak = HBM_PEAK_GBS if hbm else MFMA_BF16_PEAK_TFLOPS
    return {"workload": name, "direction": "backward", "note": w.note, "tokens": n, "segments": len(lens),
            "max_seqlen": max(lens), "heads": w.heads, "head_dim": w.head_dim, "bytes": nbytes, "flops": flops, **m,
            "roofline": {"bound": "hbm" if hbm else "mfma", "achieved": achieved, "peak": peak,
                         "unit": "GB/s" if hbm else "TFLOP/s", "frac": achieved / peak}}


def profile_driver(args, flush, dev) -> int:
    """Kernel launches for rocprofv3: warmup, then ``--profile-calls`` calls of
    the workload each after a cache flush, then one copy of known size whose
    FETCH_SIZE / WRITE_SIZE calibrate the counters (it reads and writes
    exactly ``--copy-mib`` MiB)."""
    w = WORKLOADS[args.workload]
    inp = make_inputs(w, seed=1234 + list(WORKLOADS).index(args.workload), device=dev)
    q, k, v, cos, sin, cu = (inp[x] for x in ("q", "k", "v", "cos", "sin", "cu_seqlens"))
    out = torch.empty_like(q)
    if args.bwd:
        call = backward_call(inp)
    elif args.pos:
        call, _, _ = positions_call(w, inp, dev)
    elif args.floor:
        call = floor_call(inp)
    else:
        def call():
            fused_rope_attention(q, k, v, cos, sin, cu, inp["max_seqlen"], out=out)
    for _ in range(3):
        call()
    for i in range(args.profile_calls):
        evict(flush)
        call()
    torch.cuda.synchronize()
    n = args.copy_mib << 20
    src = torch.ones(n // 4, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    evict(flush)
    dst.copy_(src)
    torch.cuda.synchronize()
    n_tok, lens, nbytes, flops = workload_cost(w, inp)
    pl = plan(q, k, v, cos, sin, cu, max_seqlen=inp["max_seqlen"])
    if args.bwd:
        nbytes = algorithmic_bytes_bwd(n_tok, w.heads, w.head_dim, q.element_size(), cos.shape[1],
                                       cos.element_size(), len(lens))
        flops = algorithmic_flops_bwd(w.heads, w.head_dim, lens)
    if args.floor:
        nbytes = 4 * q.numel() * q.element_size()
    if args.pos:
        pos, inv = positions(w, dev)
        pl = plan_pos(q, k, v, pos, inv, cu, inp["max_seqlen"])
        # no tables read; the (h, w) positions and inv_freq instead
        nbytes += n_tok * 8 + (w.head_dim // 4) * 4 - 2 * n_tok * cos.shape[1] * cos.element_size()
    print(json.dumps({"profile_driver": args.workload, "direction": "backward" if args.bwd else "forward",
                      "kernel": "floor: torch.addcmul(q, k, v)" if args.floor else pl["name"], "warmup_calls": 3,
                      "calls": args.profile_calls, "bytes": nbytes, "flops": flops,
                      "copy_bytes_each_way": n}), flush=True)
    return 0


def torch_reference_attention(q, k, v, cos, sin, cu, scale: float, mode: str = "fp32"):
    """The unfused path in plain torch float32 on q's device, for stacks too
    large for the CPU oracle: split-half rotation (reference
    fused_attn.py:340-345, 385-390), then per-segment softmax attention.
    ``mode`` "fp32" is the oracle's fp32 path; "bf16" is its rounding-point
    model (q_rot, k_rot and the unnormalised P rounded to bf16, the row sum
    from the unrounded P, the output rounded; oracle/attention.py).  Inputs
    are float32 ``[N, H, D]``; rows outside every segment come back NaN.
    ``tests/test_gpu_drift.py`` pins it to the CPU oracle."""
    import math

    n, h, d = q.shape
    half = d // 2
    c0, s0 = cos[:, None, :half], sin[:, None, :half]
    c1, s1 = (cos[:, None, half:], sin[:, None, half:]) if cos.shape[1] == d else (c0, s0)

    def rot(x):
        x0, x1 = x[..., :half], x[..., half:]
        return torch.cat([x0 * c0 - x1 * s0, x0 * s1 + x1 * c1], dim=-1)

    qr, kr = rot(q), rot(k)
    if mode == "bf16":
        qr, kr = qr.bfloat16().float(), kr.bfloat16().float()
    scale_log2 = float(torch.tensor(scale, dtype=torch.float32) * torch.tensor(math.log2(math.e), dtype=torch.float32))
    out = torch.full_like(q, float("nan"))
    bounds = [(min(max(a, 0), n), min(max(b, 0), n)) for a, b in zip(cu[:-1].tolist(), cu[1:].tolist())]
    by_len = {}
    for a, b in bounds:
        if b > a:
            by_len.setdefault(b - a, []).append(a)
    for L, starts in by_len.items():
        idx = torch.tensor(starts, device=q.device)[:, None] + torch.arange(L, device=q.device)[None, :]
        # [segments, H, L, D] blocks, several segments or one head's row chunk at a time
        per_seg = h * L * L * 4
        step = max(1, (1 << 30) // per_seg)
        for i in range(0, len(starts), step):
            sl = idx[i:i + step]
            qb, kb, vb = (x[sl].permute(0, 2, 1, 3).contiguous() for x in (qr, kr, v))
            for hh in range(h) if per_seg > (1 << 30) else [None]:
                hs = slice(None) if hh is None else slice(hh, hh + 1)
                kt = kb[:, hs].transpose(-1, -2).contiguous()
                rows = L if hh is None else max(1, (1 << 30) // (L * 4))
                for r0 in range(0, L, rows):
                    qq = qb[:, hs, r0:r0 + rows]
                    s_ = torch.matmul(qq, kt)
                    if mode == "fp32":
                        o = torch.matmul(torch.softmax(s_ * scale, dim=-1), vb[:, hs])
                    else:
                        s_ = s_ * scale_log2
                        p_ = torch.exp2(s_ - s_.amax(dim=-1, keepdim=True))
                        o = torch.matmul(p_.bfloat16().float(), vb[:, hs]) / p_.sum(dim=-1, keepdim=True)
                    blk = o.permute(0, 2, 1, 3)                   # [segments, rows, heads, D]
                    tgt = sl[:, r0:r0 + rows]
                    if hh is None:
                        out[tgt] = blk
                    else:
                        out[tgt, hh:hh + 1] = blk
    if mode == "bf16":
        out = out.bfloat16().float()
    return out


def drift_stack(wname: str, device, layers: int = 32, full_layers=(7, 15, 23, 31), seed: int = 7,
                reference: str = "cpu") -> dict:
    """Relative drift of a stack of attention layers run through the fused op
    in bf16, against the same stack in fp32 (BASELINE config 2's 32-layer
    stack; the reference's precision caveat is its README.md:10).

    Layer l normalises each token of ``x_l [N, H, D]`` to unit RMS (a
    pre-norm block, which keeps the logits O(1) however far the residual
    stream grows), maps it to q, k, v with seeded per-head ``D x D`` matrices
    (scaled by ``1/sqrt(D)``) and adds the attention output:
    ``x_{l+1} = x_l + attn_l(q, k, v)``.  Window layers use the workload's
    window ``cu_seqlens``; layers in ``full_layers`` attend over the whole
    image (the tokens stay in window order, as in the Qwen2.5-VL encoder).
    The GPU stack keeps activations in bf16.  A third stack runs the bf16
    rounding model (the same rounding points evaluated exactly): the drift
    any bf16 pipeline with these rounding points has, i.e. the floor the GPU
    stack is compared with.  The two reference stacks run in the numpy
    oracle on the CPU (``reference="cpu"``) or in plain torch float32 on the
    GPU (``reference="gpu"``, ``torch_reference_attention``) for sizes where
    the CPU model of the rounding takes minutes per layer.
    Returns per-layer ``||x - x_ref|| / ||x_ref||`` of both."""
    import math

    import numpy as np

    w = WORKLOADS[wname]
    inp = make_inputs(w, seed=seed, device="cpu", heads=1)
    cos, sin, cu_win = inp["cos"], inp["sin"], inp["cu_seqlens"]
    n, h, d = int(cu_win[-1]), w.heads, w.head_dim
    cu_full = torch.tensor([0, n], dtype=torch.int32)
    g = torch.Generator().manual_seed(seed)
    x0 = torch.randn(n, h, d, generator=g)
    cos_d, sin_d = cos.to(device), sin.to(device)
    if reference == "cpu":
        from oracle import attention as A
        from oracle.numerics import round_bf16
        cos_np, sin_np = cos.float().numpy(), sin.float().numpy()
        xr = x0.numpy().copy()
        xe = round_bf16(xr)
    else:
        xr = x0.to(device)
        xe = xr.bfloat16().float()
    xg = x0.to(torch.bfloat16).to(device)
    scale = d ** -0.5
    rows = []
    for layer in range(layers):
        wts = torch.randn(3, h, d, d, generator=g) / math.sqrt(d)
        full = layer in full_layers
        cu = cu_full if full else cu_win
        ms = int((cu[1:] - cu[:-1]).max())
        if reference == "cpu":
            cu_np, wn = cu.numpy(), wts.numpy()

            def rms(x):
                return x / np.sqrt(np.mean(np.square(x), axis=(1, 2), keepdims=True) + np.float32(1e-6))

            qkv = np.matmul(rms(xr).transpose(1, 0, 2)[None], wn).transpose(0, 2, 1, 3)
            xr = xr + A.fused_rope_attention(qkv[0], qkv[1], qkv[2], cos_np, sin_np, cu_np, mode="fp32")
            qkv = round_bf16(np.matmul(rms(xe).transpose(1, 0, 2)[None], wn).transpose(0, 2, 1, 3))
            att = A.fused_rope_attention(qkv[0], qkv[1], qkv[2], cos_np, sin_np, cu_np, mode="bf16")
            xe = round_bf16(xe + att)
        else:
            wd, cud = wts.to(device), cu.to(device)

            def rms_t(x):
                return x * torch.rsqrt(x.square().mean(dim=(1, 2), keepdim=True) + 1e-6)

            qkv = torch.matmul(rms_t(xr).transpose(0, 1)[None], wd).transpose(1, 2)
            xr = xr + torch_reference_attention(qkv[0], qkv[1], qkv[2], cos_d.float(), sin_d.float(), cud, scale)
            qkv = torch.matmul(rms_t(xe).transpose(0, 1)[None], wd).transpose(1, 2).bfloat16().float()
            att = torch_reference_attention(qkv[0], qkv[1], qkv[2], cos_d.float(), sin_d.float(), cud, scale, "bf16")
            xe = (xe + att).bfloat16().float()
        # the fused op on the GPU (projections in fp32, activations stored in bf16)
        xf = xg.float()
        xf = xf * torch.rsqrt(xf.square().mean(dim=(1, 2), keepdim=True) + 1e-6)
        qkv = torch.matmul(xf.transpose(0, 1)[None], wts.to(device)).transpose(1, 2)
        qkv = qkv.to(torch.bfloat16).contiguous()
        out = fused_rope_attention(qkv[0], qkv[1], qkv[2], cos_d, sin_d, cu.to(device), ms)
        xg = (xg.float() + out.float()).to(torch.bfloat16)
        if reference == "cpu":
            ref_norm = float(np.linalg.norm(xr))
            gpu = float(np.linalg.norm(xg.float().cpu().numpy() - xr)) / ref_norm
            emu = float(np.linalg.norm(xe - xr)) / ref_norm
        else:
            ref_norm = float(torch.linalg.vector_norm(xr))
            gpu = float(torch.linalg.vector_norm(xg.float() - xr)) / ref_norm
            emu = float(torch.linalg.vector_norm(xe - xr)) / ref_norm
        rows.append({"layer": layer, "kind": "full" if full else "window", "gpu_rel": gpu, "bf16_model_rel": emu})
        print(f"[drift] layer {layer:2d} {'full  ' if full else 'window'} gpu {gpu:.3e}  bf16-model {emu:.3e}",
              file=sys.stderr, flush=True)
    return {"workload": wname, "layers": layers, "full_layers": list(full_layers), "tokens": n, "heads": h,
            "head_dim": d, "reference": reference, "per_layer": rows, "final_gpu_rel": rows[-1]["gpu_rel"],
            "final_bf16_model_rel": rows[-1]["bf16_model_rel"]}


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
    ap.add_argument("--bwd", action="store_true", help="profiling driver: run backward calls instead")
    ap.add_argument("--comparator", default=None, metavar="FILE",
                    help="time the unfused torch path (rotation + varlen_attn) beside the fused op for every "
                         "workload and write them to FILE")
    ap.add_argument("--backward", default=None, metavar="FILE",
                    help="measure the backward of every workload and write them to FILE")
    ap.add_argument("--floor", action="store_true",
                    help="time the floor probe (one elementwise kernel reading q, k, v and writing an output) on "
                         "--workload's tensors instead of the op (also a --profile-calls driver option)")
    ap.add_argument("--positions", default=None, metavar="FILE",
                    help="time the position variant (fused_rope_attention_pos) beside the table op for every "
                         "workload and write them to FILE")
    ap.add_argument("--pos", action="store_true", help="profiling driver: run the position variant instead")
    ap.add_argument("--gather", default=None, metavar="FILE",
                    help="time window layers in image order through row_index (the window shuffle fused into the "
                         "kernel) beside the window-ordered call and the two hidden-state shuffles it removes; "
                         "write them to FILE")
    ap.add_argument("--drift", default=None, metavar="FILE",
                    help="run the 32-layer drift stack on --workload's grid and write the report to FILE")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (the op shards by head or "
              "segment with no exchange between GPUs).  Run with --gpus 1.", file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    dev = torch.device("cuda:0")
    flush = torch.ones(FLUSH_BYTES, dtype=torch.uint8, device=dev)
    if args.profile_calls:
        return profile_driver(args, flush, dev)
    if args.comparator:
        rows = []
        for name in WORKLOADS:
            r = run_comparator(name, max(10, args.steps // 2), max(3, args.warmup // 2), flush, dev)
            rows.append(r)
            print(f"[bench] comparator {name}: " + ", ".join(f"{k} {v:.4g}" if isinstance(v, float) else f"{k} {v}"
                                                          for k, v in r.items() if k not in ("workload", "note")),
                  file=sys.stderr, flush=True)
        with open(args.comparator, "w") as f:
            json.dump(rows, f, indent=1)
        return 0
    if args.positions:
        rows = []
        for name in WORKLOADS:
            r = run_positions(name, max(10, args.steps // 2), max(3, args.warmup // 2), flush, dev)
            rows.append(r)
            print(f"[bench] positions {name}: tables {r['tables_cold_us']:.1f} us, positions "
                  f"{r['positions_cold_us']:.1f} us ({r['positions_over_tables']:.3f}x), max-abs diff "
                  f"{r['max_abs_diff']:.2e}", file=sys.stderr, flush=True)
        with open(args.positions, "w") as f:
            json.dump(rows, f, indent=1)
        return 0
    if args.gather:
        rows = []
        for name in ("cfg0", "cfg1", "cfg2w", "cfg3"):
            r = run_gather(name, max(10, args.steps // 2), max(3, args.warmup // 2), flush, dev)
            rows.append(r)
            print(f"[bench] gather {name}: " + ", ".join(f"{k} {v:.4g}" for k, v in r.items()
                                                        if isinstance(v, float)), file=sys.stderr, flush=True)
        with open(args.gather, "w") as f:
            json.dump(rows, f, indent=1)
        return 0
    if args.backward:
        rows = []
        for name in WORKLOADS:
            r = run_backward(name, max(10, args.steps // 2), max(3, args.warmup // 2), flush, dev)
            rows.append(r)
            print(f"[bench] backward {name}: cold {r['cold_median_us']:.1f} us, warm {r['warm_us']:.1f} us, "
                  f"{r['roofline']['frac'] * 100:.1f}% of {r['roofline']['bound']}", file=sys.stderr, flush=True)
        with open(args.backward, "w") as f:
            json.dump(rows, f, indent=1)
        return 0
    if args.floor:
        w = WORKLOADS[args.workload]
        inp = make_inputs(w, seed=1234 + list(WORKLOADS).index(args.workload), device=dev)
        m = time_calls(floor_call(inp), args.steps, args.warmup, flush)
        nbytes = 4 * inp["q"].numel() * inp["q"].element_size()
        print(json.dumps({"floor": args.workload, "kernel": "torch.addcmul(q, k, v)", "bytes": nbytes,
                          **{k: round(v, 3) for k, v in m.items()},
                          "cold_GBps": round(nbytes / (m["cold_median_us"] * 1e-6) / 1e9, 1),
                          "warm_GBps": round(nbytes / (m["warm_us"] * 1e-6) / 1e9, 1),
                          "cold_frac_of_8TBps": round(nbytes / (m["cold_median_us"] * 1e-6) / 8e12, 4)}),
              flush=True)
        return 0
    if args.drift:
        rep = drift_stack(args.workload, dev, reference="gpu")
        with open(args.drift, "w") as f:
            json.dump(rep, f, indent=1)
        print(json.dumps({"drift": args.workload, "final_gpu_rel": rep["final_gpu_rel"],
                          "final_bf16_model_rel": rep["final_bf16_model_rel"]}), flush=True)
        return 0

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
        "roofline": dict(res["roofline"], traffic=committed_traffic(args.workload, res["kernel"])),
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
