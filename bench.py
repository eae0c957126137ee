"""Benchmark of the lgx Q8 hot path on one MI355X.

Workload: the Qwen2.5-1.5B MLP matmuls, gate and up
[8960 x 1536] and down [1536 x 8960], all Q8_0, with binary32 activations
~N(0,1).  One step = for each of the three matrices: quantise the activation
rows to Q8_0 and run the Q8 x Q8 product (M = 1: the dot4 GEMV with the
quantisation fused into its prologue; M > 1: quantise kernel + int8-MFMA
GEMM), plus the range-combine kernel where K spans more than one 32-block
range.  Weights rotate over enough distinct copies (>= 2 x the
256 MB Infinity Cache) that every step streams them from HBM.

Headline `value`: algorithmic GB/s of the M = 1 step (weights + scales +
activations + outputs, each counted once).  `roofline` is the dominant kernel
(lgx_k_q8_gemv_mfma_qx, the fused-quantise GEMV writing range partials),
timed per launch by HIP events attached to its own dispatch
(lgx_ctx_set_kernel_timing) on its stream, in a separate pass over the same
steps.  Launches are queued behind a device-side sleep before the timed
region opens, so the step time is the device's, not the Python loop's.  The M sweep
(1, 8, 32, 64) is reported alongside.  `cpu_baseline` times the CPU oracle
(a port: the reference has no CPU implementation of this path) on a bounded
sample of the same step.

    python bench.py [--gpus 1] [--steps 50] [--warmup 5]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
DOMINANT = "lgx_k_q8_gemv_mfma_qx"
MALL_BYTES = 256 << 20
SHAPES = (("gate", 8960, 1536), ("up", 8960, 1536), ("down", 1536, 8960))


def q8_weight_bytes(n, k):
    return n * k + 2 * n * (k // 32)


def step_bytes(m):
    """Algorithmic bytes of one step at m rows: weights + fp32 activations in
    + fp32 outputs (the Q8 activation copy is an intermediate)."""
    return sum(q8_weight_bytes(n, k) + 4 * m * (k + n) for _, n, k in SHAPES)


def gemv_launch_bytes(n, k):
    """Algorithmic bytes of one lgx_k_q8_gemv_mfma_qx launch: W + fp32 x +
    one fp32 range partial per row and range (= y with a single range)."""
    nr = -(-(k // 32) // 32)
    return q8_weight_bytes(n, k) + 4 * k + 4 * n * nr


def build_sets(ctx, torch, nsets, seed=1):
    import numpy as np

    rng = np.random.default_rng(seed)
    base = {}
    for name, n, k in SHAPES:
        qs = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
        d = (np.abs(rng.normal(0.0, 0.02, size=(n, k // 32))) / 127.0).astype(np.float16)
        base[name] = ctx.q8_matrix(qs, d.view(np.uint16))
    import logicaffeine_amd as lgx

    sets = [base]
    for _ in range(nsets - 1):
        sets.append({name: lgx.Q8Matrix(W.qs.clone(), W.d.clone(), W.n, W.k)
                     for name, W in base.items()})
    torch.cuda.synchronize()
    return sets


def run_step(ctx, sets, i, acts, m):
    W = sets[i % len(sets)]
    for name, n, k in SHAPES:
        x, xq, xd, y, part = acts[name]
        if m == 1:
            ctx.q8q8_gemv_quantize_partials(W[name], x[0], part=part)
            if part.dim() == 2:
                ctx.range_combine(part, y=y[0])
        else:
            ctx.quantize_q8_0(x, xq, xd)
            ctx.q8_gemm(W[name], xq, xd, y=y)


def make_acts(ctx, torch, m):
    acts = {}
    g = torch.Generator(device=ctx.dev)
    g.manual_seed(1234 + m)
    for name, n, k in SHAPES:
        x = torch.randn((m, k), generator=g, device=ctx.dev, dtype=torch.float32)
        xq = torch.empty((m, k), dtype=torch.int8, device=ctx.dev)
        xd = torch.empty((m, k // 32), dtype=torch.int16, device=ctx.dev)
        y = torch.empty((m, n), dtype=torch.float32, device=ctx.dev)
        nr = -(-(k // 32) // 32)
        part = torch.empty((nr, n), dtype=torch.float32, device=ctx.dev)
        acts[name] = (x, xq, xd, y, part if nr > 1 else y[0])
    return acts


_SLEEP_CYCLES_PER_MS = None


def queue_ahead(torch, ms):
    """Occupy the stream with a device-side spin of about `ms` so that the
    launches queued behind it run back to back."""
    global _SLEEP_CYCLES_PER_MS
    if _SLEEP_CYCLES_PER_MS is None:
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        torch.cuda._sleep(10_000_000)
        e1.record()
        torch.cuda.synchronize()
        _SLEEP_CYCLES_PER_MS = 10_000_000 / max(e0.elapsed_time(e1), 1e-3)
    torch.cuda._sleep(int(ms * _SLEEP_CYCLES_PER_MS))


def time_m(ctx, torch, sets, m, steps, warmup, per_launch=False):
    acts = make_acts(ctx, torch, m)
    for i in range(warmup):
        run_step(ctx, sets, i, acts, m)
    torch.cuda.synchronize()
    # host time to enqueue one step, to size the device-side queue-ahead
    t = time.perf_counter()
    run_step(ctx, sets, 0, acts, m)
    host_ms = (time.perf_counter() - t) * 1e3
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    if per_launch:
        ctx.kernel_timing(True)
    queue_ahead(torch, 2.0 * host_ms * steps + 5.0)
    t0.record()
    for i in range(steps):
        run_step(ctx, sets, warmup + i, acts, m)
    t1.record()
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / steps
    gemv_ms = None
    if per_launch:
        ctx.kernel_timing(False)
        n, tot = ctx.kernel_stats(DOMINANT)
        gemv_ms = tot / max(n, 1)
    return ms, gemv_ms


def cpu_baseline(seconds=12.0):
    """The CPU oracle's canonical Q8 x Q8 step (quantise + 3 matmuls, M = 1)."""
    import numpy as np

    from oracle import oracle as orc

    rng = np.random.default_rng(7)
    mats = []
    for _, n, k in SHAPES:
        qs = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
        d = (np.abs(rng.normal(0.0, 0.02, size=(n, k // 32))) / 127.0).astype(np.float16)
        x = rng.standard_normal((1, k)).astype(np.float32)
        mats.append((qs, d.view(np.uint16), x))
    orc.q8_gemm(*mats[0][:2], *orc.quantize_q8_0(mats[0][2]))  # warm (threads, pages)
    t0 = time.perf_counter()
    reps = 0
    while True:
        for qs, d, x in mats:
            xq, xd = orc.quantize_q8_0(x)
            orc.q8_gemm(qs, d, xq, xd)
        reps += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    return {
        "value": round(step_bytes(1) * reps / el / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": f"{reps} steps of config-1 M=1 (quantise + gate/up/down Q8xQ8, canonical "
                  f"schedule, OpenMP) in {el:.1f} s",
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); "
              "the path would shard by output rows, see DESIGN.md", file=sys.stderr)
        sys.exit(2)

    import torch

    import logicaffeine_amd as lgx

    ctx = lgx.Context(0)
    set_bytes = sum(q8_weight_bytes(n, k) for _, n, k in SHAPES)
    nsets = max(2, -(-2 * MALL_BYTES // set_bytes))
    sets = build_sets(ctx, torch, nsets)
    print(f"[bench] {nsets} weight sets x {set_bytes / 1e6:.1f} MB rotating", file=sys.stderr,
          flush=True)

    ms1, gemv_ms = time_m(ctx, torch, sets, 1, args.steps, args.warmup, per_launch=True)
    print(f"[bench] M=1 {ms1 * 1e3:.1f} us/step, gemv {gemv_ms * 1e3:.2f} us/launch",
          file=sys.stderr, flush=True)
    ms1_plain, _ = time_m(ctx, torch, sets, 1, args.steps, args.warmup, per_launch=False)
    sweep = {}
    for m in (1, 8, 32, 64):
        ms = ms1_plain if m == 1 else time_m(ctx, torch, sets, m, args.steps, args.warmup)[0]
        sweep[str(m)] = {"ms_per_step": round(ms, 5),
                         "GB_s": round(step_bytes(m) / (ms * 1e-3) / 1e9, 1),
                         "tokens_s": round(m / (ms * 1e-3), 1)}
        print(f"[bench] M={m}: {ms * 1e3:.1f} us/step {sweep[str(m)]['GB_s']} GB/s",
              file=sys.stderr, flush=True)

    value = step_bytes(1) / (ms1_plain * 1e-3) / 1e9
    per_launch = sum(gemv_launch_bytes(n, k) for _, n, k in SHAPES) / 3
    achieved = per_launch / (gemv_ms * 1e-3) / 1e9
    out = {
        "metric": "Q8 GEMV HBM GB/s (% peak); batched Qwen decode tokens/sec on 1 MI355X",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms1_plain, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (int8 U[-127,127], d=|N(0,0.02)|/127 f16, x~N(0,1) f32)",
        "config": {
            "workload": "config1 Qwen2.5-1.5B MLP Q8_0 gate/up [8960x1536] + down [1536x8960], "
                        "M=1 (fused quantise + Q8xQ8 GEMV per matrix, + range combine)",
            "rotating_weight_sets": nsets,
            "working_set_MB": round(nsets * set_bytes / 1e6, 1),
            "pct_hbm_peak": round(100 * value / HBM_PEAK_GBS, 1),
            "sweep_M": sweep,
        },
        "roofline": {
            "bound": "hbm",
            "kernel": DOMINANT,
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": None,
            "avg_launch_us": round(gemv_ms * 1e3, 3),
            "bytes_per_launch": int(per_launch),
        },
    }
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    ctx.close()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
