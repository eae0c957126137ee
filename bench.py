"""Benchmark of the lgx Q8 hot path on one MI355X.

Workload: the Qwen2.5-1.5B MLP matmuls, gate and up
[8960 x 1536] and down [1536 x 8960], all Q8_0, with binary32 activations
~N(0,1).  One step = for each of the three matrices: quantise the activation
rows to Q8_0 and run the Q8 x Q8 product.  At M = 1 the three products are
one launch of the grouped GEMV (lgx_q8q8_gemv_quantize_group: the Q8_0
quantisation fused into each workgroup's prologue, the canonical range tree
applied in-workgroup); at M > 1 a quantise kernel + the int8-MFMA GEMM per
matrix.  Weights rotate over enough distinct copies (>= 2 x the 256 MB
Infinity Cache) that every step streams them from HBM.

Headline `value`: algorithmic GB/s of the M = 1 step (weights + scales +
activations + outputs, each counted once).  `roofline` is the dominant kernel
(lgx_k_q8_gemv_grp16 for this group: the step is that one launch), its
average duration taken from HIP events around the K un-instrumented
back-to-back launches of the timed region, on the stream they run on (so it
can never exceed the step time; the per-dispatch event figure is reported
beside it as a diagnostic).  Launches are queued behind a device-side sleep
before the timed region opens, so the step time is the device's, not the
Python loop's.

`config0`: one Q8_0 GEMV [4864 x 896], binary32 x
(lgx_q8_gemv_f32) and the int-dot form (lgx_q8q8_gemv_quantize: Q8_0 of x
fused), per launch over > 512 MB of rotating weight copies.

The M sweep (1, 8, 32, 64) is reported alongside, with its int8 MFMA
utilisation (the M x N x K block-dot work against the dense int8 peak): at
these M the products are HBM- and epilogue-bound, far from the MFMA
roofline.  `cpu_baseline` times the CPU oracle (a port: the reference has no
CPU implementation of this path) on a bounded sample of the same step, on all
of its threads and on one.

`decode_attention`: the split-KV decode attention
alone, B = 16, 12 query / 2 KV heads, head_dim 128, at L = 512, 4096, 32768
and ragged lengths, per call against the HBM peak (K/V pages rotated past the
Infinity Cache).

The decode part (BASELINE.json configs 3 and 4) builds the seeded
random-init Qwen2.5-0.5B- and 7B-shaped Q8_0 models on the device, prefills a
random prompt for every sequence, and times the 64 greedy decode steps
(`qwen_decode`: tokens/s, and the step's algorithmic bytes -- weights,
lm_head, K/V cache read and append -- against the HBM peak).

    python bench.py [--gpus 1] [--steps 50] [--warmup 5] [--decode config3,config4]
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
INT8_MFMA_PEAK_TOPS = 5000.0   # dense int8 MFMA, MI355X datasheet
F16_MFMA_PEAK_TFLOPS = 2500.0  # dense binary16 MFMA, MI355X datasheet
# the kernels the grouped M = 1 launch may use (LGX_GEMV=whole selects the
# whole-K forms); the one with the most dispatches in the timed pass is reported
DOMINANT = ("lgx_k_q8_gemv_grp4", "lgx_k_q8_gemv_grp8", "lgx_k_q8_gemv_grp16",
            "lgx_k_q8_gemv_wg4", "lgx_k_q8_gemv_wg8", "lgx_k_q8_gemv_wg16")
DOMINANT_USED = DOMINANT[2]
# HBM bytes per dispatch of the grouped config-1 launch, from rocprofv3 --pmc
# FETCH_SIZE and WRITE_SIZE passes of this script (--copy-calibration): the
# counters scaled by what they read for a plain 256 MiB device copy (FETCH_SIZE
# x 2.0, WRITE_SIZE x 1.0); profiles/q8_gemv_grouped_config1.md.
TRAFFIC_BYTES = (21710.5 * 2.0 + 76.0) * 1024
MALL_BYTES = 256 << 20
SHAPES = (("gate", 8960, 1536), ("up", 8960, 1536), ("down", 1536, 8960))


def q8_weight_bytes(n, k):
    return n * k + 2 * n * (k // 32)


def step_bytes(m):
    """Algorithmic bytes of one step at m rows: weights + fp32 activations in
    + fp32 outputs (the Q8 activation copy is an intermediate)."""
    return sum(q8_weight_bytes(n, k) + 4 * m * (k + n) for _, n, k in SHAPES)


def gemv_launch_bytes():
    """Algorithmic bytes of the grouped lgx_k_q8_gemv_grp16 launch of one M = 1
    step: the three Q8_0 matrices, their binary32 activations and outputs."""
    return step_bytes(1)


_SM_GAMMA = 0x9E3779B97F4A7C15


def _sm_mix(z):
    """SplitMix64 finaliser on a numpy uint64 array (wrapping arithmetic)."""
    import numpy as np

    z = np.asarray(z, np.uint64)
    z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
    z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return z ^ (z >> np.uint64(31))


def splitmix_stream(seed, stream, n):
    """Elements 0..n-1 of SplitMix64 stream `stream` of `seed`: element i is
    mix(base + (i + 1) * gamma), base = mix(seed + gamma) ^
    mix((stream + 1) * 0xD1B54A32D192ED03) -- the generator convention of the
    model's tensors (after crates/logicaffeine_runtime/src/seed.rs)."""
    import numpy as np

    with np.errstate(over="ignore"):
        base = (_sm_mix(np.uint64((seed + _SM_GAMMA) % 2**64)) ^
                _sm_mix(np.uint64(((stream + 1) * 0xD1B54A32D192ED03) % 2**64)))
        i = np.arange(1, n + 1, dtype=np.uint64)
        return _sm_mix(base + i * np.uint64(_SM_GAMMA))


def config1_inputs(seed=1):
    """Config 1's Q8_0 weights from the seed-1 SplitMix64 streams, one stream
    pair per matrix: quants uniform on [-127, 127] by the multiply-high map
    of the top 32 bits, scales |N(0, 0.02)| / 127 by Box-Muller (binary64)
    on draws 2i and 2i + 1, rounded to binary16.  Host arrays, shared by the
    GPU leg and the CPU baseline."""
    import numpy as np

    out = {}
    for j, (name, n, k) in enumerate(SHAPES):
        u = splitmix_stream(seed, 10 + 2 * j, n * k)
        qs = ((((u >> np.uint64(32)) * np.uint64(255)) >> np.uint64(32)).astype(np.int32) - 127)
        qs = qs.astype(np.int8).reshape(n, k)
        z = splitmix_normal_f32(seed, 11 + 2 * j, (n * (k // 32),)).astype(np.float64)
        d = (np.abs(0.02 * z) / 127.0).astype(np.float32).astype(np.float16).view(np.uint16)
        out[name] = (qs, d.reshape(n, k // 32))
    return out


def build_sets(ctx, torch, nsets, inputs):
    base = {name: ctx.q8_matrix(*inputs[name]) for name, _, _ in SHAPES}
    import logicaffeine_amd as lgx

    sets = [base]
    for _ in range(nsets - 1):
        sets.append({name: lgx.Q8Matrix(W.qs.clone(), W.d.clone(), W.n, W.k)
                     for name, W in base.items()})
    torch.cuda.synchronize()
    return sets


def run_step(ctx, sets, i, acts, m):
    W = sets[i % len(sets)]
    if m == 1:
        # the three products in one launch of the grouped GEMV
        ctx.q8q8_gemv_quantize_group([W[name] for name, _, _ in SHAPES],
                                     [acts[name][0][0] for name, _, _ in SHAPES],
                                     [acts[name][3][0] for name, _, _ in SHAPES])
        return
    # quantisation, products and range trees of the three matrices in three
    # launches of the grouped M > 1 product
    ctx.q8_gemm_quantize_group([W[name] for name, _, _ in SHAPES],
                               [acts[name][0] for name, _, _ in SHAPES],
                               [acts[name][3] for name, _, _ in SHAPES])


def splitmix_normal_f32(seed, stream, shape):
    """N(0, 1) binary32 values by Box-Muller (binary64) on draws 2i, 2i + 1 of
    a SplitMix64 stream."""
    import numpy as np

    n = int(np.prod(shape))
    u = splitmix_stream(seed, stream, 2 * n)
    u1 = ((u[0::2] >> np.uint64(11)) + np.uint64(1)).astype(np.float64) * 2.0**-53
    u2 = (u[1::2] >> np.uint64(11)).astype(np.float64) * 2.0**-53
    return (np.sqrt(-2.0 * np.log(u1)) * np.cos(6.283185307179586 * u2)).astype(np.float32).reshape(shape)


def make_acts(ctx, torch, m):
    """The step's activations: rows of the seed-1 streams 20, 21, 22 (the
    CPU baseline's x is row 0 of the same streams)."""
    acts = {}
    for j, (name, n, k) in enumerate(SHAPES):
        x = ctx.to_device(splitmix_normal_f32(1, 20 + j, (m, k)))
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
        stats = [ctx.kernel_stats(name) for name in DOMINANT]
        n, tot = sum(st[0] for st in stats), sum(st[1] for st in stats)
        gemv_ms = tot / max(n, 1)
        global DOMINANT_USED
        DOMINANT_USED = DOMINANT[max(range(len(stats)), key=lambda i: stats[i][0])]
    return ms, gemv_ms


def cpu_model_name():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(inputs, seconds=12.0, copies=4):
    """The CPU oracle's canonical Q8 x Q8 step (quantise + 3 matmuls, M = 1)
    on the GPU leg's seed-1 weights, rotating over `copies` copies of them
    (176 MB, past the host's last-level cache, so the weights stream from
    DRAM as the GPU leg's stream from HBM), on all the oracle's OpenMP
    threads, then on one."""
    import numpy as np

    from oracle import oracle as orc

    xs = {name: splitmix_normal_f32(1, 20 + j, (1, k)) for j, (name, _, k) in enumerate(SHAPES)}
    sets = [[(inputs[name][0].copy(), inputs[name][1].copy(), xs[name]) for name, _, _ in SHAPES]
            for _ in range(copies)]

    def run(budget):
        orc.q8_gemm(*sets[0][0][:2], *orc.quantize_q8_0(sets[0][0][2]))  # warm (threads, pages)
        t0 = time.perf_counter()
        reps = 0
        while True:
            for qs, d, x in sets[reps % copies]:
                xq, xd = orc.quantize_q8_0(x)
                orc.q8_gemm(qs, d, xq, xd)
            reps += 1
            el = time.perf_counter() - t0
            if el >= budget:
                return reps, el

    threads = orc.max_threads()
    reps, el = run(seconds)
    orc.set_threads(1)
    try:
        reps1, el1 = run(seconds / 2)
    finally:
        orc.set_threads(threads)
    return {
        "value": round(step_bytes(1) * reps / el / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "value_1core": round(step_bytes(1) * reps1 / el1 / 1e9, 3),
        "cpu_model": cpu_model_name(),
        "sample": f"config-1 M=1 steps (quantise + gate/up/down Q8xQ8, canonical schedule) on "
                  f"the seed-1 SplitMix64 weights, {copies} copies rotating "
                  f"({copies * sum(q8_weight_bytes(n, k) for _, n, k in SHAPES) / 1e6:.0f} MB): "
                  f"{reps} in {el:.1f} s on {threads} OpenMP threads, {reps1} in {el1:.1f} s "
                  f"on 1",
    }


CONFIG0_SHAPE = (4864, 896)


def config0_bench(ctx, torch, launches=400, seed=0):
    """One Q8_0 GEMV [4864 x 896] per launch (config 0): lgx_q8_gemv_f32
    (binary32 x) and lgx_q8q8_gemv_quantize (x quantised to Q8_0 in the
    prologue), over enough weight copies (> 2 x the 256 MB Infinity Cache)
    that every launch streams from HBM; HIP events around the back-to-back
    launches, queued behind a device-side sleep."""
    import numpy as np

    import logicaffeine_amd as lgx

    n, k = CONFIG0_SHAPE
    wbytes = q8_weight_bytes(n, k)
    nbytes = wbytes + 4 * (k + n)
    ncopy = -(-2 * MALL_BYTES // wbytes)
    rng = np.random.default_rng(seed)
    qs = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
    d = (np.abs(rng.normal(0.0, 0.02, size=(n, k // 32))) / 127.0).astype(np.float16)
    W0 = ctx.q8_matrix(qs, d.view(np.uint16))
    Ws = [W0] + [lgx.Q8Matrix(W0.qs.clone(), W0.d.clone(), n, k) for _ in range(ncopy - 1)]
    x = torch.from_numpy(rng.standard_normal(k).astype(np.float32)).to(ctx.dev)
    y = torch.empty(n, dtype=torch.float32, device=ctx.dev)
    out = {"shape": [n, k], "bytes_per_launch": nbytes, "copies": ncopy,
           "working_set_MB": round(ncopy * wbytes / 1e6, 1)}
    for name, call, kern in (
            ("f32", lambda W: ctx.q8_gemv_f32(W, x, y=y), "lgx_k_q8_gemv_f32"),
            ("int_dot", lambda W: ctx.q8q8_gemv_quantize(W, x, y=y), "lgx_k_q8_gemv_grp4")):
        for i in range(2 * ncopy):
            call(Ws[i % ncopy])
        torch.cuda.synchronize()
        t = time.perf_counter()
        call(Ws[0])
        host_ms = (time.perf_counter() - t) * 1e3
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        queue_ahead(torch, 2.0 * host_ms * launches + 5.0)
        e0.record()
        for i in range(launches):
            call(Ws[i % ncopy])
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) / launches * 1e3
        out[name] = {"kernel": kern, "us_per_launch": round(us, 3),
                     "GB_s": round(nbytes / us / 1e3, 1),
                     "frac": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4)}
    del Ws, W0
    torch.cuda.empty_cache()
    return out


SUSTAINED_SHAPE = (152064, 3584)   # Qwen2.5-7B lm_head as a Q8_0 matrix (579 MB)


def sustained_gemv(ctx, torch, iters=60):
    """Fused-quantise M = 1 GEMV streaming one large Q8_0 matrix (two copies
    alternate, > 2 x the Infinity Cache), HIP events around back-to-back
    launches."""
    import numpy as np

    import logicaffeine_amd as lgx

    n, k = SUSTAINED_SHAPE
    rng = np.random.default_rng(11)
    qs = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
    d = (np.abs(rng.normal(0.0, 0.02, size=(n, k // 32))) / 127.0).astype(np.float16)
    W0 = ctx.q8_matrix(qs, d.view(np.uint16))
    Ws = [W0, lgx.Q8Matrix(W0.qs.clone(), W0.d.clone(), n, k)]
    x = torch.randn(k, device=ctx.dev)
    y = torch.empty(n, device=ctx.dev)
    for i in range(4):
        ctx.q8q8_gemv_quantize(Ws[i % 2], x, y=y)
    torch.cuda.synchronize()
    ctx.kernel_timing(True)
    ctx.q8q8_gemv_quantize(Ws[0], x, y=y)
    torch.cuda.synchronize()
    ctx.kernel_timing(False)
    name = max(DOMINANT, key=lambda nm: ctx.kernel_stats(nm)[0])
    # back-to-back launches, HIP events around them
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    queue_ahead(torch, 1.0 * iters + 5.0)
    e0.record()
    for i in range(iters):
        ctx.q8q8_gemv_quantize(Ws[i % 2], x, y=y)
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) / iters * 1e3
    nbytes = q8_weight_bytes(n, k) + 4 * (k + n)
    del Ws, W0
    torch.cuda.empty_cache()
    return {"shape": [n, k], "kernel": name, "us_per_launch": round(us, 2),
            "GB_s": round(nbytes / us / 1e3, 1), "frac": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4)}


def kernel_probe_config4(torch, iters=20):
    """The config-4 decode step's two dominant kernels alone, at the shapes the
    step runs them (for counter passes, which cannot run beside the resident
    27 GB model): the tiled Q8 product at M = 64 with 64 activation rows per
    workgroup (lgx_k_q8_gemm_tiled64) for gate|up [37888 x 3584] and down
    [3584 x 18944], and the d = 128 decode attention chunk kernel
    (lgx_k_attn_chunk_d128_g7) at B = 64, 28 / 4 heads, context 4128.  Weights
    and K/V pages rotate over two copies (> the Infinity Cache per pass).
    Returns per-launch times from HIP events attached to each dispatch."""
    import numpy as np

    import logicaffeine_amd as lgx

    os.environ["LGX_GEMM_TILED_ROWS"] = "64"
    ctx = lgx.Context(0)
    rng = np.random.default_rng(4)
    out = {}
    m = 64
    for name, n, k in (("gate_up", 37888, 3584), ("down", 3584, 18944)):
        qs = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
        d = (np.abs(rng.normal(0.0, 0.02, size=(n, k // 32))) / 127.0).astype(np.float16)
        W0 = ctx.q8_matrix(qs, d.view(np.uint16))
        Ws = [W0, lgx.Q8Matrix(W0.qs.clone(), W0.d.clone(), n, k)]
        xq = ctx.to_device(rng.integers(-127, 128, size=(m, k), dtype=np.int8))
        xd = ctx.to_device((np.abs(rng.normal(0.0, 0.01, size=(m, k // 32)))).astype(np.float16).view(np.uint16))
        y = torch.empty((m, n), dtype=torch.float32, device=ctx.dev)
        ctx.kernel_timing(True)
        for i in range(iters):
            ctx.q8_gemm(Ws[i % 2], xq, xd, y=y)
        torch.cuda.synchronize()
        ctx.kernel_timing(False)
        cnt, tot = ctx.kernel_stats("lgx_k_q8_gemm_tiled64")
        nbytes = q8_weight_bytes(n, k) + m * k * (1 + 2 / 32) + 4 * m * n
        us = tot / max(cnt, 1) * 1e3
        out[name] = {"shape": [n, k], "m": m, "kernel": "lgx_k_q8_gemm_tiled64", "launches": cnt,
                     "us_per_launch": round(us, 2), "GB_s": round(nbytes / us / 1e3, 1)}
        del Ws, W0
        torch.cuda.empty_cache()
    B, hq, hkv, dh, L = 64, 28, 4, 128, 4128
    maxp = -(-L // 16)
    pages = [torch.randn((B * maxp, hkv, 16, dh), device=ctx.dev).to(torch.float16).view(torch.int16)
             for _ in range(4)]
    pt = torch.randperm(B * maxp, device=ctx.dev).to(torch.int32).reshape(B, maxp)
    lens = torch.full((B,), L, dtype=torch.int32, device=ctx.dev)
    q = torch.randn((B, hq, dh), device=ctx.dev)
    ctx.kernel_timing(True)
    for i in range(iters):
        ctx.gqa_decode_attn(q, pages[2 * (i % 2)], pages[2 * (i % 2) + 1], pt, lens, L)
    torch.cuda.synchronize()
    ctx.kernel_timing(False)
    cnt, tot = ctx.kernel_stats("lgx_k_attn_chunk_d128_g7")
    us = tot / max(cnt, 1) * 1e3
    kv = B * L * hkv * dh * 2 * 2
    out["attention"] = {"shape": {"batch": B, "hq": hq, "hkv": hkv, "head_dim": dh, "context": L},
                        "kernel": "lgx_k_attn_chunk_d128_g7", "launches": cnt,
                        "us_per_launch": round(us, 2), "GB_s": round(kv / us / 1e3, 1)}
    ctx.close()
    return out


ATTN_SHAPE = (16, 12, 2, 128)   # batch, query heads, KV heads, head_dim


def attention_bench(ctx, torch, iters=50, seed=2):
    """Config-2 decode attention over paged binary16 K/V in a random page
    order: the split-KV chunk kernel and the chunk merge of one call, at
    L = 512 / 4096 / 32768 and ragged lengths U[256, 32768].  The pages rotate
    over enough copies (>= 2 x the Infinity Cache) that every call streams
    them from HBM.  Algorithmic bytes per call: the attended K and V rows
    (sum of L x hkv x d x 2 B x 2) plus q and the output.  Times are per
    launch, from HIP events attached to each dispatch."""
    B, hq, hkv, d = ATTN_SHAPE
    chunk_k, merge_k = f"lgx_k_attn_chunk_d{d}_g{hq // hkv}", f"lgx_k_attn_combine_d{d}"
    g = torch.Generator(device=ctx.dev)
    g.manual_seed(seed)
    ragged = torch.randint(256, 32769, (B,), generator=g, device=ctx.dev).tolist()
    cases = [("L512", [512] * B), ("L4096", [4096] * B), ("L32768", [32768] * B),
             ("ragged", ragged)]
    res = {}
    for name, lens in cases:
        maxlen = max(lens)
        maxp = -(-maxlen // 16)
        npg = B * maxp
        page_bytes = npg * hkv * 16 * d * 2
        ncopy = max(1, -(-2 * MALL_BYTES // (2 * page_bytes)))
        sets = []
        for _ in range(ncopy):
            k = torch.randn((npg, hkv, 16, d), generator=g, device=ctx.dev).half().view(torch.int16)
            v = torch.randn((npg, hkv, 16, d), generator=g, device=ctx.dev).half().view(torch.int16)
            pt = torch.randperm(npg, generator=g, device=ctx.dev).to(torch.int32).reshape(B, maxp)
            sets.append((k, v, pt))
        sl = torch.tensor(lens, dtype=torch.int32, device=ctx.dev)
        q = torch.randn((B, hq, d), generator=g, device=ctx.dev)
        o = torch.empty((B, hq, d), dtype=torch.float32, device=ctx.dev)
        for i in range(3):
            k, v, pt = sets[i % ncopy]
            ctx.gqa_decode_attn(q, k, v, pt, sl, maxlen, out=o)
        torch.cuda.synchronize()
        ctx.kernel_timing(True)
        for i in range(iters):
            k, v, pt = sets[i % ncopy]
            ctx.gqa_decode_attn(q, k, v, pt, sl, maxlen, out=o)
        torch.cuda.synchronize()
        ctx.kernel_timing(False)
        (nc, tc), (nm, tm) = ctx.kernel_stats(chunk_k), ctx.kernel_stats(merge_k)
        chunk_us, merge_us = tc / max(nc, 1) * 1e3, tm / max(nm, 1) * 1e3
        kv = sum(lens) * hkv * d * 2 * 2
        nbytes = kv + 2 * B * hq * d * 4
        call_us = chunk_us + merge_us
        res[name] = {
            "kv_MiB": round(kv / 2**20, 1), "copies": ncopy,
            "chunk_kernel_us": round(chunk_us, 2), "merge_us": round(merge_us, 2),
            "GB_s": round(nbytes / call_us / 1e3, 1),
            "frac": round(nbytes / call_us / 1e3 / HBM_PEAK_GBS, 4),
            "chunk_kernel_GB_s": round(kv / chunk_us / 1e3, 1),
        }
        del sets, sl, q, o
        torch.cuda.empty_cache()
    return {"kernel": chunk_k, "shape": {"batch": B, "hq": hq, "hkv": hkv, "head_dim": d},
            "unit": "GB/s", "peak": HBM_PEAK_GBS, "cases": res}


DECODE_CONFIGS = {
    # BASELINE.json config 3 and 4: (shape, batch, prompt tokens, greedy steps)
    "config3": ("0.5b", 32, 2048, 64),
    "config4": ("7b", 64, 4096, 64),
}


def decode_bench(ctx, torch, key, seed=3, with_cpu=True):
    """Prefill a random prompt per sequence, then time the greedy decode
    steps (each: the whole model for B sequences + argmax + KV append)."""
    import logicaffeine_amd as lgx

    shape, B, P, steps = DECODE_CONFIGS[key]
    eager_steps = min(8, steps)
    cfg = lgx.qwen_shape(shape, B, P + 1 + steps + eager_steps)
    t = time.perf_counter()
    gm = lgx.Model(ctx, cfg, seed)
    torch.cuda.synchronize()
    create_s = time.perf_counter() - t
    g = torch.Generator(device=ctx.dev)
    g.manual_seed(seed)
    prompt = torch.randint(0, cfg["vocab"], (B, P), generator=g, device=ctx.dev,
                           dtype=torch.int32)
    t = time.perf_counter()
    tok = gm.prefill(prompt)
    torch.cuda.synchronize()
    prefill_s = time.perf_counter() - t
    pf_ops = lgx.prefill_valu_ops(cfg, B, P)
    print(f"[bench] {key}: model {create_s:.1f} s, prefill {B}x{P} in {prefill_s:.1f} s "
          f"({B * P / prefill_s:.0f} tok/s, {pf_ops / prefill_s / lgx.VALU_LANE_OPS_PEAK:.2f} of the VALU bound)",
          file=sys.stderr, flush=True)
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    gm.generate(tok, 1)                       # records the step's HIP graph (untimed)
    torch.cuda.synchronize()
    e0.record()
    gm.generate(tok, steps)                   # `steps` graph replays
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    # the same step launched kernel by kernel, for the launch-overhead figure
    e0.record()
    for _ in range(eager_steps):
        gm.decode_step(tok)
    e1.record()
    torch.cuda.synchronize()
    eager_ms = e0.elapsed_time(e1) / eager_steps
    ctxlen = P + 1 + (steps + 1) / 2.0        # mean attended tokens over the timed steps
    step_bytes_ = lgx.decode_step_bytes(cfg, B, ctxlen)
    gbs = step_bytes_ / (ms * 1e-3) / 1e9
    # sequence 0's cache and current token, for the CPU baseline at this context
    import numpy as np

    ctx_now = P + 1 + steps + eager_steps
    kv0 = None
    if with_cpu:
        maxp = -(-cfg["max_seq"] // 16)
        pt = gm.tensor_bytes("page_table").view(np.int32).reshape(B, maxp)
        kv0 = [[gm.kv_rows(layer, w, 0, ctx_now, pt) for w in (0, 1)]
               for layer in range(cfg["n_layers"])]
    tok0 = int(tok[0].item())
    prompt0 = prompt[0].cpu().numpy()
    # the same prompts again through the opt-in fast prefill (binary16 GEMMs
    # and flash attention; the last position exact)
    gm.reset()
    torch.cuda.synchronize()
    t = time.perf_counter()
    gm.set_prefill_mode(True)                 # one-time: binary16 weights, GEMM plans
    fast_setup_s = time.perf_counter() - t
    fast_runs = []
    for _ in range(2):                        # the first prefill after the setup, then again
        gm.reset()
        torch.cuda.synchronize()
        t = time.perf_counter()
        gm.prefill(prompt)
        torch.cuda.synchronize()
        fast_runs.append(time.perf_counter() - t)
    fast_s = fast_runs[1]
    print(f"[bench] {key}: fast prefill setup {fast_setup_s:.2f} s, prefill {B}x{P} in "
          f"{fast_runs[0]:.2f} / {fast_s:.2f} s ({B * P / fast_s:.0f} tok/s)",
          file=sys.stderr, flush=True)
    gm.close()
    torch.cuda.empty_cache()
    pf_int8 = lgx.prefill_int8_ops(cfg, B, P)
    f16_flops, f8_ops = lgx.prefill_fast_flops(cfg, B, P)
    # fast prefill: the time its MFMA work takes at the dense peaks (binary16
    # GEMMs and attention at the binary16 peak, the exact last position's
    # int8 products at the int8 peak) over its measured time
    mfma_frac = (f16_flops / (F16_MFMA_PEAK_TFLOPS * 1e12) + f8_ops / (INT8_MFMA_PEAK_TOPS * 1e12)) / fast_s
    out = {
        "model": f"random-init Qwen2.5-{shape.upper()}-shaped Q8_0 "
                 f"({'tied binary16' if cfg['tied'] else 'Q8_0'} lm_head)",
        "batch": B, "prompt": P, "steps": steps,
        "tokens_per_s": round(B / (ms * 1e-3), 1),
        "ms_per_step": round(ms, 4),
        "eager_ms_per_step": round(eager_ms, 4),
        "prefill_s": round(prefill_s, 2),
        "prefill": {"tokens_per_s": round(B * P / prefill_s, 1),
                    "roofline": {"bound": "valu", "achieved": round(pf_ops / prefill_s / 1e12, 2),
                                 "peak": round(lgx.VALU_LANE_OPS_PEAK / 1e12, 2),
                                 "unit": "T lane-op/s", "frac": round(pf_ops / prefill_s / lgx.VALU_LANE_OPS_PEAK, 4),
                                 "ops": pf_ops},
                    "mfma": {"int8_ops": pf_int8,
                             "achieved_TOPS": round(pf_int8 / prefill_s / 1e12, 1),
                             "peak_TOPS": INT8_MFMA_PEAK_TOPS,
                             "utilisation": round(pf_int8 / prefill_s / 1e12 / INT8_MFMA_PEAK_TOPS, 4)}},
        "prefill_fast_s": round(fast_s, 2),
        "prefill_fast": {"tokens_per_s": round(B * P / fast_s, 1),
                         "mode": "LGX_PREFILL_FAST: binary16 GEMMs (hipBLASLt) on dequantised "
                                 "weights, binary16 MFMA causal flash attention, the last "
                                 "position exact; the second prefill after the mode's setup",
                         "setup_s": round(fast_setup_s, 3),
                         "first_prefill_s": round(fast_runs[0], 3),
                         "mfma": {"f16_flops": f16_flops, "int8_ops": f8_ops,
                                  "achieved_f16_TFLOPS": round(f16_flops / fast_s / 1e12, 1),
                                  "f16_peak_TFLOPS": F16_MFMA_PEAK_TFLOPS,
                                  "int8_peak_TOPS": INT8_MFMA_PEAK_TOPS,
                                  "utilisation": round(mfma_frac, 4)}},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                     "bytes_per_step": int(step_bytes_),
                     "roofline_tokens_per_s": round(B * HBM_PEAK_GBS * 1e9 / step_bytes_, 1)},
    }
    print(f"[bench] {key}: {out['tokens_per_s']} tok/s, {ms:.3f} ms/step (graph), "
          f"{eager_ms:.3f} ms/step (eager), {gbs:.0f} GB/s",
          file=sys.stderr, flush=True)
    if with_cpu:
        out["cpu_baseline"] = cpu_decode_baseline(key, cfg, seed, kv0, ctx_now, tok0, prompt0)
    return out


# prompt tokens of sequence 0 the CPU oracle prefills for its prefill figure
PREFILL_SAMPLE = {"config3": 1024, "config4": 512}


def cpu_decode_baseline(key, cfg, seed, kv0, ctx_now, tok0, prompt0, seconds=8.0):
    """The CPU oracle model (a port; exact canonical arithmetic) on sequence 0
    of the benchmark.  Prefill: the first tokens of its prompt, timed on all
    of the oracle's threads (a bounded sample: PREFILL_SAMPLE tokens) and on
    one (an eighth of them).  Decode at the benchmark's context: the device's
    prefilled cache of that sequence (bit-identical to the oracle's, which the
    GPU tests check) is loaded into the oracle, then greedy steps are timed
    for `seconds` on all of its threads and for seconds / 2 on one."""
    import numpy as np

    from oracle import oracle as orc

    shape = DECODE_CONFIGS[key][0]
    ocfg = dict(cfg, max_batch=1, max_seq=ctx_now + 64)
    om = orc.Model(ocfg, seed)
    threads = orc.max_threads()
    npf = PREFILL_SAMPLE[key]

    def prefill(n):
        om.set_seq_len(0, 0)
        t0 = time.perf_counter()
        om.prefill([0], np.ascontiguousarray(prompt0[None, :n], np.int32))
        return time.perf_counter() - t0

    pf_el = prefill(npf)
    orc.set_threads(1)
    try:
        pf_el1 = prefill(npf // 8)
    finally:
        orc.set_threads(threads)
    for layer, (k, v) in enumerate(kv0):
        om.load_kv(layer, 0, 0, k)
        om.load_kv(layer, 1, 0, v)
    om.set_seq_len(0, ctx_now)

    def run(budget, cap):
        nxt = np.array([tok0], np.int32)
        t0 = time.perf_counter()
        n = 0
        while n < cap:
            nxt = om.step(np.zeros(1, np.int32), nxt)
            n += 1
            if time.perf_counter() - t0 >= budget:
                break
        return n, time.perf_counter() - t0

    n, el = run(seconds, 32)
    om.set_seq_len(0, ctx_now)
    orc.set_threads(1)
    try:
        n1, el1 = run(seconds / 2, 16)
    finally:
        orc.set_threads(threads)
    om.close()
    return {"value": round(n / el, 3), "unit": "tokens/s", "cores": threads, "kind": "port",
            "value_1core": round(n1 / el1, 4), "cpu_model": cpu_model_name(),
            "sample": f"{shape} shape, sequence 0 of the batch at context {ctx_now} (device-"
                      f"prefilled cache loaded into the oracle), batch 1: {n} greedy steps in "
                      f"{el:.1f} s on {threads} threads, {n1} in {el1:.1f} s on 1",
            "prefill": {"value": round(npf / pf_el, 2), "unit": "tokens/s", "cores": threads,
                        "value_1core": round((npf // 8) / pf_el1, 3),
                        "sample": f"the first {npf} prompt tokens of sequence 0 prefilled by the "
                                  f"oracle (batched over positions) in {pf_el:.1f} s on {threads} "
                                  f"threads; {npf // 8} in {pf_el1:.1f} s on 1"}}


def decode_trace(torch, key, seed=3):
    """The decode benchmark's model and prompts, the exact prefill, then only
    graph-replayed greedy steps (one recording replay + `steps`): under a
    kernel trace, every dispatch after the last prefill kernel belongs to a
    graph-replayed step."""
    import logicaffeine_amd as lgx

    shape, B, P, steps = DECODE_CONFIGS[key]
    ctx = lgx.Context(0)
    cfg = lgx.qwen_shape(shape, B, P + 1 + steps + min(8, steps))
    gm = lgx.Model(ctx, cfg, seed)
    g = torch.Generator(device=ctx.dev)
    g.manual_seed(seed)
    prompt = torch.randint(0, cfg["vocab"], (B, P), generator=g, device=ctx.dev,
                           dtype=torch.int32)
    tok = gm.prefill(prompt)
    gm.generate(tok, 1)
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    gm.generate(tok, steps)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    gm.close()
    return {"workload": f"{key} decode B={B}, {P}-token prompts", "graph_steps": steps + 1,
            "ms_per_step": round(ms, 4), "tokens_per_s": round(B / (ms * 1e-3), 1)}


def prefill_probe(torch, mode, key="config4", seed=3):
    """One prefill of the decode benchmark's prompts (config 4: 64 x 4096) in
    the given mode (exact | fast), alone, for kernel traces of the prefill."""
    import logicaffeine_amd as lgx

    shape, B, P, steps = DECODE_CONFIGS[key]
    ctx = lgx.Context(0)
    cfg = lgx.qwen_shape(shape, B, P + 1 + steps + min(8, steps))
    gm = lgx.Model(ctx, cfg, seed)
    g = torch.Generator(device=ctx.dev)
    g.manual_seed(seed)
    prompt = torch.randint(0, cfg["vocab"], (B, P), generator=g, device=ctx.dev,
                           dtype=torch.int32)
    gm.set_prefill_mode(mode == "fast")
    torch.cuda.synchronize()
    t = time.perf_counter()
    gm.prefill(prompt)
    torch.cuda.synchronize()
    el = time.perf_counter() - t
    gm.close()
    return {"mode": mode, "workload": f"{key} prefill {B}x{P}", "seconds": round(el, 3),
            "tokens_per_s": round(B * P / el, 1)}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--decode", default="config3,config4",
                    help="decode configs to run (comma list; empty for none)")
    ap.add_argument("--kernel-probe", action="store_true",
                    help="only run the config-4 decode's tiled product and attention kernels "
                         "standalone (for counter passes) and print their timings")
    ap.add_argument("--prefill-probe", choices=["exact", "fast"],
                    help="only run one prefill of --probe-config in that mode and print its "
                         "time (for kernel traces of the prefill)")
    ap.add_argument("--probe-config", default="config4", choices=sorted(DECODE_CONFIGS))
    ap.add_argument("--decode-trace", choices=sorted(DECODE_CONFIGS),
                    help="only run that config's prefill and graph-replayed decode steps "
                         "(for kernel traces of the decode step)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run 4 plain 256 MiB device copies (HBM counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); "
              "the products would shard by output rows and the attention by (sequence, KV head), "
              "with no collective in the decode step", file=sys.stderr)
        sys.exit(2)

    import torch

    import logicaffeine_amd as lgx

    if args.kernel_probe:
        print(json.dumps({"config4_kernels": kernel_probe_config4(torch)}), flush=True)
        return
    if args.prefill_probe:
        print(json.dumps({"prefill_probe": prefill_probe(torch, args.prefill_probe,
                                                         args.probe_config)}), flush=True)
        return
    if args.decode_trace:
        print(json.dumps({"decode_trace": decode_trace(torch, args.decode_trace)}), flush=True)
        return
    ctx = lgx.Context(0)
    set_bytes = sum(q8_weight_bytes(n, k) for _, n, k in SHAPES)
    nsets = max(2, -(-2 * MALL_BYTES // set_bytes))
    inputs = config1_inputs(1)
    sets = build_sets(ctx, torch, nsets, inputs)
    print(f"[bench] {nsets} weight sets x {set_bytes / 1e6:.1f} MB rotating", file=sys.stderr,
          flush=True)

    ms1, gemv_ms = time_m(ctx, torch, sets, 1, args.steps, args.warmup, per_launch=True)
    print(f"[bench] M=1 {ms1 * 1e3:.1f} us/step, gemv {gemv_ms * 1e3:.2f} us/launch",
          file=sys.stderr, flush=True)
    ms1_plain, _ = time_m(ctx, torch, sets, 1, args.steps, args.warmup, per_launch=False)
    sweep = {}
    for m in (1, 8, 32, 64):
        ms = ms1_plain if m == 1 else time_m(ctx, torch, sets, m, args.steps, args.warmup)[0]
        # int8 MFMA work of the step: the M x N x K block dots (2 ops per MAC)
        tops = 2.0 * m * sum(n * k for _, n, k in SHAPES) / (ms * 1e-3) / 1e12
        sweep[str(m)] = {"ms_per_step": round(ms, 5),
                         "GB_s": round(step_bytes(m) / (ms * 1e-3) / 1e9, 1),
                         "tokens_s": round(m / (ms * 1e-3), 1),
                         "int8_TOPS": round(tops, 2),
                         "mfma_util": round(tops / INT8_MFMA_PEAK_TOPS, 5)}
        print(f"[bench] M={m}: {ms * 1e3:.1f} us/step {sweep[str(m)]['GB_s']} GB/s",
              file=sys.stderr, flush=True)

    value = step_bytes(1) / (ms1_plain * 1e-3) / 1e9
    per_launch = gemv_launch_bytes()
    if not gemv_ms:
        raise SystemExit("bench: no dispatch of the grouped GEMV kernels was timed")
    # the step is one launch of the dominant kernel: its average duration is
    # the un-instrumented back-to-back time of the timed region
    launch_ms = ms1_plain
    achieved = per_launch / (launch_ms * 1e-3) / 1e9
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
        "data": "synthetic, seed-1 SplitMix64 streams (int8 U[-127,127], d=|N(0,0.02)|/127 f16, "
                "x~N(0,1) f32)",
        "config": {
            "workload": "config1 Qwen2.5-1.5B MLP Q8_0 gate/up [8960x1536] + down [1536x8960], "
                        "M=1 (one grouped launch: fused quantise + whole-K Q8xQ8 GEMV of the "
                        "three matrices)",
            "rotating_weight_sets": nsets,
            "working_set_MB": round(nsets * set_bytes / 1e6, 1),
            "pct_hbm_peak": round(100 * value / HBM_PEAK_GBS, 1),
            "sweep_M": sweep,
        },
        "roofline": {
            "bound": "hbm",
            "kernel": DOMINANT_USED,
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": TRAFFIC_BYTES if DOMINANT_USED == "lgx_k_q8_gemv_grp16" else None,
            "avg_launch_us": round(launch_ms * 1e3, 3),
            "timing": "HIP events around the timed region's back-to-back launches (one per step)",
            "dispatch_event_us": round(gemv_ms * 1e3, 3),
            "bytes_per_launch": int(per_launch),
        },
    }
    assert launch_ms <= ms1_plain
    del sets
    torch.cuda.empty_cache()
    if args.copy_calibration:
        # reference kernel for the FETCH_SIZE / WRITE_SIZE counters: reads and
        # writes exactly 256 MiB each
        src = torch.empty(64 << 20, dtype=torch.float32, device=ctx.dev).fill_(1.0)
        dst = torch.empty_like(src)
        for _ in range(4):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
        torch.cuda.empty_cache()
    sustained = sustained_gemv(ctx, torch)
    print(f"[bench] sustained GEMV {SUSTAINED_SHAPE}: {sustained['us_per_launch']} us, "
          f"{sustained['GB_s']} GB/s", file=sys.stderr, flush=True)
    out["config"]["sustained_gemv_m1"] = sustained
    c0 = config0_bench(ctx, torch)
    print(f"[bench] config0 4864x896: f32 {c0['f32']['us_per_launch']} us "
          f"{c0['f32']['GB_s']} GB/s, int-dot {c0['int_dot']['us_per_launch']} us "
          f"{c0['int_dot']['GB_s']} GB/s", file=sys.stderr, flush=True)
    out["config0"] = c0
    attn = attention_bench(ctx, torch)
    print("[bench] config-2 decode attention: " + ", ".join(
        f"{k} {v['chunk_kernel_us'] + v['merge_us']:.1f} us {v['GB_s']} GB/s"
        for k, v in attn["cases"].items()), file=sys.stderr, flush=True)
    out["decode_attention"] = attn
    decode = {}
    for key in [k for k in args.decode.split(",") if k]:
        decode[key] = decode_bench(ctx, torch, key, with_cpu=not args.no_cpu)
    if decode:
        out["qwen_decode"] = decode
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(inputs, args.cpu_seconds)
    ctx.close()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
