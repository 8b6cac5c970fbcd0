#!/usr/bin/env python3
"""Decode-attention benchmark on one MI355X.

Metric: decode-attention achieved HBM GB/s (% of the 8 TB/s
peak) + us/call at KV 512 / 8K / 32K.  Workload of `value`: config 2 -- one
qd_decode_attention call over 16 heads x 128 dims x 8192 fp16 KV rows in the
reference engine's [pos][16*128] cache layout.

A step is one call of the public C ABI over one layer.  Steps cycle through
enough layers (>= 1 GiB of K+V) that every call streams its rows from HBM, not
from the 256 MB Infinity Cache.  The timed loop runs natively
(libqdiy_bench.so) on torch's current stream between two HIP events; us/call
= elapsed / steps.  L=8192 is measured first, then the other lengths in
ascending order; each length allocates its own buffers.  achieved GB/s =
algorithmic bytes per call / us per call with B(L) = 8192 + 8192*L (Q in,
O out, K and V rows read once).

Warm-up: before the first timed region of each length, at least --warmup calls
and WARMUP_FLOOR_S of wall time of calls run, and the last ~2 ms of them are
queued without a host synchronisation, so the first timed call follows busy
GPU work.  (From an idle GPU, the first 20 calls ran ~8% slower per call than
the steady state, which a 20-step window would report.)  The warm-up that ran
is reported in config.warmup_run.

roofline: the dominant kernel of the call -- at every length of the bench on
MI355X the call's only kernel, the split scan with the merge inside it -- timed
live between two HIP events on the call's stream over `steps` launches
(qd_decode_attention_stage, scan stage) on the same rotated layers; achieved =
its algorithmic bytes (K and V rows and Q: 8192*L + 4096) / its mean duration
per launch.  config.scan_without_in_kernel_merge_us is the same plan's scan
kernel alone (a two-launch context's scan stage: plain partials, no merge);
with a separate merge kernel, config.merge_kernel_us times that kernel.
config.read_ceiling_us is a load-only kernel over the same layers in a
one-workgroup-per-CU launch shape: what one kernel streaming those bytes takes on
this box.  config.empty_kernel_us is an empty kernel of 16 workgroups launched
back to back: the dispatch floor any dependent launch pays.
config.read_sweep_L8192 times the same L=8192 bytes read by kernels of other
launch shapes (1, 2 or 4 waves per SIMD; 8-64 KB in flight per wave;
contiguous, grid-strided, per-head and head-group access patterns);
config.read_ceiling_best_us is the fastest of them, and
config.read_merge_floor_L8192 the fastest of them followed, in the same launch,
by the tagged hand-off of 16 partials per head group to one merger: what any
design that reads the bytes once and merges split partials in one launch could
reach on this box.

The CPU baseline is the repository's C restatement of the reference kernels
(oracle/) on the host cores of the same box, on a bounded sample of the same
workload.

Also measured and reported under `config`: config 4 (the fused QKV front end
followed by attention at L=2048) and config 5 (greedy decode of a random-init
Qwen-1.8B-shaped model through the engine: tokens/s, an estimate of the
attention share of a decode step, and the prefill time of the 127-token prompt
and of a 2048-token one, exact and with the projections on the matrix cores).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-e2e]
       python bench.py --only call|scan|merge|read|empty --kv L [--steps K]   (for rocprofv3)
       python bench.py --only prefill --kv T [--steps K]   (MFMA prefill attention of T tokens)
       python bench.py --only sweep --kv L [--steps K]     (read-ceiling sweep over launch shapes)
       python bench.py --only front [--steps K]            (config 4's three loops, for a profiler)
       python bench.py --only gemm --kv T [--gemm qkv,...] [--vendor]   (MFMA prefill products)
"""
from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "llm-inference-diy_amd")
for _p in (ROOT, PKG):
    if _p not in sys.path:
        sys.path.insert(0, _p)

H, D = 16, 128
HID = H * D
PEAK_GBPS = 8000.0
KV_LENS = (512, 8192, 16384, 32768)
HEADLINE_L = 8192
METRIC = "decode-attention achieved HBM GB/s (% of peak) + µs/call at KV 512/8K/32K"
WARMUP_FLOOR_S = 0.1     # wall time of calls before the first timed region of a length
WARMUP_TAIL_S = 0.002    # GPU time of calls queued, unsynchronised, right before a region


def traffic_file(L: int) -> str:
    """rocprofv3 FETCH_SIZE / WRITE_SIZE summary of one call at L (profiles/)."""
    return os.path.join(ROOT, "profiles", f"traffic_decode_attention_L{L}.json")


def algo_bytes(L: int) -> int:
    return 2 * H * D * 2 + 2 * H * L * D * 2     # Q + O, K + V


def scan_bytes(L: int) -> int:
    return H * D * 2 + 2 * H * L * D * 2         # Q, K + V: what the scan kernel must read


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def bench_lib():
    import qdiy

    qdiy.load()
    path = os.path.join(PKG, "lib", "libqdiy_bench.so")
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is not built: run python llm-inference-diy_amd/build.py")
    lib = ctypes.CDLL(path)
    vp, i, ll = ctypes.c_void_p, ctypes.c_int, ctypes.c_longlong
    lib.qd_bench_decode_attention.argtypes = [vp, vp, vp, vp, vp, ll, ll, i, i, i, i, i, i, vp]
    lib.qd_bench_read_ceiling.argtypes = [vp, vp, ll, ll, i, i, i, vp, vp]
    lib.qd_bench_empty.argtypes = [i, i, vp]
    lib.qd_bench_read_sweep.argtypes = [vp, vp, ll, i, i, i, i, i, i, i, i, i, vp, vp]
    lib.qd_bench_read_merge.argtypes = [vp, vp, ll, i, i, i, i, i, i, i, i, i, vp, vp, ctypes.c_uint,
                                        vp, vp]
    lib.qd_bench_attn_front.argtypes = [vp, vp, vp, vp, vp, vp, vp, vp, ll, ll, i, i, i, i, i, i, vp]
    return lib


def warm_up(run, warmup: int, floor_s: float = WARMUP_FLOOR_S):
    """Runs max(warmup, 1) calls, then host-synchronised chunks of ~10 ms until
    floor_s of wall time has passed, then queues ~WARMUP_TAIL_S of calls without
    synchronising: the caller records its first event behind them, so the GPU is
    busy right up to the timed region.  Returns (calls run, wall ms)."""
    import torch

    t0 = time.perf_counter()
    n = max(1, warmup)
    run(n)
    torch.cuda.synchronize()
    per_call = (time.perf_counter() - t0) / n
    while time.perf_counter() - t0 < floor_s:
        chunk = max(1, int(0.01 / max(per_call, 1e-6)))
        t1 = time.perf_counter()
        run(chunk)
        torch.cuda.synchronize()
        per_call = (time.perf_counter() - t1) / chunk
        n += chunk
    tail = max(20, int(WARMUP_TAIL_S / max(per_call, 1e-6)))
    run(tail)
    return n + tail, (time.perf_counter() - t0) * 1e3


def kv_layers(L: int):
    """Synthetic config-2/3 inputs at L: (n_layers, K, V, Q, O), with enough layers
    (>= 1 GiB of K+V) that a call reading layer i % n_layers streams from HBM."""
    import torch

    layer_bytes = 2 * L * HID * 2
    n_layers = max(3, math.ceil((1 << 30) / layer_bytes))
    gen = torch.Generator(device="cuda")
    gen.manual_seed(1000 + L)
    kscale = 0.5 if L == HEADLINE_L else 1.0       # config 2 scales K by 0.5
    kc = torch.empty(n_layers * L * HID, dtype=torch.float16, device="cuda")
    vc = torch.empty_like(kc)
    kc.normal_(0.0, kscale, generator=gen)
    vc.normal_(0.0, 1.0, generator=gen)
    q = torch.empty(n_layers * HID, dtype=torch.float16, device="cuda").normal_(generator=gen)
    return n_layers, kc, vc, q, torch.empty_like(q)


def attention_loop(lib, ctx, L, n_layers, kc, vc, q, out, sh, kind, splits=0):
    """fn(iters, layers=n_layers): back-to-back calls from the native loop; kind is the
    loop's variant (0 auto, 1 fused, 2 split, 3 scan kernel only, 4 merge kernel only)."""
    import qdiy

    def fn(iters, layers=n_layers):
        rc = lib.qd_bench_decode_attention(ctx._h, q.data_ptr(), kc.data_ptr(), vc.data_ptr(),
                                           out.data_ptr(), HID, L * HID, layers, L, H, iters,
                                           kind, splits, sh)
        if rc != 0:
            raise RuntimeError(f"bench loop failed: {qdiy.load().qd_last_error().decode()}")
    return fn


def read_loop(lib, L, n_layers, kc, vc, sh):
    """fn(iters): the read-ceiling kernel over the same layers' K and V rows, in the
    split scan's launch shape (256 workgroups of 256 threads)."""
    import torch

    sink = torch.empty(256 * 16, dtype=torch.uint8, device="cuda")

    def fn(iters):
        if lib.qd_bench_read_ceiling(kc.data_ptr(), vc.data_ptr(), L * HID * 2, L * HID * 2,
                                     n_layers, 256, iters, sink.data_ptr(), sh) != 0:
            raise RuntimeError("read-ceiling launch failed")
    return fn


# Read-ceiling sweep shapes: (threads per workgroup, workgroups per CU) -> 1, 2 or 4
# waves per SIMD on 256 CUs; loads per lane per stream (K and V) in flight: 8, 16,
# 32 or 64 KB per wave at 2, 4, 8, 16; patterns: 0 contiguous per workgroup, 1 the
# scan's per-head 256-byte slices, 2 grid-strided contiguous chunks, 3 per-head slices
# with the rows dealt to the splits in blocks of one workgroup load round, 4-6
# workgroups over 4, 8 or 16 heads reading 1, 2 or 4 KB of each row; 7 pattern 3 with each
# wave's next tile in flight while it folds one.
SWEEP_SHAPES = [(256, 1), (512, 1), (256, 2), (1024, 1), (512, 2), (256, 4)]
SWEEP_LOADS = (2, 4, 8, 16)
SWEEP_PATTERNS = {0: "contiguous", 1: "per-head slices", 2: "grid-strided chunks",
                  3: "per-head slices, split-interleaved blocks", 4: "4-head (1 KB) row slices",
                  5: "8-head (2 KB) row slices", 6: "whole rows (16 heads)",
                  7: "per-head slices, split-interleaved blocks, next tile in flight"}


def read_sweep(lib, L, n_layers, kc, vc, sh, steps, num_cus):
    """Times the read-sweep kernels over the same layers' K and V rows: us per launch,
    back to back, for every shape in SWEEP_SHAPES x SWEEP_LOADS x SWEEP_PATTERNS.
    Returns {name: us} and the best (name, us)."""
    import torch

    sink = torch.empty(65536 * 16, dtype=torch.uint8, device="cuda")
    stream = torch.cuda.current_stream()
    out = {}
    for threads, per_cu in SWEEP_SHAPES:
        grid = num_cus * per_cu
        for loads in SWEEP_LOADS:
            if threads == 1024 and loads == 16:
                continue
            for pat in SWEEP_PATTERNS:
                def fn(iters):
                    return lib.qd_bench_read_sweep(kc.data_ptr(), vc.data_ptr(), L * HID * 2, L, HID * 2,
                                                   H, n_layers, threads, loads, pat, grid, iters,
                                                   sink.data_ptr(), sh)
                rc = fn(max(20, n_layers))
                if rc == 1:
                    continue          # shape does not divide this length's rows
                if rc != 0:
                    raise RuntimeError(f"read sweep launch failed ({threads}, {grid}, {loads}, {pat})")
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record(stream)
                fn(steps)
                e1.record(stream)
                e1.synchronize()
                out[f"t{threads}_g{grid}_u{loads}_p{pat}"] = round(e0.elapsed_time(e1) * 1e3 / steps, 3)
    best = min(out.items(), key=lambda kv: kv[1])
    log(f"[bench] read sweep L={L}: best {best[0]} {best[1]:.2f} us "
        f"({2 * L * HID * 2 / best[1] / 1e3:.0f} GB/s) over {len(out)} shapes")
    return out, best


def read_merge_floor(lib, L, n_layers, kc, vc, sh, steps, sweep):
    """Read-and-merge floor (qd_bench_read_merge): for the sweep's three fastest
    shapes and the fastest per-head-slice shapes of one workgroup per CU
    (patterns 1, 3 and 7 at 256 workgroups: one head per workgroup, 16 splits
    per head, as the attention plans run), the read followed by a 16-partial
    tagged hand-off to one merging workgroup per head group in the same launch
    -- what any design that reads the bytes once and merges its splits in the
    launch could reach with that read.  Returns ({shape: {"read": us,
    "read_merge": us}}, (best per-head shape, its read_merge us))."""
    import torch

    slots = torch.zeros(16 * 64 * 144 * 2, dtype=torch.float32, device="cuda")
    mout = torch.zeros(16 * 128, dtype=torch.float32, device="cuda")
    stale = torch.zeros(1, dtype=torch.int32, device="cuda")
    stream = torch.cuda.current_stream()
    ranked = sorted(sweep.items(), key=lambda kv: kv[1])
    names = [k for k, _ in ranked[:3]]
    for pat in (1, 3, 7):
        per_head = [k for k, _ in ranked if k.endswith(f"_p{pat}") and "_g256_" in k]
        names += per_head[:2]
    tag = [1]
    out = {}
    for name in dict.fromkeys(names):
        t, g, u, pat = (int(x[1:]) for x in name.split("_"))

        def fn(iters):
            rc = lib.qd_bench_read_merge(kc.data_ptr(), vc.data_ptr(), L * HID * 2, L, HID * 2, H,
                                         n_layers, t, u, pat, g, iters, slots.data_ptr(), mout.data_ptr(),
                                         tag[0], stale.data_ptr(), sh)
            if rc != 0:
                raise RuntimeError(f"read-merge launch failed ({name}): {rc}")
            tag[0] += iters
        fn(max(200, n_layers))
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        fn(steps)
        e1.record(stream)
        e1.synchronize()
        out[name] = {"read": sweep[name], "read_merge": round(e0.elapsed_time(e1) * 1e3 / steps, 3)}
    if int(stale.item()) != 0:
        raise RuntimeError(f"read-merge floor: {int(stale.item())} merging waves saw stale partials")
    per_head = {k: v["read_merge"] for k, v in out.items() if "_g256_" in k and k[-2:] in ("p1", "p3", "p7")}
    best = min(per_head.items(), key=lambda kv: kv[1]) if per_head else (None, None)
    log(f"[bench] read+merge floor L={L}: per-head best {best[0]} {best[1]} us; "
        + ", ".join(f"{k} {v['read']}/{v['read_merge']}" for k, v in out.items()))
    return out, best


def empty_loop(lib, sh, grid=H):
    """fn(iters): empty kernels of `grid` workgroups, back to back (the dispatch floor)."""
    def fn(iters):
        if lib.qd_bench_empty(grid, iters, sh) != 0:
            raise RuntimeError("empty-kernel launch failed")
    return fn


def profile_loop(lib, L: int, only: str, steps: int, warmup: int, variant: int, splits: int):
    """For a profiler: warmup + steps launches of one loop at L, nothing else timed or
    launched (so every dispatch in the trace belongs to that loop)."""
    import torch

    import qdiy

    n_layers, kc, vc, q, out = kv_layers(L)
    ctx = qdiy.Context(num_heads=H, max_seqlen=L)
    sh = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    kind = {"call": variant, "scan": 3, "merge": 4}.get(only)
    fn = (read_loop(lib, L, n_layers, kc, vc, sh) if only == "read" else
          empty_loop(lib, sh) if only == "empty" else
          attention_loop(lib, ctx, L, n_layers, kc, vc, q, out, sh, kind, splits))
    torch.cuda.synchronize()
    fn(warmup + steps)
    torch.cuda.synchronize()
    d = ctx.plan_detail(L, {0: "auto", 1: "fused", 2: "split"}[variant], splits)
    log(f"[bench] profile loop '{only}' at L={L}: {warmup + steps} launches, {n_layers} layers "
        f"rotated, plan {'fused' if d.variant == qdiy.FUSED else 'split'}x{d.num_splits}"
        f"{' merge in kernel' if d.merge_in_kernel else ''}")
    ctx.close()


def prefill_attention_loop(T: int, steps: int, warmup: int):
    """For a profiler: warmup + steps calls of qd_prefill_attention in the MFMA mode
    (the causal FlashAttention kernel) over a T-token prompt at position 0, 16 heads,
    the engine's cache layout, fp16 N(0,1) inputs; nothing else launched after the
    inputs are made."""
    import torch

    import qdiy

    torch.manual_seed(0)
    q = torch.randn(T, H * D, device="cuda").half()
    k = torch.randn(T, H * D, device="cuda").half()
    v = torch.randn(T, H * D, device="cuda").half()
    out = torch.empty_like(q)
    ctx = qdiy.Context(num_heads=H, max_seqlen=T)
    torch.cuda.synchronize()
    for _ in range(warmup + steps):
        ctx.prefill_attention(q, k, v, out, 0, T, qdiy.GEMM_MFMA)
    torch.cuda.synchronize()
    log(f"[bench] profile loop 'prefill' at T={T}: {warmup + steps} qd_prefill_attention calls (MFMA)")
    ctx.close()


def gemm_loops(T: int, steps: int, warmup: int, vendor: bool, which: str):
    """For a profiler, and as a timing of the MFMA prefill's products: the four
    products of one Qwen-1.8B-shaped layer at T tokens (QKV 6144 x 2048, gate and up
    with the SwiGLU 2 x 5504 x 2048, o_proj and c_proj with the residual) through
    qd_gemm_nt / qd_gemm_swiglu in the MFMA mode, weights of 12 layers rotated, fp16
    N(0,1) activations and N(0, 0.02) weights; with `vendor`, the same plain products
    through torch.matmul (hipBLASLt) after each.  `which` is a comma-separated subset
    of qkv, gateup, oproj, cproj.  Prints one JSON line of us per call (best of three
    windows of `steps` calls after `warmup`)."""
    import torch

    import qdiy

    HID, INTER, NL = H * D, 5504, 12
    dev = torch.device("cuda")
    gen = torch.Generator(device=dev)
    gen.manual_seed(1)

    def rnd(*shape, scale=1.0):
        return (torch.randn(*shape, device=dev, generator=gen) * scale).half()

    def timeit(fn):
        for i in range(warmup):
            fn(i)
        torch.cuda.synchronize()
        best = float("inf")
        for _ in range(3):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for i in range(steps):
                fn(i)
            e1.record()
            e1.synchronize()
            best = min(best, e0.elapsed_time(e1) * 1e3 / steps)
        return round(best, 2)

    x, xi = rnd(T, HID), rnd(T, INTER)
    res = {"tokens": T}
    sel = which.split(",")
    if "qkv" in sel:
        w = rnd(NL, 3 * HID, HID, scale=0.02)
        y = torch.empty(T, 3 * HID, dtype=torch.half, device=dev)
        res["qkv"] = timeit(lambda i: qdiy.gemm_nt(x, w[i % NL], y, T, 3 * HID, HID, mode=qdiy.GEMM_MFMA))
        if vendor:
            res["qkv_vendor"] = timeit(lambda i: torch.matmul(x, w[i % NL].t(), out=y))
        del w, y
    if "gateup" in sel:
        w1, w2 = rnd(NL, INTER, HID, scale=0.02), rnd(NL, INTER, HID, scale=0.02)
        act = torch.empty(T, INTER, dtype=torch.half, device=dev)
        res["gateup_swiglu"] = timeit(lambda i: qdiy.gemm_swiglu(x, w1[i % NL], w2[i % NL], act, T, INTER, HID))
        if vendor:
            w12 = torch.cat([w1, w2], dim=1)
            yy = torch.empty(T, 2 * INTER, dtype=torch.half, device=dev)
            res["gateup_vendor_plain"] = timeit(lambda i: torch.matmul(x, w12[i % NL].t(), out=yy))
            del w12, yy
        del w1, w2, act
    for name, k_in, xin in (("oproj", HID, x), ("cproj", INTER, xi)):
        if name not in sel:
            continue
        w = rnd(NL, HID, k_in, scale=0.02)
        y = rnd(T, HID)
        res[name + "_residual"] = timeit(
            lambda i: qdiy.gemm_nt(xin, w[i % NL], y, T, HID, k_in, residual=y, mode=qdiy.GEMM_MFMA))
        if vendor:
            res[name + "_vendor"] = timeit(lambda i: torch.matmul(xin, w[i % NL].t(), out=y))
        del w, y
    print(json.dumps(res), flush=True)


def measure(lib, L: int, steps: int, warmup: int, variant: int = 0, splits: int = 0,
            detail: bool = False):
    """us per call at L, cold (layers rotated) and hot (one layer).  detail: also the
    call's kernels alone (scan, merge), the read ceiling and the dispatch floor."""
    import torch

    import qdiy

    n_layers, kc, vc, q, out = kv_layers(L)
    ctx = qdiy.Context(num_heads=H, max_seqlen=L)
    stream = torch.cuda.current_stream()
    sh = ctypes.c_void_p(stream.cuda_stream)
    loop = attention_loop(lib, ctx, L, n_layers, kc, vc, q, out, sh, variant, splits)

    def run(iters, layers):
        loop(iters, layers)

    def timed(iters, fn):
        # no host synchronisation before e0: it is recorded behind the warm-up tail
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        fn(iters)
        e1.record(stream)
        e1.synchronize()
        return e0.elapsed_time(e1) * 1e3 / iters          # us per call

    cold = lambda n: run(n, n_layers)
    warm_calls, warm_ms = warm_up(cold, warmup)
    us_cold = timed(steps, cold)
    scan_us = merge_us = ceiling_us = floor_us = scan_alone_us = None
    sweep, sweep_best = None, (None, None)
    floor, floor_best = None, (None, None)
    tail = max(20, int(WARMUP_TAIL_S / (us_cold * 1e-6)))
    if detail:
        # the call's kernels on their own, back to back over the same layers
        # (qd_decode_attention_stage): scan only, then merge only
        stage = lambda kind: attention_loop(lib, ctx, L, n_layers, kc, vc, q, out, sh, kind)
        stage(3)(tail)
        scan_us = timed(steps, stage(3))
        pd = ctx.plan_detail(L)
        if pd.variant == qdiy.SPLIT and not pd.merge_in_kernel:
            stage(4)(tail)
            merge_us = timed(steps, stage(4))
        elif pd.variant == qdiy.SPLIT:
            # the same plan's scan alone (a two-launch context plans the same splits and
            # writes plain partials): the call's kernel less its in-kernel merge
            ctx2 = qdiy.Context(num_heads=H, max_seqlen=L)
            ctx2.set_merge(qdiy.MERGE_TWO_LAUNCHES)
            if ctx2.plan_detail(L).as_tuple() == pd.as_tuple():
                s2 = attention_loop(lib, ctx2, L, n_layers, kc, vc, q, out, sh, 3)
                s2(tail)
                scan_alone_us = timed(steps, s2)
            ctx2.close()
        # load-only kernel over the same layers' K and V rows, same launch shape
        read = read_loop(lib, L, n_layers, kc, vc, sh)
        read(tail)
        ceiling_us = timed(steps, read)
        # empty kernels of the merge's grid: what any dependent launch costs
        empty = empty_loop(lib, sh)
        empty(tail)
        floor_us = timed(steps, empty)
    hot = lambda n: run(n, 1)
    warm_up(hot, warmup, floor_s=0.0)
    us_hot = timed(steps, hot)
    if detail and L == HEADLINE_L:
        # the same bytes read by other launch shapes: what any one-launch design could
        # reach (last, so that its thousands of launches disturb no other figure)
        num_cus = torch.cuda.get_device_properties(0).multi_processor_count
        sweep, sweep_best = read_sweep(lib, L, n_layers, kc, vc, sh, max(steps, 200), num_cus)
        floor, floor_best = read_merge_floor(lib, L, n_layers, kc, vc, sh, max(steps, 500), sweep)
    if not torch.isfinite(out).all():
        raise RuntimeError("non-finite attention output")
    d = ctx.plan_detail(L, {0: "auto", 1: "fused", 2: "split"}[variant], splits)
    plan = ("fused" if d.variant == qdiy.FUSED else
            "split+merge-in-kernel" if d.merge_in_kernel else "split", d.num_splits)
    smax = 16 if d.num_splits <= 16 else 32 if d.num_splits <= 32 else 64
    inter = ", true" if d.block_rows else ""
    kernel = (f"decode_attention_xmerge_kernel<{d.rows_per_tile}, {smax}, {d.loads_per_round}, "
              f"{d.waves}{inter}>" if d.merge_in_kernel else
              f"decode_attention_scan_kernel<{d.waves}, {d.rows_per_tile}, "
              f"{'false' if d.variant == qdiy.FUSED else 'true'}, false, {d.loads_per_round}{inter}>")
    ctx.close()
    del kc, vc
    torch.cuda.empty_cache()
    gbps = algo_bytes(L) / (us_cold * 1e-6) / 1e9
    res = {"L": L, "us_cold": us_cold, "us_hot": us_hot, "gbps": gbps,
           "gbps_hot": algo_bytes(L) / (us_hot * 1e-6) / 1e9, "frac": gbps / PEAK_GBPS,
           "layers": n_layers, "plan": f"{plan[0]}x{plan[1]}", "kernel": kernel,
           "warmup_calls": warm_calls, "warmup_ms": round(warm_ms, 1),
           "scan_us": scan_us, "merge_us": merge_us, "read_ceiling_us": ceiling_us,
           "scan_alone_us": scan_alone_us,
           "launch_floor_us": floor_us, "read_sweep": sweep, "read_best_shape": sweep_best[0],
           "read_best_us": sweep_best[1], "read_merge_floor": floor,
           "read_merge_floor_best_shape": floor_best[0], "read_merge_floor_best_us": floor_best[1]}
    extra = ""
    if detail:
        res["scan_gbps"] = scan_bytes(L) / (scan_us * 1e-6) / 1e9
        res["ceiling_gbps"] = 2 * L * HID * 2 / (ceiling_us * 1e-6) / 1e9
        extra = (f"; alone: scan kernel {scan_us:.2f} us ({res['scan_gbps']:.0f} GB/s), merge "
                 f"kernel {merge_us if merge_us is None else round(merge_us, 2)} us; read ceiling "
                 f"{ceiling_us:.2f} us ({res['ceiling_gbps']:.0f} GB/s); empty kernel {floor_us:.2f} us")
    log(f"[bench] L={L}: {us_cold:.2f} us/call cold ({gbps:.0f} GB/s, {100 * gbps / PEAK_GBPS:.1f}% "
        f"of 8 TB/s), {us_hot:.2f} us hot, plan {res['plan']}, {n_layers} layers rotated, "
        f"warm-up {warm_calls} calls / {warm_ms:.0f} ms{extra}")
    return res


def front_loops(lib, steps: int, warmup: int):
    """For a profiler: config 4's three loops (bench.py's config4_front_end), warmup +
    steps launches each, in order: qd_qkv_proj_rope_cache alone, then followed by
    qd_decode_attention over 2048 rows (two calls), then qd_qkv_proj_rope_cache_attention
    (one launch); nothing else is launched after the inputs are made."""
    import torch

    run, close = _front_setup(lib)
    for mode in (0, 1, 2):
        run(warmup + steps, mode)
        torch.cuda.synchronize()
    log(f"[bench] profile loops 'front': {warmup + steps} calls each of the front end alone, "
        f"front end + attention as two calls, and as one call")
    close()


def _front_setup(lib):
    """Config 4's inputs and a runner run(iters, mode) over the rotated layers (mode 0
    front end alone, 1 front end then attention as two calls, 2 one call); returns
    (run, close)."""
    import torch

    import qdiy

    L, pos = 2048, 2047
    w_elems = 3 * HID * HID
    kv_elems = L * HID
    n_layers = max(3, math.ceil((1 << 30) / (2 * (w_elems + 2 * kv_elems))))
    gen = torch.Generator(device="cuda")
    gen.manual_seed(4)
    x = torch.empty(n_layers * HID, dtype=torch.float16, device="cuda").normal_(generator=gen)
    w = torch.empty(n_layers * w_elems, dtype=torch.float16, device="cuda").normal_(0.0, 0.02, generator=gen)
    b = torch.empty(n_layers * 3 * HID, dtype=torch.float16, device="cuda").normal_(0.0, 0.02, generator=gen)
    kc = torch.empty(n_layers * kv_elems, dtype=torch.float16, device="cuda").normal_(generator=gen)
    vc = torch.empty_like(kc).normal_(generator=gen)
    qkv = torch.empty(n_layers * 3 * HID, dtype=torch.float16, device="cuda")
    out = torch.empty(n_layers * HID, dtype=torch.float16, device="cuda")
    ctx = qdiy.Context(num_heads=H, max_seqlen=L)
    sh = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    def run(iters, mode):
        rc = lib.qd_bench_attn_front(ctx._h, x.data_ptr(), w.data_ptr(), b.data_ptr(), qkv.data_ptr(),
                                     kc.data_ptr(), vc.data_ptr(), out.data_ptr(), w_elems, kv_elems,
                                     n_layers, pos, L, H, iters, mode, sh)
        if rc != 0:
            raise RuntimeError(f"front-end bench failed: {qdiy.load().qd_last_error().decode()}")

    def close():
        ctx.close()
        torch.cuda.empty_cache()
    return run, close


def measure_front(lib, steps: int, warmup: int):
    """Config 4: QKV GEMV [6144 x 2048] + bias + RoPE at pos 2047 + append, then
    attention over 2048 rows; weights and KV rotate over enough layers (>= 1 GiB)
    that every call streams from HBM."""
    import torch

    import qdiy

    L, pos = 2048, 2047
    w_elems = 3 * HID * HID
    kv_elems = L * HID
    n_layers = max(3, math.ceil((1 << 30) / (2 * (w_elems + 2 * kv_elems))))
    gen = torch.Generator(device="cuda")
    gen.manual_seed(4)
    x = torch.empty(n_layers * HID, dtype=torch.float16, device="cuda").normal_(generator=gen)
    w = torch.empty(n_layers * w_elems, dtype=torch.float16, device="cuda").normal_(0.0, 0.02, generator=gen)
    b = torch.empty(n_layers * 3 * HID, dtype=torch.float16, device="cuda").normal_(0.0, 0.02, generator=gen)
    kc = torch.empty(n_layers * kv_elems, dtype=torch.float16, device="cuda").normal_(generator=gen)
    vc = torch.empty_like(kc).normal_(generator=gen)
    qkv = torch.empty(n_layers * 3 * HID, dtype=torch.float16, device="cuda")
    out = torch.empty(n_layers * HID, dtype=torch.float16, device="cuda")
    ctx = qdiy.Context(num_heads=H, max_seqlen=L)
    stream = torch.cuda.current_stream()
    sh = ctypes.c_void_p(stream.cuda_stream)

    def run(iters, with_attn):
        rc = lib.qd_bench_attn_front(ctx._h, x.data_ptr(), w.data_ptr(), b.data_ptr(), qkv.data_ptr(),
                                     kc.data_ptr(), vc.data_ptr(), out.data_ptr(), w_elems, kv_elems,
                                     n_layers, pos, L, H, iters, with_attn, sh)
        if rc != 0:
            raise RuntimeError(f"front-end bench failed: {qdiy.load().qd_last_error().decode()}")

    def timed(iters, with_attn, floor_s):
        warm_up(lambda n: run(n, with_attn), warmup, floor_s)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        run(iters, with_attn)
        e1.record(stream)
        e1.synchronize()
        return e0.elapsed_time(e1) * 1e3 / iters

    us_front = timed(steps, 0, WARMUP_FLOOR_S)
    us_two = timed(steps, 1, 0.0)        # qd_qkv_proj_rope_cache, then qd_decode_attention
    us_all = timed(steps, 2, 0.0)        # qd_qkv_proj_rope_cache_attention (one launch)
    ctx.close()
    del w, kc, vc
    torch.cuda.empty_cache()
    front_bytes = w_elems * 2 + HID * 2 + 3 * HID * 2 + 2 * HID * 2
    all_bytes = front_bytes + 2 * L * HID * 2 + HID * 2      # config 4 (L=2048): 41,971,712 B
    log(f"[bench] config 4 (L=2048, pos 2047): front end {us_front:.2f} us "
        f"({front_bytes / us_front / 1e3:.0f} GB/s), front end + attention {us_all:.2f} us in one "
        f"call ({all_bytes / us_all / 1e3:.0f} GB/s; {us_two:.2f} us as two calls), {n_layers} layers "
        f"rotated")
    return {"us_front_end": round(us_front, 3), "us_front_end_plus_attention": round(us_all, 3),
            "entry": "qd_qkv_proj_rope_cache_attention",
            "us_front_end_plus_attention_two_calls": round(us_two, 3),
            "bytes": all_bytes, "gbps": round(all_bytes / us_all / 1e3, 1),
            "pct_of_peak": round(100 * all_bytes / us_all / 1e3 / PEAK_GBPS, 1),
            "front_end_gbps": round(front_bytes / us_front / 1e3, 1)}


def measure_e2e(lib, seed: int = 5, n_prompt: int = 128, n_new: int = 256):
    """Config 5: random-init Qwen-1.8B (24 layers, hidden 2048, 16 heads, FFN
    5504, vocab 151936; weights ~N(0, 0.02) by the library's generator, norm
    weights 1) in the .bin format, a prompt of n_prompt uniform-random ids, then
    n_new greedy tokens through qdiy.Engine (one synchronising step per token,
    as the reference engine).  Decode tokens/s is timed over the n_new steps;
    the prompt's first n_prompt - 1 tokens go through the batched prefill first
    and are timed separately, and so, afterwards, is a 2048-token prompt."""
    import numpy as np

    import qdiy

    cfg = qdiy.model_cfg()
    t0 = time.perf_counter()
    img = qdiy.random_model_image(cfg, seed, 0.02, nthreads=16)
    t_fill = time.perf_counter() - t0
    eng = qdiy.Engine(image=img)
    del img
    rng = np.random.default_rng(seed)
    prompt = [int(t) for t in rng.integers(0, cfg.vocab_size, n_prompt)]
    eng.generate(prompt[:8], 8, stop_at_eos=False)            # warm-up
    eng.reset()
    t0 = time.perf_counter()
    pos = eng.prefill(prompt[:-1])
    t_prompt = time.perf_counter() - t0
    last, toks = prompt[-1], []
    t0 = time.perf_counter()
    for _ in range(n_new):
        last = eng.step(last, pos)
        pos += 1
        toks.append(last)
    t_dec = time.perf_counter() - t0
    # A long prompt: 2048 uniform-random ids through the batched exact prefill
    # (fused attention up to 224 rows, batched split launches beyond), best of 2;
    # then both prompts with the projections on the matrix cores
    # (qd_engine_set_prefill_mode(QD_GEMM_MFMA): not bit-identical to decode).
    long_prompt = [int(t) for t in rng.integers(0, cfg.vocab_size, 2048)]

    def best_prefill(tokens):
        best = float("inf")
        for _ in range(2):
            eng.reset()
            t0 = time.perf_counter()
            eng.prefill(tokens)
            best = min(best, time.perf_counter() - t0)
        return best

    t_long = best_prefill(long_prompt)
    eng.set_prefill_mode(qdiy.GEMM_MFMA)
    t_prompt_mfma, t_long_mfma = best_prefill(prompt[:-1]), best_prefill(long_prompt)
    eng.close()
    ms_tok = t_dec * 1e3 / n_new
    # Attention per token: 24 qd_decode_attention calls at the mean KV length of
    # the generated tokens, timed cold in isolation.
    mean_L = n_prompt + n_new // 2
    att = measure(lib, mean_L, 400, 40, 0, 0)
    share = cfg.num_layers * att["us_cold"] / 1e3 / ms_tok
    H_, I_, V_, NL = cfg.hidden_size, cfg.intermediate_size, cfg.vocab_size, cfg.num_layers
    w_bytes = 2 * (NL * (3 * H_ * H_ + 3 * H_ + H_ * H_ + 2 * H_ + 3 * I_ * H_) + H_ + V_ * H_ + H_)
    tok_bytes = w_bytes + NL * 2 * mean_L * H_ * 2
    log(f"[bench] config 5: {n_new / t_dec:.1f} tokens/s ({ms_tok:.3f} ms/token, "
        f"{tok_bytes / (ms_tok * 1e-3) / 1e9:.0f} GB/s over {tok_bytes / 1e9:.3f} GB/token), "
        f"prompt {n_prompt - 1} tokens in {t_prompt * 1e3:.1f} ms ({len(long_prompt)} in {t_long * 1e3:.0f} ms; "
        f"MFMA prefill {t_prompt_mfma * 1e3:.1f} / {t_long_mfma * 1e3:.0f} ms), "
        f"attention share ~{100 * share:.1f}% "
        f"(24 x {att['us_cold']:.2f} us at L={mean_L}), image fill {t_fill:.1f} s")
    return {"model": "Qwen-1.8B shape, random init (library generator, std 0.02, norm weights 1)",
            "prompt_tokens": n_prompt, "generated_tokens": n_new,
            "tokens_per_s": round(n_new / t_dec, 2), "ms_per_token": round(ms_tok, 4),
            "prompt_ms": round(t_prompt * 1e3, 2),
            "prompt_2048_ms": round(t_long * 1e3, 1),
            "prompt_ms_mfma_prefill": round(t_prompt_mfma * 1e3, 2),
            "prompt_2048_ms_mfma_prefill": round(t_long_mfma * 1e3, 1), "bytes_per_token": tok_bytes,
            "gbps": round(tok_bytes / (ms_tok * 1e-3) / 1e9, 1),
            "attention_share_est": round(share, 4),
            "attention_us_per_call_at_mean_L": round(att["us_cold"], 3), "mean_L": mean_L,
            "first_tokens": toks[:8]}


def cpu_baseline(L: int, seconds: float):
    """Times the C oracle (restatement of the reference kernels) on host cores."""
    import numpy as np

    from oracle import oracle

    rng = np.random.default_rng(7)
    q = rng.standard_normal((H, D), dtype=np.float32).astype(np.float16)
    kc = (rng.standard_normal(L * HID, dtype=np.float32) * 0.5).astype(np.float16)
    vc = rng.standard_normal(L * HID, dtype=np.float32).astype(np.float16)
    try:
        ncores = len(os.sched_getaffinity(0))
    except AttributeError:
        ncores = os.cpu_count() or 1
    threads = max(1, min(16, ncores))

    def rate(nthreads, budget):
        n, t0 = 0, time.perf_counter()
        while True:
            oracle.decode_attention(q, kc, vc, L, H, HID, D, oracle.ENGINE, nthreads)
            n += 1
            el = time.perf_counter() - t0
            if el >= budget:
                return el / n, n

    t1, n1 = rate(1, seconds * 0.4)
    tn, nn = rate(threads, seconds * 0.6)
    log(f"[bench] CPU oracle L={L}: {t1 * 1e6:.0f} us/call on 1 thread, {tn * 1e6:.0f} us/call on "
        f"{threads} threads ({ncores} cores visible)")
    return {"value": algo_bytes(L) / tn / 1e9, "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"{nn} calls at L={L} on {threads} threads + {n1} on 1 thread, "
                      f"16 heads x 128, fp16 N(0,1) (K x0.5), engine dispatch (split 256-row chunks)",
            "us_per_call": tn * 1e6, "us_per_call_1thread": t1 * 1e6,
            "gbps_1thread": algo_bytes(L) / t1 / 1e9, "cores_visible": ncores}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--kv", type=int, nargs="*", default=list(KV_LENS))
    ap.add_argument("--variant", choices=["auto", "fused", "split"], default="auto")
    ap.add_argument("--splits", type=int, default=0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-front", action="store_true", help="skip the config-4 front-end timing")
    ap.add_argument("--no-e2e", action="store_true", help="skip the config-5 end-to-end timing")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--pmc-calibration", action="store_true",
                    help="run one 256 MiB device copy (known FETCH_SIZE/WRITE_SIZE) and exit")
    ap.add_argument("--only", choices=["call", "scan", "merge", "read", "empty", "prefill", "sweep", "front",
                                       "gemm"],
                    help="for a profiler: run warmup + steps launches of this loop per --kv length "
                         "(call: qd_decode_attention; scan / merge: that kernel alone; read: the "
                         "read-ceiling kernel; empty: empty kernels; prefill: qd_prefill_attention "
                         "in the MFMA mode over a --kv-token prompt; front: config 4's front end "
                         "alone, with attention as two calls, and as one call; gemm: the MFMA "
                         "prefill's four products at --kv tokens, see --gemm), print no bench "
                         "JSON, and exit")
    ap.add_argument("--gemm", default="qkv,gateup,oproj,cproj",
                    help="--only gemm: products to run (qkv, gateup, oproj, cproj)")
    ap.add_argument("--vendor", action="store_true",
                    help="--only gemm: also time the plain products through torch.matmul (hipBLASLt)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: this build has no multi-GPU path "
              f"(--gpus {args.gpus} requested)", file=sys.stderr)
        return 2
    if int(os.environ.get("RANK", "0")) != 0:
        return 0

    import torch

    torch.cuda.set_device(0)
    if args.pmc_calibration:
        # Counter calibration: a copy of exactly 256 MiB reads and writes 256 MiB of
        # HBM.  A third buffer is streamed first so the source is not cache-resident.
        n = (256 << 20) // 2
        a = torch.zeros(n, dtype=torch.float16, device="cuda")
        b = torch.zeros_like(a)
        c = torch.zeros_like(a)
        c.add_(1.0)
        torch.cuda.synchronize()
        b.copy_(a)
        torch.cuda.synchronize()
        log("[bench] pmc calibration: copied 268435456 bytes")
        return 0
    lib = bench_lib()
    variant = {"auto": 0, "fused": 1, "split": 2}[args.variant]
    if args.only == "prefill":
        for T in args.kv:
            prefill_attention_loop(T, args.steps, args.warmup)
        return 0
    if args.only == "front":
        front_loops(lib, args.steps, args.warmup)
        return 0
    if args.only == "gemm":
        for T in args.kv:
            gemm_loops(T, args.steps, args.warmup, args.vendor, args.gemm)
        return 0
    if args.only == "sweep":
        num_cus = torch.cuda.get_device_properties(0).multi_processor_count
        for L in args.kv:
            n_layers, kc, vc, _, _ = kv_layers(L)
            sh = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
            sweep, best = read_sweep(lib, L, n_layers, kc, vc, sh, args.steps, num_cus)
            print(json.dumps({"L": L, "best": best, "sweep": sweep}), flush=True)
            del kc, vc
            torch.cuda.empty_cache()
        return 0
    if args.only:
        for L in args.kv:
            profile_loop(lib, L, args.only, args.steps, args.warmup, variant, args.splits)
        return 0
    kv = sorted(set(args.kv) | {HEADLINE_L})
    # The headline length is measured first, in the process's first KV buffers, as
    # an engine allocates its cache once at start-up.  Buffers allocated again after
    # an earlier phase freed its own can land on physical pages that run the same
    # calls up to ~3% slower (15.45 against 14.97-15.05 us per call at L=8192).
    order = [HEADLINE_L] + [L for L in kv if L != HEADLINE_L]
    detail = variant == 0
    measured = {L: measure(lib, L, args.steps, args.warmup, variant, args.splits, detail)
                for L in order}
    res = {L: measured[L] for L in kv}
    head = res[HEADLINE_L]
    # config 1 names the fused single-workgroup-per-head path at L=512
    fused512 = measure(lib, 512, args.steps, args.warmup, 1, 0) if 512 in kv and variant == 0 else None
    front = None if args.no_front else measure_front(lib, args.steps, args.warmup)
    e2e = None if args.no_e2e else measure_e2e(lib)
    # counter evidence per length (profiles/traffic_decode_attention_L*.json)
    traffic = {}
    for L in kv:
        if os.path.exists(traffic_file(L)):
            with open(traffic_file(L)) as f:
                traffic[L] = json.load(f)
    cpu = None if args.no_cpu else cpu_baseline(HEADLINE_L, args.cpu_seconds)
    per_l = lambda key, nd=3: {str(L): (None if r.get(key) is None else round(r[key], nd))
                               for L, r in res.items()}
    line = {
        "metric": METRIC,
        "value": round(head["gbps"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["us_cold"] / 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic",
        "config": {
            "workload": f"decode_attention_L{HEADLINE_L}",
            "heads": H, "head_dim": D, "kv_len": HEADLINE_L,
            "io": "fp16 Q/K/V/O, fp32 accumulate",
            "cache_layout": "[pos][16*128] (reference engine layout)",
            "cache": "cold: each step reads a different layer; >= 1 GiB rotated; "
                     f"L={HEADLINE_L} measured first, in the process's first KV buffers",
            "warmup_run": {"floor_ms": WARMUP_FLOOR_S * 1e3,
                           "calls": {str(L): r["warmup_calls"] for L, r in res.items()},
                           "ms": {str(L): r["warmup_ms"] for L, r in res.items()}},
            "plan": head["plan"],
            "us_per_call": per_l("us_cold"),
            "gbps": per_l("gbps", 1),
            "pct_of_peak": {str(L): round(100 * r["frac"], 1) for L, r in res.items()},
            "us_per_call_hot": per_l("us_hot"),
            "plans": {str(L): r["plan"] for L, r in res.items()},
            "scan_kernel_us": per_l("scan_us"),
            "scan_kernel_gbps": per_l("scan_gbps", 1),
            "merge_kernel_us": per_l("merge_us"),
            "scan_without_in_kernel_merge_us": per_l("scan_alone_us"),
            "read_ceiling_us": per_l("read_ceiling_us"),
            "read_ceiling_gbps": per_l("ceiling_gbps", 1),
            "read_ceiling_best_us": head.get("read_best_us"),
            "read_ceiling_best_shape": head.get("read_best_shape"),
            "read_sweep_L8192": head.get("read_sweep"),
            "read_merge_floor_L8192": head.get("read_merge_floor"),
            "read_merge_floor_per_head_best_us": head.get("read_merge_floor_best_us"),
            "read_merge_floor_per_head_best_shape": head.get("read_merge_floor_best_shape"),
            "empty_kernel_us": per_l("launch_floor_us"),
            "traffic_over_algorithmic": {str(L): t.get("traffic_over_algorithmic")
                                         for L, t in traffic.items()},
            "fused_path_us_per_call_512": None if fused512 is None else round(fused512["us_cold"], 3),
            "config4_front_end": front,
            "config5_e2e": e2e,
        },
        "roofline": None if not detail else {
            "bound": "hbm",
            "kernel": f"{head['kernel']} (the {'only' if 'in-kernel' in head['plan'] else 'scan'} "
                      f"kernel of qd_decode_attention at L={HEADLINE_L}, plan {head['plan']})",
            "achieved": round(head["scan_gbps"], 1), "peak": PEAK_GBPS, "unit": "GB/s",
            "frac": round(head["scan_gbps"] / PEAK_GBPS, 4),
            "traffic": traffic.get(HEADLINE_L, {}).get("scan_kernel_traffic_bytes"),
            "traffic_source": (f"{os.path.relpath(traffic_file(HEADLINE_L), ROOT)}: rocprofv3 --pmc "
                               f"FETCH_SIZE and WRITE_SIZE runs of bench.py --only call, scaled by a "
                               f"copy kernel's counts (not measured in this run)"),
            "algorithmic_bytes_per_launch": scan_bytes(HEADLINE_L),
            "launch_us": round(head["scan_us"], 3),
            "launch_timing": ("the call's one kernel, back to back on the same rotated layers "
                              "(qd_decode_attention_stage, scan stage: the whole call for a plan "
                              "that merges in the scan kernel)" if "in-kernel" in head["plan"] else
                              "scan-only launches back to back on the same rotated layers "
                              "(qd_decode_attention_stage); inside the call, after each merge "
                              "kernel, the same kernel runs ~0.7 us longer per launch in the "
                              "committed kernel trace"),
            "call_frac": round(head["frac"], 4),
            "per_kernel_trace": "profiles/decode_attention_kernel_trace_L512_to_L32768.md"},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
