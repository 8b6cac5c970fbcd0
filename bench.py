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

The CPU baseline is the repository's C restatement of the reference kernels
(oracle/) on the host cores of the same box, on a bounded sample of the same
workload.

Also measured and reported under `config`: config 4 (the fused QKV front end
followed by attention at L=2048) and config 5 (greedy decode of a random-init
Qwen-1.8B-shaped model through the engine: tokens/s, an estimate of the
attention share of a decode step, and the prefill time of the 127-token prompt
and of a 2048-token one, exact and with the projections on the matrix cores).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-e2e]
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
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic_decode_attention_L8192.json")


def algo_bytes(L: int) -> int:
    return 2 * H * D * 2 + 2 * H * L * D * 2     # Q + O, K + V


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
    lib.qd_bench_attn_front.argtypes = [vp, vp, vp, vp, vp, vp, vp, vp, ll, ll, i, i, i, i, i, i, vp]
    return lib


def measure(lib, L: int, steps: int, warmup: int, variant: int = 0, splits: int = 0):
    import torch

    import qdiy

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
    out = torch.empty_like(q)
    ctx = qdiy.Context(num_heads=H, max_seqlen=L)
    stream = torch.cuda.current_stream()
    sh = ctypes.c_void_p(stream.cuda_stream)

    def run(iters, layers):
        rc = lib.qd_bench_decode_attention(ctx._h, q.data_ptr(), kc.data_ptr(), vc.data_ptr(),
                                           out.data_ptr(), HID, L * HID, layers, L, H, iters,
                                           variant, splits, sh)
        if rc != 0:
            raise RuntimeError(f"bench loop failed: {qdiy.load().qd_last_error().decode()}")

    def timed(iters, layers):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record(stream)
        run(iters, layers)
        e1.record(stream)
        e1.synchronize()
        return e0.elapsed_time(e1) * 1e3 / iters          # us per call

    run(warmup, n_layers)
    us_cold = timed(steps, n_layers)
    run(warmup, 1)
    us_hot = timed(steps, 1)
    if not torch.isfinite(out).all():
        raise RuntimeError("non-finite attention output")
    if variant == 1:
        plan = ("fused", 1)
    else:
        d = ctx.plan_detail(L, "split" if variant == 2 else "auto", splits)
        plan = ("fused" if d.variant == qdiy.FUSED else "split", d.num_splits)
    ctx.close()
    del kc, vc
    torch.cuda.empty_cache()
    gbps = algo_bytes(L) / (us_cold * 1e-6) / 1e9
    res = {"L": L, "us_cold": us_cold, "us_hot": us_hot, "gbps": gbps,
           "gbps_hot": algo_bytes(L) / (us_hot * 1e-6) / 1e9, "frac": gbps / PEAK_GBPS,
           "layers": n_layers, "plan": f"{plan[0]}x{plan[1]}"}
    log(f"[bench] L={L}: {us_cold:.2f} us/call cold ({gbps:.0f} GB/s, {100 * gbps / PEAK_GBPS:.1f}% "
        f"of 8 TB/s), {us_hot:.2f} us hot, plan {res['plan']}, {n_layers} layers rotated")
    return res


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

    def timed(iters, with_attn):
        run(warmup, with_attn)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record(stream)
        run(iters, with_attn)
        e1.record(stream)
        e1.synchronize()
        return e0.elapsed_time(e1) * 1e3 / iters

    us_front = timed(steps, 0)
    us_all = timed(steps, 1)
    ctx.close()
    del w, kc, vc
    torch.cuda.empty_cache()
    front_bytes = w_elems * 2 + HID * 2 + 3 * HID * 2 + 2 * HID * 2
    all_bytes = front_bytes + 2 * L * HID * 2 + HID * 2      # config 4 (L=2048): 41,971,712 B
    log(f"[bench] config 4 (L=2048, pos 2047): front end {us_front:.2f} us "
        f"({front_bytes / us_front / 1e3:.0f} GB/s), front end + attention {us_all:.2f} us "
        f"({all_bytes / us_all / 1e3:.0f} GB/s), {n_layers} layers rotated")
    return {"us_front_end": round(us_front, 3), "us_front_end_plus_attention": round(us_all, 3),
            "bytes": all_bytes, "gbps": round(all_bytes / us_all / 1e3, 1),
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
    kv = sorted(set(args.kv) | {HEADLINE_L})
    # The headline length is measured first, in the process's first KV buffers, as
    # an engine allocates its cache once at start-up.  Buffers allocated again after
    # an earlier phase freed its own can land on physical pages that run the same
    # calls up to ~3% slower (15.45 against 14.97-15.05 us per call at L=8192).
    order = [HEADLINE_L] + [L for L in kv if L != HEADLINE_L]
    measured = {L: measure(lib, L, args.steps, args.warmup, variant, args.splits) for L in order}
    res = {L: measured[L] for L in kv}
    head = res[HEADLINE_L]
    # config 1 names the fused single-workgroup-per-head path at L=512
    fused512 = measure(lib, 512, args.steps, args.warmup, 1, 0) if 512 in kv and variant == 0 else None
    front = None if args.no_front else measure_front(lib, args.steps, args.warmup)
    e2e = None if args.no_e2e else measure_e2e(lib)
    traffic = None
    if os.path.exists(TRAFFIC_FILE):
        with open(TRAFFIC_FILE) as f:
            traffic = json.load(f).get("traffic_bytes_per_launch")
    cpu = None if args.no_cpu else cpu_baseline(HEADLINE_L, args.cpu_seconds)
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
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": f"decode_attention_L{HEADLINE_L}",
            "heads": H, "head_dim": D, "kv_len": HEADLINE_L,
            "io": "fp16 Q/K/V/O, fp32 accumulate",
            "cache_layout": "[pos][16*128] (reference engine layout)",
            "cache": "cold: each step reads a different layer; >= 1 GiB rotated; "
                     f"L={HEADLINE_L} measured first, in the process's first KV buffers",
            "plan": head["plan"],
            "us_per_call": {str(L): round(r["us_cold"], 3) for L, r in res.items()},
            "gbps": {str(L): round(r["gbps"], 1) for L, r in res.items()},
            "pct_of_peak": {str(L): round(100 * r["frac"], 1) for L, r in res.items()},
            "us_per_call_hot": {str(L): round(r["us_hot"], 3) for L, r in res.items()},
            "plans": {str(L): r["plan"] for L, r in res.items()},
            "fused_path_us_per_call_512": None if fused512 is None else round(fused512["us_cold"], 3),
            "config4_front_end": front,
            "config5_e2e": e2e,
        },
        "roofline": {"bound": "hbm",
                     "kernel": f"qd_decode_attention call ({head['plan']}: "
                               "decode_attention_scan_kernel + decode_attention_merge_kernel)",
                     "achieved": round(head["gbps"], 1), "peak": PEAK_GBPS,
                     "unit": "GB/s", "frac": round(head["frac"], 4), "traffic": traffic,
                     "per_kernel_trace": "profiles/decode_attention_kernel_trace_L512_to_L32768.md"},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
