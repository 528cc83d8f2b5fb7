"""Benchmark of the Gemma 4 E2B attention hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]

Prints ONE JSON line. The headline (`value`) is BASELINE config 2 global: decode
attention, nH 8 / kvH 2, hd 256, KV length 4096, f16 cache, in GB/s of K+V bytes
attended (8,388,608 B per call). A step is one decode call; the timed region
replays a HIP graph of K calls that rotate over 64 distinct KV caches (512 MiB, more
than the 256 MiB Infinity Cache), so every call streams its cache from HBM.
`secondary` carries the other BASELINE rows: config 2 sliding (W 512), config 3
prefill (S 1024, global and W 512, TFLOP/s of 4*hd*nH*attended-pairs), config 4
(16 sequences, KV ~ U[1024, 32768]). Times come from HIP events on the stream the
kernels run on. `cpu_baseline` is the numpy oracle on this host for the headline
workload (a bounded sample).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np
import torch

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E, published
F16_PEAK_TFLOPS = 2500.0     # MI355X dense f16 MFMA, published
NH, KVH, HD = 8, 2, 256


def graph_time_ms(fn_list, steps, warmup):
    """Capture `steps` calls (cycling fn_list) in one HIP graph; return mean ms per call."""
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for i in range(max(warmup, 1)):
            fn_list[i % len(fn_list)]()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        for i in range(steps):
            fn_list[i % len(fn_list)]()
    torch.cuda.synchronize()
    g.replay()                      # warm replay (untimed)
    torch.cuda.synchronize()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        ev0.record(stream)
        g.replay()
        ev1.record(stream)
    torch.cuda.synchronize()
    return ev0.elapsed_time(ev1) / steps


def make_caches(sa, n, T, theta, gen, window=0):
    """n distinct f16 caches [T][kvH][hd] written by the library's kv_write from N(0,1) k/v."""
    cos, sin = sa.rope_tables(np.arange(T), HD, theta)
    kg = 1 + 0.1 * torch.randn(HD, device="cuda", generator=gen)
    out = []
    for _ in range(n):
        kr = torch.randn(T, KVH, HD, device="cuda", generator=gen)
        vr = torch.randn(T, KVH, HD, device="cuda", generator=gen)
        kc = torch.empty(T, KVH, HD, device="cuda", dtype=torch.float16)
        vc = torch.empty_like(kc)
        sa.kv_write(kr, vr, kc, vc, 0, sa.AttnConfig(KVH, KVH, HD), k_gain=kg, rope_cos=cos, rope_sin=sin)
        out.append((kc, vc))
    torch.cuda.synchronize()
    return out


def decode_case(sa, T, window, theta, steps, warmup, n_caches, gen):
    caches = make_caches(sa, n_caches, T, theta, gen)
    q = torch.randn(NH, HD, device="cuda", generator=gen)
    qg = 1 + 0.1 * torch.randn(HD, device="cuda", generator=gen)
    cos, sin = sa.rope_tables([T - 1], HD, theta)
    kl = torch.tensor([T], dtype=torch.int32, device="cuda")
    cfg = sa.AttnConfig(NH, KVH, HD, window)
    ws = sa.DecodeWorkspace("cuda")
    out = torch.empty(1, NH, HD, device="cuda")
    fns = [lambda kc=kc, vc=vc: sa.decode(q, kc, vc, kl, cfg, q_gain=qg, rope_cos=cos, rope_sin=sin,
                                          out=out, workspace=ws) for kc, vc in caches]
    ms = graph_time_ms(fns, steps, warmup)
    attended = min(T, window) if window else T
    nbytes = 2 * attended * KVH * HD * 2
    return ms, nbytes, (q, qg, cos, sin, caches[0], cfg)


def prefill_case(sa, S, window, theta, steps, warmup, gen):
    q = torch.randn(S, NH, HD, device="cuda", generator=gen)
    qg = 1 + 0.1 * torch.randn(HD, device="cuda", generator=gen)
    cos, sin = sa.rope_tables(np.arange(S), HD, theta)
    kc, vc = make_caches(sa, 1, S, theta, gen)[0]
    cfg = sa.AttnConfig(NH, KVH, HD, window)
    out = torch.empty(S, NH, HD, device="cuda", dtype=torch.float16)
    fn = lambda: sa.prefill(q, kc, vc, 0, cfg, q_gain=qg, rope_cos=cos, rope_sin=sin, out=out)  # noqa: E731
    ms = graph_time_ms([fn], steps, warmup)
    pairs = sum(min(p + 1, window) if window else p + 1 for p in range(S))
    flops = 4 * HD * NH * pairs
    return ms, flops


def batched_decode_case(sa, steps, warmup, gen):
    B, Tmax = 16, 32768
    lens = np.random.default_rng(4).integers(1024, Tmax + 1, size=B).astype(np.int32)
    k = torch.randn(B, Tmax, KVH, HD, device="cuda", generator=gen).half()
    v = torch.randn(B, Tmax, KVH, HD, device="cuda", generator=gen).half()
    q = torch.randn(B, NH, HD, device="cuda", generator=gen)
    kl = torch.from_numpy(lens).cuda()
    cfg = sa.AttnConfig(NH, KVH, HD)
    ws = sa.DecodeWorkspace("cuda")
    out = torch.empty_like(q)
    fn = lambda: sa.decode(q, k, v, kl, cfg, out=out, workspace=ws)  # noqa: E731
    ms = graph_time_ms([fn], steps, warmup)
    return ms, int(2 * lens.sum()) * KVH * HD * 2, int(lens.sum())


def cpu_baseline(case, seconds):
    """The numpy oracle (oracle/attention.py) on this host for the headline decode call."""
    import oracle.attention as O
    try:
        from threadpoolctl import threadpool_limits
    except ImportError:  # pragma: no cover
        threadpool_limits = None
    q, qg, cos, sin, (kc, vc), cfg = case
    qn, qgn = q.cpu().numpy(), qg.cpu().numpy()
    c, s = cos.cpu().numpy()[0], sin.cpu().numpy()[0]
    k, v = kc.cpu().numpy(), vc.cpu().numpy()
    T = k.shape[0]
    threads = min(16, os.cpu_count() or 1)
    ctx = threadpool_limits(limits=threads) if threadpool_limits else None
    try:
        O.decode_attention(qn, k, v, T, KVH, q_gain=qgn, cos=c, sin=s, window=cfg.window)
        n, t0 = 0, time.perf_counter()
        while True:
            O.decode_attention(qn, k, v, T, KVH, q_gain=qgn, cos=c, sin=s, window=cfg.window)
            n += 1
            el = time.perf_counter() - t0
            if el >= seconds or n >= 100000:
                break
    finally:
        if ctx is not None:
            ctx.__exit__(None, None, None)
    per = el / n
    nbytes = 2 * T * KVH * HD * 2
    return {"value": round(nbytes / per / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "us_per_call": round(per * 1e6, 1),
            "sample": f"{n} calls of oracle.decode_attention on the headline workload "
                      f"(T {T}, nH {NH}/kvH {KVH}, hd {HD}, f16 cache) over {el:.1f} s, numpy BLAS "
                      f"limited to {threads} threads"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--only-headline", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build's path runs on a single MI355X "
              "(multi-GPU sharding is a design note, not a measured mode)", file=sys.stderr)
        sys.exit(2)
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    import slang_amd as sa

    gen = torch.Generator(device="cuda").manual_seed(2024)
    ms, nbytes, case = decode_case(sa, 4096, 0, 1e6, args.steps, args.warmup, 64, gen)
    gbs = nbytes / (ms * 1e-3) / 1e9
    rec = {
        "metric": "decode attn GB/s (% HBM peak) @KV=4096; prefill attn TFLOP/s (% MFMA) @S=1024",
        "value": round(gbs, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms, 6), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f16", "data": "synthetic",
        "config": {"workload": "decode_2g: BASELINE config 2 global layer, 1 query, nH 8/kvH 2, hd 256, "
                               "KV 4096 f16 cache, q/k RMSNorm+RoPE theta 1e6, 64 rotated caches",
                   "accumulate": "f32", "kv_bytes_per_call": nbytes},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None},
    }
    if not args.only_headline:
        sec = {}
        ms2, nb2, _ = decode_case(sa, 4096, 512, 1e4, args.steps, args.warmup, 64, gen)
        sec["decode_2s"] = {"us_per_call": round(ms2 * 1e3, 3), "GB/s": round(nb2 / ms2 / 1e6, 2),
                            "hbm_frac": round(nb2 / ms2 / 1e6 / HBM_PEAK_GBS, 4), "kv_bytes": nb2}
        for tag, win, th in (("prefill_3g", 0, 1e6), ("prefill_3s", 512, 1e4)):
            msp, fl = prefill_case(sa, 1024, win, th, max(8, args.steps // 8), args.warmup, gen)
            tf = fl / (msp * 1e-3) / 1e12
            sec[tag] = {"us_per_call": round(msp * 1e3, 3), "TFLOP/s": round(tf, 2),
                        "mfma_frac": round(tf / F16_PEAK_TFLOPS, 4), "flops": fl}
        ms4, nb4, toks = batched_decode_case(sa, max(8, args.steps // 16), args.warmup, gen)
        sec["decode_4"] = {"us_per_call": round(ms4 * 1e3, 3), "GB/s": round(nb4 / ms4 / 1e6, 2),
                           "hbm_frac": round(nb4 / ms4 / 1e6 / HBM_PEAK_GBS, 4), "kv_bytes": nb4,
                           "sum_kv_len": toks}
        rec["secondary"] = sec
    if not args.no_cpu_baseline:
        rec["cpu_baseline"] = cpu_baseline(case, args.cpu_seconds)
    print(json.dumps(rec), flush=True)


if __name__ == "__main__":
    main()
