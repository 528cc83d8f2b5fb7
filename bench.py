"""Benchmark of the Gemma 4 E2B attention hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]

Prints ONE JSON line. The headline (`value`) is BASELINE config 2 global: decode
attention, nH 8 / kvH 2, hd 256, KV length 4096, f16 cache, in GB/s of K+V bytes
attended (8,388,608 B per call). A step is one decode call; the timed region
replays a HIP graph of K calls that rotate over 64 distinct KV caches (512 MiB, more
than the 256 MiB Infinity Cache), so every call streams its cache from HBM.
`secondary` carries the other BASELINE rows: config 1 on the GPU (f32 caches, 256
rotated), config 2 sliding (W 512), config 3
prefill (S 1024, global and W 512, TFLOP/s of 4*hd*nH*attended-pairs), config 4
(16 sequences, KV ~ U[1024, 32768]), the q/k/v producer in front of the path (decode
4-bit GEMV at the config-2 layer shape, prefill projection GEMMs at config 3) and the
config-5 35-layer stack. Times come from HIP events on the stream the
kernels run on; the MALL is flushed before every timed replay. `cpu_baseline` is the
numpy oracle on this host for the headline decode and the config-3 global prefill,
min-of-5 at the BLAS default thread count and at one thread.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np
import torch

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E, published
F16_PEAK_TFLOPS = 2500.0     # MI355X dense f16 MFMA, published
NH, KVH, HD = 8, 2, 256


EAGER = False                 # --eager: time plain back-to-back launches instead of a HIP graph


_FLUSH = None


def flush_mall():
    """Evict the 256 MB MALL (Infinity Cache) and the L2s: read 1 GiB that no timed call
    touches, so the first calls of a timed region find nothing of theirs cached. The pass
    only reads: a flush that also wrote the 1 GiB left dirty MALL lines whose write-back
    then ran inside the timed region (the headline measured 20.6 us a call over 20 calls,
    12.7 over 64, against 8.8 over 256)."""
    global _FLUSH
    if _FLUSH is None:
        _FLUSH = torch.empty(256 << 20, dtype=torch.float32, device="cuda")
        _FLUSH.fill_(0.0)
        torch.cuda.synchronize()
    torch.sum(_FLUSH)


WARM_S = 0.3  # seconds of the measured work before each timed region


def warm_clocks(run):
    """Repeat `run` (GPU work, launched asynchronously) until the GPU has been busy with it for
    WARM_S seconds. From idle the MI355X's shader clock takes a few hundred milliseconds to
    reach its ~2.35 GHz (rocm-smi: 104 MHz idle, 1.7 GHz, then 2.33-2.35 GHz at 0.3-s
    samples under load); timed right after a short warm-up, the S 8192 prefill layer read
    341 us a call against 294 us once the clocks were up. A serving GPU runs at the
    sustained clock, which is what the timed regions measure."""
    t0 = time.perf_counter()
    while True:
        run()
        torch.cuda.synchronize()
        if time.perf_counter() - t0 >= WARM_S:
            return


def graph_time_ms(fn_list, steps, warmup, flush=True):
    """Capture `steps` calls (cycling fn_list) in one HIP graph; return mean ms per call.

    The MALL is flushed before the timed replay (flush_mall), so a call whose operands are
    distinct from those of the previous len(fn_list) - 1 calls streams them from HBM: with
    len(fn_list) rotated sets of >= 512 MiB in total, no set is revisited before the MALL has
    been overwritten. With --eager the same calls are launched one by one on the stream
    (for profilers that count per dispatch); the figure then includes host launch gaps.
    """
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for i in range(max(warmup, 1)):
            fn_list[i % len(fn_list)]()
    torch.cuda.synchronize()
    if EAGER:
        with torch.cuda.stream(stream):
            warm_clocks(lambda: [fn() for fn in fn_list])
        ev0 = torch.cuda.Event(enable_timing=True)
        ev1 = torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(stream):
            if flush:
                flush_mall()
            ev0.record(stream)
            for i in range(steps):
                fn_list[i % len(fn_list)]()
            ev1.record(stream)
        torch.cuda.synchronize()
        return ev0.elapsed_time(ev1) / steps
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        for i in range(steps):
            fn_list[i % len(fn_list)]()
    torch.cuda.synchronize()
    warm_clocks(g.replay)           # warm replays (untimed) until the clocks are up
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        # a second warm replay, the flush and the timed replay are queued back to back: the
        # GPU does not idle (and drop its clocks) before the timed region, and the host
        # launches the timed graph while the flush still runs, so the first call starts at ev0
        g.replay()
        if flush:
            flush_mall()
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


def decode_case(sa, T, window, theta, steps, warmup, n_caches, gen, device_len=True):
    """One query at position T-1, its key length in a device array; device_len=False gives
    the length on the host instead (key_len NULL at the C ABI). The two forms measure within
    0.2-0.3 us of each other a call, the faster one changing between boxes and runs."""
    caches = make_caches(sa, n_caches, T, theta, gen)
    q = torch.randn(NH, HD, device="cuda", generator=gen)
    qg = 1 + 0.1 * torch.randn(HD, device="cuda", generator=gen)
    cos, sin = sa.rope_tables([T - 1], HD, theta)
    kl = torch.tensor([T], dtype=torch.int32, device="cuda") if device_len else [T]
    cfg = sa.AttnConfig(NH, KVH, HD, window)
    ws = sa.DecodeWorkspace("cuda")
    out = torch.empty(1, NH, HD, device="cuda")
    fns = [lambda kc=kc, vc=vc: sa.decode(q, kc, vc, kl, cfg, q_gain=qg, rope_cos=cos, rope_sin=sin,
                                          out=out, workspace=ws, max_key_len=T) for kc, vc in caches]
    ms = graph_time_ms(fns, steps, warmup)
    attended = min(T, window) if window else T
    nbytes = 2 * attended * KVH * HD * 2
    return ms, nbytes, (q, qg, cos, sin, caches[0], cfg)


def config1_case(sa, steps, warmup, gen, n_caches=256):
    """BASELINE config 1 on the GPU: nH 4 / kvH 1, hd 256, T 1024, f32 caches (the
    reference's own cache type), scale 1/16, no norms or RoPE; n_caches rotated 2 MiB caches
    (512 MiB, beyond the MALL)."""
    T, nh, kvh, hd = 1024, 4, 1, 256
    caches = [(torch.randn(T, kvh, hd, device="cuda", generator=gen),
               torch.randn(T, kvh, hd, device="cuda", generator=gen)) for _ in range(n_caches)]
    q = torch.randn(nh, hd, device="cuda", generator=gen)
    kl = torch.tensor([T], dtype=torch.int32, device="cuda")
    cfg = sa.AttnConfig(nh, kvh, hd, 0, 1.0 / 16)
    ws = sa.DecodeWorkspace("cuda")
    out = torch.empty(1, nh, hd, device="cuda")
    fns = [lambda kc=kc, vc=vc: sa.decode(q, kc, vc, kl, cfg, out=out, workspace=ws) for kc, vc in caches]
    ms = graph_time_ms(fns, steps, warmup)
    return ms, 2 * T * kvh * hd * 4


def prefill_case(sa, S, window, theta, steps, warmup, gen, nH=NH, kvH=KVH, hd=HD, kv32=False, hilo=False):
    """One layer's prefill attention over S tokens (config 3 by default). The other modes:
    kv32 f32 caches (the reference's own cache type), hilo the f32-q attn_prefill form, hd
    512 with nH 8 / kvH 1 the global layers of Gemma 4 E2B; their caches hold N(0,1) rows."""
    q = torch.randn(S, nH, hd, device="cuda", generator=gen)
    qg = 1 + 0.1 * torch.randn(hd, device="cuda", generator=gen)
    cos, sin = sa.rope_tables(np.arange(S), hd, theta)
    if (nH, kvH, hd, kv32) == (NH, KVH, HD, False):
        kc, vc = make_caches(sa, 1, S, theta, gen)[0]
    else:
        kc = torch.randn(S, kvH, hd, device="cuda", generator=gen)
        vc = torch.randn(S, kvH, hd, device="cuda", generator=gen)
        if not kv32:
            kc, vc = kc.half(), vc.half()
    cfg = sa.AttnConfig(nH, kvH, hd, window)
    out = torch.empty(S, nH, hd, device="cuda", dtype=torch.float16)
    ws = sa.DecodeWorkspace("cuda")
    fn = lambda: sa.prefill(q, kc, vc, 0, cfg, q_gain=qg, rope_cos=cos, rope_sin=sin, out=out,  # noqa: E731
                            q_hilo=hilo, workspace=ws)
    ms = graph_time_ms([fn], steps, warmup)
    pairs = sum(min(p + 1, window) if window else p + 1 for p in range(S))
    flops = 4 * hd * nH * pairs
    host = tuple(x.cpu().numpy() for x in (q, qg, kc, vc, cos, sin)) + (flops,)
    return ms, flops, host


# the prefill modes beside config 3's default (tag: prefill_case keywords): the fused form's
# f32 q (hilo), the GEMM form on f32 caches (f32kv: both caches rounded to f16 as its srqh_b
# does), the fused form on its own f32 caches (fused32: f32 q, K at f32 accuracy), hd 512
PREFILL_MODES = {"hilo": dict(hilo=True), "f32kv": dict(kv32=True), "fused32": dict(kv32=True, hilo=True),
                 "hd512": dict(nH=8, kvH=1, hd=512)}


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


def stack_case(sa, gen, S=8192, steps=256, n_layers=35):
    """35 layers (4 sliding(512) then 1 global, repeated), prefill of S
    tokens then `steps` decode steps against the growing f16 caches, one cache per layer.

    Each layer's prefill is kv_write(S rows) + prefill; each decode step per layer is one
    decode call with the row's KV write fused in (g4a_decode_kv). Both phases are timed
    as whole-stack HIP graphs. q and the raw k/v rows are N(0,1) (the projections that
    would produce them are not part of the attention path). Returns per-phase totals and
    per-layer-type figures.
    """
    T = S + steps
    kinds = ["global" if (i % 5) == 4 else "sliding" for i in range(n_layers)]
    theta = {"global": 1e6, "sliding": 1e4}
    win = {"global": 0, "sliding": 512}
    tabs = {k: sa.rope_tables(np.arange(T), HD, theta[k]) for k in theta}
    cfgs = {k: sa.AttnConfig(NH, KVH, HD, win[k]) for k in theta}
    kvcfg = sa.AttnConfig(KVH, KVH, HD)
    qg = 1 + 0.1 * torch.randn(HD, device="cuda", generator=gen)
    kg = 1 + 0.1 * torch.randn(HD, device="cuda", generator=gen)
    qp = torch.randn(S, NH, HD, device="cuda", generator=gen)
    kp = torch.randn(S, KVH, HD, device="cuda", generator=gen).half()
    vp = torch.randn(S, KVH, HD, device="cuda", generator=gen).half()
    qd = torch.randn(NH, HD, device="cuda", generator=gen)
    kd = torch.randn(steps, KVH, HD, device="cuda", generator=gen)
    vd = torch.randn(steps, KVH, HD, device="cuda", generator=gen)
    caches = [(torch.zeros(T, KVH, HD, device="cuda", dtype=torch.float16),
               torch.zeros(T, KVH, HD, device="cuda", dtype=torch.float16)) for _ in range(n_layers)]
    outp = torch.empty(S, NH, HD, device="cuda", dtype=torch.float16)
    outd = torch.empty(1, NH, HD, device="cuda")
    kl = torch.arange(S + 1, T + 1, dtype=torch.int32, device="cuda")
    ws = sa.DecodeWorkspace("cuda")

    def prefill_layer(i):
        kc, vc = caches[i]
        c, sn = tabs[kinds[i]]
        sa.kv_write(kp, vp, kc, vc, 0, kvcfg, k_gain=kg, rope_cos=c[:S], rope_sin=sn[:S])
        sa.prefill(qp, kc, vc, 0, cfgs[kinds[i]], q_gain=qg, rope_cos=c[:S], rope_sin=sn[:S], out=outp,
                   workspace=ws)

    def decode_layer(i, t, fused=True):
        kc, vc = caches[i]
        c, sn = tabs[kinds[i]]
        p = S + t
        if fused:  # g4a_decode_kv: the step's KV write inside the decode call
            sa.decode(qd, kc, vc, kl[t:t + 1], cfgs[kinds[i]], q_gain=qg, rope_cos=c[p:p + 1],
                      rope_sin=sn[p:p + 1], out=outd, workspace=ws, max_key_len=p + 1,
                      k_new=kd[t], v_new=vd[t], k_gain=kg)
            return
        sa.kv_write(kd[t:t + 1], vd[t:t + 1], kc, vc, p, kvcfg, k_gain=kg,
                    rope_cos=c[p:p + 1], rope_sin=sn[p:p + 1])
        sa.decode(qd, kc, vc, kl[t:t + 1], cfgs[kinds[i]], q_gain=qg, rope_cos=c[p:p + 1],
                  rope_sin=sn[p:p + 1], out=outd, workspace=ws, max_key_len=p + 1)

    pre_ms = graph_time_ms([lambda: [prefill_layer(i) for i in range(n_layers)]], 1, 1)
    dec_ms = graph_time_ms([lambda: [decode_layer(i, t) for t in range(steps) for i in range(n_layers)]], 1, 0)
    # per-layer-type figures: one layer of each kind (the same calls, graphs of their own)
    per = {}
    for kind, li in (("global", 4), ("sliding", 0)):
        pm = graph_time_ms([lambda li=li: prefill_layer(li)], 16, 2)
        dm = graph_time_ms([lambda li=li: [decode_layer(li, t) for t in range(steps)]], 1, 0) / steps
        dms = graph_time_ms([lambda li=li: [decode_layer(li, t, False) for t in range(steps)]], 1, 0) / steps
        pairs = sum(min(p + 1, win[kind]) if win[kind] else p + 1 for p in range(S))
        dbytes = sum(2 * (min(S + t + 1, win[kind]) if win[kind] else S + t + 1) * KVH * HD * 2
                     for t in range(steps)) / steps
        per[kind] = {"prefill_us": round(pm * 1e3, 2),
                     "prefill_TFLOP/s": round(4 * HD * NH * pairs / (pm * 1e-3) / 1e12, 2),
                     "decode_step_us": round(dm * 1e3, 3),
                     "decode_GB/s": round(dbytes / (dm * 1e-3) / 1e9, 2),
                     "decode_step_us_kv_write_separate": round(dms * 1e3, 3)}
    return {"layers": n_layers, "S": S, "decode_steps": steps,
            "prefill_ms_35_layers": round(pre_ms, 3),
            "decode_ms_per_step_35_layers": round(dec_ms / steps, 4),
            "per_layer": per,
            "note": "prefill per layer = kv_write(S) + prefill; decode per layer-step = decode with the "
                    "step's KV write fused in (g4a_decode_kv); the separate kv_write(1) + decode figure "
                    "is given beside it"}


def e2b_manifest(seed=0, vocab=262144, n_layers=35, H=1536, nH=8, ple_d=256, window=512, wide_from=15):
    """A Gemma 4 E2B-shaped model in the exported format (export.py:64-181), built in host
    memory over random weights (no checkpoint): 35 layers, every fifth global (hd 512,
    partial RoPE cutoff 64, theta 1e6), the others sliding (hd 256, W 512, theta 1e4),
    nH 8 / kvH 1, layers 15.. sharing the caches of layers 13/14, 4-bit q/k/v/o, the MLP as
    the QAT checkpoint packs it (loader.py:25, prefill_gpu.py:191-192): intermediate 6144 at
    4 bits on layers 0-14, the double-wide 12288 at 2 bits on layers 15-34 (the runner's
    gateup_95 / down_96 path, runner.py:448-458), int8 per-layer-embedding linears, 2-bit
    lm_head over 262144 tokens. Packed rows are uniform random bytes, i.e. uniform codes of
    any width."""
    from slang_amd.manifest import Manifest
    rng = np.random.default_rng(seed)
    parts, tensors, pos, keep = [], {}, 0, {}

    def put(name, arr, dt):
        nonlocal pos
        arr = np.ascontiguousarray(arr)
        keep[name] = arr  # the bytes below are a view: contents may still be set until the end
        b = arr.view(np.uint8).reshape(-1)
        tensors[name] = {"off": pos, "len": int(b.size), "dtype": dt, "shape": list(arr.shape)}
        parts.append(b)
        pos += b.size
        if pos % 4:
            parts.append(np.zeros(4 - pos % 4, np.uint8))
            pos += 4 - pos % 4

    rbytes = lambda n_out, nb: np.frombuffer(rng.bytes(n_out * nb), np.uint8).reshape(n_out, nb)  # noqa: E731
    rows = lambda n_out, n_in, bits: rbytes(n_out, n_in * bits // 8).view(np.uint32)  # noqa: E731
    gains = lambda n: (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)  # noqa: E731
    rsc = lambda n, s: (s * (1 + 0.2 * rng.random(n))).astype(np.float32)  # noqa: E731
    put("embed_q", rbytes(vocab, H // 4), "u8")
    put("embed_scale", rsc(vocab, 0.02), "f32")
    put("ple_q", rbytes(vocab, n_layers * ple_d // 2), "u8")
    put("ple_scale", rsc(vocab * n_layers, 0.05), "f32")
    put("lmhead_blk", rows(H // 64 * vocab, 128, 1).reshape(H // 64, vocab, 4), "u32")
    put("lmhead_scale", rsc(vocab, 0.02), "f32")
    put("pl_model_proj", (0.02 * rng.standard_normal((n_layers * ple_d, H))).astype(np.float16), "f16")
    put("final_norm", gains(H), "f32")
    put("pl_proj_norm", gains(ple_d), "f32")
    layers, first_shared = [], 15
    for L in range(n_layers):
        glob = L % 5 == 4
        hd = 512 if glob else 256
        shared = L >= first_shared
        src = L if not shared else (14 if glob else 13)
        q_dim = nH * hd
        for n, a in (("in_norm", gains(H)), ("q_norm", gains(hd)), ("o_w12", gains(2 * H)),
                     ("down_nw", gains(H)), ("pleproj_w12s", np.append(gains(2 * H), np.float32(0.8)))):
            put(f"L{L}.{n}", a, "f32")
        put(f"L{L}.q_bits", rows(q_dim, H, 4), "u32")
        if shared:
            put(f"L{L}.q_scale", rsc(q_dim, 0.01), "f32")
        else:
            put(f"L{L}.k_norm", gains(hd), "f32")
            put(f"L{L}.k_bits", rows(hd, H, 4), "u32")
            put(f"L{L}.v_bits", rows(hd, H, 4), "u32")
            put(f"L{L}.qkv_scales", rsc(q_dim + 2 * hd, 0.01), "f32")
        put(f"L{L}.o_bits", rows(H, q_dim, 4), "u32")
        put(f"L{L}.o_scale", rsc(H, 0.01), "f32")
        inter, mlp_bits = (6144, 4) if L < wide_from else (12288, 2)
        for tag, n_out, n_in in (("gate", inter, H), ("up", inter, H), ("down", H, inter)):
            put(f"L{L}.{tag}_bits", rows(n_out, n_in, mlp_bits), "u32")
            put(f"L{L}.{tag}_scale", rsc(n_out, 0.01), "f32")
        for tag, n_out, n_in in (("plegate", ple_d, H), ("pleproj", H, ple_d)):
            put(f"L{L}.{tag}_codes", rows(n_out, n_in, 8), "u32")
            put(f"L{L}.{tag}_rowscale", rsc(n_out, 0.002), "f32")
        sc = {"qkv_in": 0.05, "q_out": 0.02, "o_in": 0.01, "o_out": 0.05, "gate_in": 0.05, "gate_out": 0.02,
              "up_in": 0.04, "up_out": 0.02, "down_in": 0.01, "down_out": 0.02, "plegate_in": 0.05,
              "plegate_out": 0.03, "pleproj_in": 0.03, "pleproj_out": 0.01}
        if not shared:
            sc.update(k_out=0.02, v_out=0.02)
        # the GELU tables of the two gate grids, as export.py:30-33 writes them (:150, :161)
        for tag, step in (("gate", sc["gate_out"]), ("plegate", sc["plegate_out"])):
            gv = (np.arange(256) - 128).astype(np.float64) * step
            put(f"L{L}.gelu_{tag}",
                (0.5 * gv * (1.0 + np.tanh(0.7978845608028654 * (gv + 0.044715 * gv ** 3)))).astype(np.float32), "f32")
        layers.append({"index": L, "sliding": not glob, "head_dim": hd, "q_dim": q_dim, "intermediate": inter,
                       "shared": shared, "kv_source": src, "rope_theta": 1e6 if glob else 1e4,
                       "rope_cutoff": 64 if glob else hd // 2, "scales": sc})
    for L in range(n_layers):  # export.py:110, 119-122: the next layer's input norm (the final norm last)
        keep[f"L{L}.pleproj_w12s"][H:2 * H] = keep[f"L{L + 1}.in_norm"] if L + 1 < n_layers else keep["final_norm"]
    meta = {"config": {"H": H, "nL": n_layers, "nH": nH, "vocab": vocab, "window": window, "softcap": 30.0,
                       "ple_d": ple_d, "embed_scale": float(np.sqrt(H)), "ple_scale": float(np.sqrt(ple_d)),
                       "bos": 2, "eos": 1},
            "layers": layers, "tensors": tensors, "bytes": pos}
    return Manifest(meta, np.concatenate(parts))


def decoder_case(steps=32, T=4096):
    """Resident greedy decode of the E2B-shaped model (e2b_manifest): `steps` consecutive
    tokens at positions T.., each step's token the previous step's device argmax, captured
    as one HIP graph. Returns ms per token and the bytes one token must read (every weight
    row once, the attended K/V rows, the lm_head and the per-layer-input projection)."""
    from slang_amd.decoder import DecoderStack
    man = e2b_manifest()
    st = DecoderStack(man, max_seq=T + steps + 1)
    del man
    st.tok.fill_(2)
    ms = graph_time_ms([lambda: [st.step(T + t) for t in range(steps)]], 1, 1) / steps
    wbytes = sum(t.numel() * t.element_size() for w in st.w for k, t in w.items()
                 if isinstance(t, torch.Tensor) and k.endswith(("_bits", "_codes")))
    wbytes += sum(t.numel() * t.element_size() for w in st.attn.w.values() for k, t in w.items() if k.endswith("_bits"))
    wbytes += st.lm_rows.numel() * 4 + st.pl_proj.numel() * 2
    kv = 0
    for s in st.man.layers:
        rows = T + steps // 2 + 1  # the middle step's key count
        rows = min(rows, st.man.window) if s.sliding else rows
        kv += 2 * rows * st.man.n_kv_heads(s.index) * s.head_dim * 2
    pre = decoder_prefill_case(st)
    gen = generate_case(st)
    return ms, wbytes + kv, wbytes, kv, (pre, gen)


def generate_case(st, S=1024, n_new=64):
    """Prompt to tokens on the device (DecoderStack.generate, the reference's generate_resident,
    runner.py:542-569): the layers-outer prefill of S - 1 prompt tokens, then n_new greedy
    steps from the last one, every token kept on the GPU, the whole call one HIP graph.
    Returns ms per call."""
    ids = torch.randint(0, st.vocab, (S,), generator=torch.Generator().manual_seed(7)).to(torch.int32).cuda()
    st.generate(ids, n_new)  # sizes the prefill buffers before the capture
    torch.cuda.synchronize()
    return graph_time_ms([lambda: st.generate(ids, n_new)], 1, 1), S, n_new


def generate_row(gen):
    ms, S, n_new = gen
    return {"ms_per_call": round(ms, 3), "prompt_tokens": S, "new_tokens": n_new,
            "tokens/s": round(n_new / ms * 1e3, 1), "note": "prefill of the prompt's first S-1 tokens "
            "(layers outer), then greedy decode steps from its last token with every token kept on the "
            "GPU (DecoderStack.generate), one HIP graph per call"}


def decoder_prefill_case(st, S=1024, reps=4):
    """The layers-outer batched prefill of the same model (DecoderStack.prefill, the reference's
    PrefillGPU.prefill): an S-token prompt through all 35 layers, the token ids on the device,
    one prompt per step of a HIP graph. Returns ms per prompt and the FLOPs of its GEMMs
    (every linear over S rows) and of its attention (4*hd*nH*attended pairs per layer)."""
    man = st.man
    H, nL, d = st.H, st.nL, st.d
    ids = torch.randint(0, st.vocab, (S,), dtype=torch.int32, device="cuda")
    st.prefill(ids, 0)  # dequantises every layer's weights once (kept resident), sizes the buffers
    torch.cuda.synchronize()
    ms = graph_time_ms([lambda: st.prefill(ids, 0)], reps, 1)
    gemm = 2 * S * H * nL * d
    att = 0
    for s in man.layers:
        kv = 0 if s.shared else man.kv_dim(s.index)
        gemm += 2 * S * H * (s.q_dim + 2 * kv) + 2 * S * s.q_dim * H + 3 * 2 * S * H * s.intermediate + 2 * 2 * S * H * d
        W = man.window if s.sliding else 0
        pairs = sum(min(p + 1, W) if W else p + 1 for p in range(S))
        att += 4 * s.head_dim * s.n_q_heads * pairs
    return ms, gemm, att


def qkv_gemv_case(sa, steps, warmup, gen, n_sets=128):
    """Decode q/k/v projections of one token (qkv_70) at the config-2 layer shape: H 1536,
    q 8x256, k/v 2x256 rows of 4-bit weights; n_sets distinct weight sets (302 MB, more
    than the 256 MB Infinity Cache) rotate so every call streams its weights from HBM."""
    H, qd, kvd = 1536, NH * HD, KVH * HD
    words = lambda rows: torch.randint(-2**31, 2**31 - 1, (rows * H // 8,), device="cuda",  # noqa: E731
                                       dtype=torch.int32, generator=gen)
    sets = [(words(qd), words(kvd), words(kvd)) for _ in range(n_sets)]
    sc = 0.01 * torch.rand(qd + 2 * kvd, device="cuda", generator=gen)
    a = torch.randn(H, device="cuda", generator=gen)
    sa_ = a.sum().reshape(1)
    oq = torch.empty(qd, device="cuda")
    ok = torch.empty(kvd, device="cuda")
    ov = torch.empty(kvd, device="cuda")
    fns = [lambda w=w: sa.qkv_gemv(a, sa_, w[0], sc, qd, kvd, k_bits=w[1], v_bits=w[2], q_out=0.02,
                                   k_out=0.02, v_out=0.02, out_q=oq, out_k=ok, out_v=ov) for w in sets]
    ms = graph_time_ms(fns, steps, warmup)
    return ms, (qd + 2 * kvd) * H // 2


def proj_case(sa, steps, warmup, gen, S=1024):
    """Prefill q/k/v projections at config 3 (S 1024 tokens, H 1536 -> q 2048, k 512, v 512)
    on dequantised f16 weights: srqh_b of the input, then the three GEMMs of one layer."""
    H = 1536
    a = torch.randn(S, H, device="cuda", generator=gen)
    wq = (0.02 * torch.randn(NH * HD, H, device="cuda", generator=gen)).half()
    wk = (0.02 * torch.randn(KVH * HD, H, device="cuda", generator=gen)).half()
    wv = (0.02 * torch.randn(KVH * HD, H, device="cuda", generator=gen)).half()
    a16 = torch.empty(S, H, device="cuda", dtype=torch.float16)
    oq = torch.empty(S, NH * HD, device="cuda")
    ok = torch.empty(S, KVH * HD, device="cuda", dtype=torch.float16)
    ov = torch.empty_like(ok)

    def fn():  # prefill_qkv: srqh_b once, then the three GEMMs in one launch
        sa.srqh(a, 0.05, out=a16)
        sa.gemm16(a16, [(wq, oq, 0.02), (wk, ok, None), (wv, ov, None)])
    ms = graph_time_ms([fn], steps, warmup)
    return ms, 2 * S * H * (NH * HD + 2 * KVH * HD)


def prefill_row(pre, S=1024):
    ms, gemm, att = pre
    return {"ms_per_prompt": round(ms, 3), "prompt_tokens": S, "tokens/s": round(S / ms * 1e3, 1),
            "gemm_TFLOP/s": round(gemm / ms / 1e9, 2), "attention_TFLOP/s": round(att / ms / 1e9, 2),
            "mfma_frac": round((gemm + att) / ms / 1e9 / F16_PEAK_TFLOPS, 4), "gemm_flops": gemm,
            "attention_flops": att,
            "note": "layers-outer batched prefill of the E2B-shaped synthetic model (35 layers): every "
                    "linear one f16 GEMM over the prompt (weights dequantised once, kept resident), "
                    "batched causal attention, the row tails between them; a HIP graph of whole prompts"}


def copy_calibration(steps):
    """A plain elementwise kernel of known traffic (torch.neg over 256 MiB f16: 256 MiB read,
    256 MiB written per launch) for scaling FETCH_SIZE / WRITE_SIZE counter readings."""
    n = 128 << 20
    src = torch.randn(n, device="cuda").half()
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(steps):
        torch.neg(src, out=dst)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration": "torch.neg f16", "read_bytes": 2 * n, "write_bytes": 2 * n,
                      "launches": steps}), flush=True)


def roofline_probes(steps, warmup):
    """Measured denominators beside the published peaks (the library's roofline probes,
    g4a_probe_read / g4a_probe_mfma): a read-only stream of 8 MiB, 64 MiB and 512 MiB, each
    call on a region no call in the previous 1 GiB touched (the MALL flushed first, so every
    call reads cold from HBM), best over 256-2048 workgroups; and 32x32x16 f16 MFMAs from
    registers on every SIMD (2 and 4 waves a SIMD, the better). Returns the JSON object."""
    from slang_amd import _lib
    lib = _lib.load()
    sink = torch.empty(lib.g4a_probe_sink_bytes(), dtype=torch.uint8, device="cuda")
    arena = torch.ones(1 << 30, dtype=torch.uint8, device="cuda")
    base = arena.data_ptr()

    def check(rc):
        if rc != 0:
            raise RuntimeError(f"probe: {lib.g4a_last_error().decode()}")

    def stream():
        return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    out = {}
    for mib in (8, 64, 512):
        size, n = mib << 20, max(2, 1024 // mib)
        best = None
        for wg in (256, 512, 1024, 2048):
            fns = [lambda off=i * size, wg=wg: check(lib.g4a_probe_read(ctypes.c_void_p(base + off), size, wg,
                                                                         ctypes.c_void_p(sink.data_ptr()), stream()))
                   for i in range(n)]
            ms = graph_time_ms(fns, max(n, 16), warmup)
            if best is None or ms < best[0]:
                best = (ms, wg)
        out[f"read_{mib}MiB"] = {"us": round(best[0] * 1e3, 3), "GB/s": round(size / best[0] / 1e6, 1),
                                 "workgroups": best[1]}
    iters, best = 2000, None
    for wgs in (256, 512):  # one or two 512-thread workgroups a CU: 2 or 4 waves a SIMD
        fn = lambda wgs=wgs: check(lib.g4a_probe_mfma(wgs, iters, ctypes.c_void_p(sink.data_ptr()), stream()))  # noqa: E731
        ms = graph_time_ms([fn], 4, 1, flush=False)
        tf = wgs * 8 * iters * 8 * 32768 / (ms * 1e-3) / 1e12
        if best is None or tf > best[0]:
            best = (tf, wgs)
    out["mfma_f16"] = {"TFLOP/s": round(best[0], 1), "workgroups": best[1], "waves_per_simd": best[1] // 128}
    del arena
    torch.cuda.empty_cache()
    return {"hbm_GB/s": out["read_512MiB"]["GB/s"], "read_8MiB_cold_us": out["read_8MiB"]["us"],
            "mfma_f16_TFLOP/s": out["mfma_f16"]["TFLOP/s"], "detail": out,
            "note": "measured on this GPU by the library's roofline probes: a read-only 16-byte "
                    "non-temporal stream (cold: 1 GiB rotation, MALL flushed) and register-operand "
                    "v_mfma_f32_32x32x16_f16 on every SIMD; the published peaks stay `peak`"}


def load_traffic():
    """HBM bytes per decode call from the committed PMC summary (profiles/traffic.json), or None."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "traffic.json")
    try:
        with open(path) as f:
            return json.load(f).get("decode_2g", {}).get("bytes_per_call")
    except (OSError, ValueError):
        return None


def _blas_info():
    """The BLAS numpy is built against (numpy.show_config) and its thread pools right now."""
    blas = "unknown"
    try:
        cfg = np.show_config(mode="dicts")
        dep = cfg.get("Build Dependencies", {}).get("blas", {})
        blas = f"{dep.get('name', '?')} {dep.get('version', '')}".strip()
    except Exception:  # pragma: no cover - older numpy
        pass
    try:
        from threadpoolctl import threadpool_info
        threads = max((p.get("num_threads", 1) for p in threadpool_info() if p.get("user_api") == "blas"),
                      default=1)
    except ImportError:  # pragma: no cover
        threads = None
    return blas, threads


def _min_of(fn, reps=5, min_s=2.5):
    """min and median of at least `reps` timed calls (and at least `min_s` seconds of them)
    after one warm-up call (time.perf_counter)."""
    fn()
    ts = []
    while len(ts) < reps or sum(ts) < min_s:
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return min(ts), float(np.median(ts))


def cpu_baseline(case, prefill_inputs):
    """The numpy oracle (oracle/attention.py) on this host, timed as the build's CPU baseline
    protocol asks: min-of-5 after a warm-up, at the BLAS library's default thread count (this
    host's share of cores) and at one thread, for the headline decode call and for the
    config-3 global prefill (S 1024). `value` is the headline decode at the default threads."""
    import oracle.attention as O
    from threadpoolctl import threadpool_limits
    q, qg, cos, sin, (kc, vc), cfg = case
    qn, qgn = q.cpu().numpy(), qg.cpu().numpy()
    c, s = cos.cpu().numpy()[0], sin.cpu().numpy()[0]
    k, v = kc.cpu().numpy(), vc.cpu().numpy()
    T = k.shape[0]
    nbytes = 2 * T * KVH * HD * 2
    pq, pqg, pk, pv, pcos, psin, pflops = prefill_inputs
    blas, default_threads = _blas_info()

    def dec():
        O.decode_attention(qn, k, v, T, KVH, q_gain=qgn, cos=c, sin=s, window=cfg.window)

    def pre():
        O.prefill_attention(pq, pk, pv, 0, KVH, q_gain=pqg, cos=pcos, sin=psin)

    res = {}
    for tag, limit in (("default", None), ("one_thread", 1)):
        ctx = threadpool_limits(limits=limit) if limit else None
        try:
            dmin, dmed = _min_of(dec)
            pmin, pmed = _min_of(pre)
        finally:
            if ctx is not None:
                ctx.__exit__(None, None, None)
        res[tag] = {"threads": limit or default_threads,
                    "decode_2g_us_min": round(dmin * 1e6, 1), "decode_2g_us_median": round(dmed * 1e6, 1),
                    "decode_2g_GB/s": round(nbytes / dmin / 1e9, 3),
                    "prefill_3g_ms_min": round(pmin * 1e3, 2), "prefill_3g_ms_median": round(pmed * 1e3, 2),
                    "prefill_3g_GFLOP/s": round(pflops / pmin / 1e9, 2)}
    d = res["default"]
    return {"value": d["decode_2g_GB/s"], "unit": "GB/s", "cores": d["threads"], "kind": "port",
            "us_per_call": d["decode_2g_us_min"], "cpu_count": os.cpu_count(), "blas": blas,
            "one_thread": res["one_thread"], "default_threads": d,
            "sample": f"oracle.decode_attention on the headline workload (T {T}, nH {NH}/kvH {KVH}, hd {HD}, f16 "
                      f"cache) and oracle.prefill_attention on config 3 global (S 1024), each the minimum of >= 5 "
                      f"calls (>= 2.5 s) after a warm-up, at the BLAS default of {d['threads']} threads ({blas}; os.cpu_count() "
                      f"{os.cpu_count()}) and at 1 thread"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--only-headline", action="store_true")
    ap.add_argument("--no-stack", action="store_true", help="skip the 35-layer config 5 stack")
    ap.add_argument("--no-decoder", action="store_true", help="skip the E2B-shaped whole-decoder step")
    ap.add_argument("--decoder-only", action="store_true", help="only the whole-decoder step row")
    ap.add_argument("--eager", action="store_true",
                    help="launch calls one by one instead of replaying a HIP graph (for profilers)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a known-size copy kernel (counter calibration) and exit")
    ap.add_argument("--prefill-only", action="store_true",
                    help="only the config 3 prefill rows (for profiling the prefill kernel)")
    ap.add_argument("--prefill-seq", type=int, default=1024,
                    help="prompt length of the --prefill-only rows (1024 = config 3, 8192 = config 5's layer)")
    ap.add_argument("--prefill-mode", default="f16", choices=["f16"] + list(PREFILL_MODES),
                    help="the --prefill-only rows' mode: config 3 as is, its f32-q (hilo) form, f32 caches, "
                         "or hd 512 (nH 8 / kvH 1, the E2B global layers)")
    ap.add_argument("--batched-only", action="store_true",
                    help="only the config 4 batched decode row (for profiling its kernels)")
    ap.add_argument("--decode-only", action="store_true",
                    help="only single-sequence decode rows (2G, 2S, T 16K / 32K, T 8448) for profiling")
    ap.add_argument("--roofline-only", action="store_true",
                    help="only the measured roofline denominators (read-only stream, MFMA loop)")
    args = ap.parse_args()
    global EAGER
    EAGER = args.eager
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build's path runs on a single MI355X "
              "(multi-GPU sharding is a design note, not a measured mode)", file=sys.stderr)
        sys.exit(2)
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    import slang_amd as sa

    if args.copy_calibration:
        copy_calibration(max(args.steps, 1))
        return
    gen = torch.Generator(device="cuda").manual_seed(2024)
    if args.prefill_only:
        out = {}
        cfgn = "3" if args.prefill_seq == 1024 else f"S{args.prefill_seq}"
        mkw = PREFILL_MODES.get(args.prefill_mode, {})
        sfx = "" if args.prefill_mode == "f16" else f"_{args.prefill_mode}"
        for tag, win, th in ((f"prefill_{cfgn}g{sfx}", 0, 1e6), (f"prefill_{cfgn}s{sfx}", 512, 1e4)):
            msp, fl, _ = prefill_case(sa, args.prefill_seq, win, th, args.steps, args.warmup, gen, **mkw)
            out[tag] = {"us_per_call": round(msp * 1e3, 3), "TFLOP/s": round(fl / msp / 1e9, 2)}
        print(json.dumps(out), flush=True)
        return
    if args.decoder_only:
        msd, nbd, wb, kvb, (pre, gen) = decoder_case()
        print(json.dumps({"decoder_e2b": {"ms_per_token": round(msd, 4), "GB/s": round(nbd / msd / 1e6, 2),
                                          "weight_bytes": wb, "kv_bytes": kvb},
                          "decoder_e2b_prefill": prefill_row(pre), "decoder_e2b_generate": generate_row(gen)}),
              flush=True)
        return
    if args.roofline_only:
        print(json.dumps({"peak_measured": roofline_probes(args.steps, args.warmup)}), flush=True)
        return
    if args.decode_only:
        out = {}
        for tag, T, win, th, n in (("decode_2g", 4096, 0, 1e6, 64), ("decode_2s", 4096, 512, 1e4, 64),
                                   ("decode_1seq_16k", 16384, 0, 1e6, 16), ("decode_1seq_32k", 32768, 0, 1e6, 8),
                                   ("decode_5g", 8448, 0, 1e6, 32)):
            msd, nbd, _ = decode_case(sa, T, win, th, max(args.steps, 2 * n), args.warmup, n, gen)
            out[tag] = {"us_per_call": round(msd * 1e3, 3), "GB/s": round(nbd / msd / 1e6, 2)}
        print(json.dumps(out), flush=True)
        return
    if args.batched_only:
        ms4, nb4, toks = batched_decode_case(sa, args.steps, args.warmup, gen)
        print(json.dumps({"decode_4": {"us_per_call": round(ms4 * 1e3, 3), "GB/s": round(nb4 / ms4 / 1e6, 2),
                                       "sum_kv_len": toks}}), flush=True)
        return
    ms, nbytes, case = decode_case(sa, 4096, 0, 1e6, args.steps, args.warmup, 64, gen)
    gbs = nbytes / (ms * 1e-3) / 1e9
    rec = {
        "metric": "decode attn GB/s (% HBM peak) @KV=4096; prefill attn TFLOP/s (% MFMA) @S=1024",
        "value": round(gbs, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms, 6), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f16", "data": "synthetic",
        "config": {"workload": "decode_2g: BASELINE config 2 global layer, 1 query, nH 8/kvH 2, hd 256, "
                               "KV 4096 f16 cache, q/k RMSNorm+RoPE theta 1e6, 64 rotated caches",
                   "accumulate": "f32", "kv_bytes_per_call": nbytes,
                   "timing": {"graph_calls": args.steps, "distinct_caches_timed": min(args.steps, 64),
                              "rotation_bytes": 64 * nbytes, "mall_flushed_before_timing": True,
                              "note": "one HIP graph of exactly `steps` calls over 64 rotated caches (512 MiB); "
                                      "1 GiB is read before the timed replay, so every timed call "
                                      "streams a cache that is not in the 256 MB MALL"}},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": load_traffic(),
                     "kernels": "decode_kernel + decode_merge_kernel (one g4a_decode call)"},
    }
    pm = roofline_probes(args.steps, args.warmup)
    rec["roofline"].update({"peak_measured": pm["hbm_GB/s"], "frac_measured": round(gbs / pm["hbm_GB/s"], 4),
                            "floor_8MiB_cold_us": pm["read_8MiB_cold_us"],
                            "note": "peak_measured: a read-only stream of 512 MiB on this GPU; floor_8MiB_cold_us: "
                                    "the same stream over the headline's 8 MiB, cold (see peak_measured)"})
    rec["peak_measured"] = pm
    prefill_host = None
    if not args.only_headline:
        sec = {}
        # HBM-bound rows: at least one call per rotated set in the timed graph, whatever --steps
        hs = max(args.steps, 64)
        ms2, nb2, _ = decode_case(sa, 4096, 512, 1e4, hs, args.warmup, 64, gen)
        msd, _, _ = decode_case(sa, 4096, 0, 1e6, hs, args.warmup, 64, gen, device_len=False)
        sec["decode_2g_host_len"] = {"us_per_call": round(msd * 1e3, 3), "GB/s": round(nbytes / msd / 1e6, 2),
                                     "note": "the headline call with the key length given on the host "
                                             "(key_len NULL at the C ABI)"}
        ms1, nb1 = config1_case(sa, max(args.steps, 256), args.warmup, gen)
        sec["decode_1"] = {"us_per_call": round(ms1 * 1e3, 3), "GB/s": round(nb1 / ms1 / 1e6, 2),
                           "hbm_frac": round(nb1 / ms1 / 1e6 / HBM_PEAK_GBS, 4), "kv_bytes": nb1,
                           "note": "config 1 on the GPU: f32 caches, nH 4/kvH 1, T 1024, scale 1/16"}
        sec["decode_2s"] = {"us_per_call": round(ms2 * 1e3, 3), "GB/s": round(nb2 / ms2 / 1e6, 2),
                            "hbm_frac": round(nb2 / ms2 / 1e6 / HBM_PEAK_GBS, 4), "kv_bytes": nb2,
                            "note": f"{hs} calls over 64 rotated 8 MiB caches, MALL flushed first"}
        sec["decode_1"]["note"] += f"; {max(args.steps, 256)} calls over 256 rotated 2 MiB caches, MALL flushed first"
        for tag, win, th in (("prefill_3g", 0, 1e6), ("prefill_3s", 512, 1e4)):
            msp, fl, host = prefill_case(sa, 1024, win, th, max(8, args.steps // 8), args.warmup, gen)
            if tag == "prefill_3g":
                prefill_host = host
            tf = fl / (msp * 1e-3) / 1e12
            sec[tag] = {"us_per_call": round(msp * 1e3, 3), "TFLOP/s": round(tf, 2),
                        "mfma_frac": round(tf / F16_PEAK_TFLOPS, 4),
                        "mfma_frac_measured": round(tf / pm["mfma_f16_TFLOP/s"], 4), "flops": fl,
                        "note": "one 8 MiB cache re-read by every call (MFMA-bound; the cache of a "
                                "prefill layer was just written by its kv_write)"}
        for mode, mkw in PREFILL_MODES.items():
            cases = (((f"prefill_3g_{mode}", 0, 1e6), (f"prefill_3s_{mode}", 512, 1e4)) if mode != "hd512"
                     else (("prefill_hd512g", 0, 1e6),))  # E2B's hd-512 layers are its global ones
            for tag, win, th in cases:
                msp, fl, _ = prefill_case(sa, 1024, win, th, max(8, args.steps // 8), args.warmup, gen, **mkw)
                tf = fl / (msp * 1e-3) / 1e12
                sec[tag] = {"us_per_call": round(msp * 1e3, 3), "TFLOP/s": round(tf, 2),
                            "mfma_frac": round(tf / F16_PEAK_TFLOPS, 4), "flops": fl,
                            "note": {"hilo": "config 3 in the f32-q attn_prefill form (G4A_Q_HILO)",
                                     "f32kv": "config 3 on f32 caches, GEMM form (caches rounded to f16 as "
                                              "srqh_b does)",
                                     "fused32": "config 3 as attn_prefill on its own f32 caches: f32 q, K at "
                                                "f32 accuracy (high and low f16 parts)",
                                     "hd512": "S 1024 at hd 512, nH 8 / kvH 1 (E2B global layer shape)"}[mode]}
        for T in (16384, 32768):  # one sequence, long context: 512 MiB of rotated caches
            msl, nbl, _ = decode_case(sa, T, 0, 1e6, max(args.steps, 64), args.warmup, (512 << 20) // (T * 2048), gen)
            sec[f"decode_1seq_{T // 1024}k"] = {"us_per_call": round(msl * 1e3, 3), "GB/s": round(nbl / msl / 1e6, 2),
                                                "hbm_frac": round(nbl / msl / 1e6 / HBM_PEAK_GBS, 4),
                                                "hbm_frac_measured": round(nbl / msl / 1e6 / pm["hbm_GB/s"], 4),
                                                "kv_bytes": nbl,
                                                "note": f"one sequence at T {T}, global, nH 8/kvH 2, f16 caches, "
                                                        f"{(512 << 20) // (T * 2048)} rotated caches, MALL flushed first"}
        msh, flh, _ = prefill_case(sa, 8192, 0, 1e6, 4, 1, gen, nH=8, kvH=1, hd=512)
        tfh = flh / (msh * 1e-3) / 1e12
        sec["prefill_hd512g_8k"] = {"us_per_call": round(msh * 1e3, 3), "TFLOP/s": round(tfh, 2),
                                    "mfma_frac": round(tfh / F16_PEAK_TFLOPS, 4),
                                    "mfma_frac_measured": round(tfh / pm["mfma_f16_TFLOP/s"], 4), "flops": flh,
                                    "note": "S 8192 at hd 512, nH 8 / kvH 1, global (E2B global layer shape)"}
        ms4, nb4, toks = batched_decode_case(sa, max(8, args.steps // 16), args.warmup, gen)
        sec["decode_4"] = {"us_per_call": round(ms4 * 1e3, 3), "GB/s": round(nb4 / ms4 / 1e6, 2),
                           "hbm_frac": round(nb4 / ms4 / 1e6 / HBM_PEAK_GBS, 4), "kv_bytes": nb4,
                           "sum_kv_len": toks}
        msg, nbg = qkv_gemv_case(sa, max(args.steps, 128), args.warmup, gen)
        sec["qkv_gemv_2"] = {"us_per_call": round(msg * 1e3, 3), "GB/s": round(nbg / msg / 1e6, 2),
                             "hbm_frac": round(nbg / msg / 1e6 / HBM_PEAK_GBS, 4), "weight_bytes": nbg,
                             "note": "decode q/k/v projections (qkv_70), 4-bit weights, 128 rotated sets"}
        msp, flp = proj_case(sa, max(8, args.steps // 8), args.warmup, gen)
        tfp = flp / (msp * 1e-3) / 1e12
        sec["proj_3"] = {"us_per_call": round(msp * 1e3, 3), "TFLOP/s": round(tfp, 2),
                         "mfma_frac": round(tfp / F16_PEAK_TFLOPS, 4), "flops": flp,
                         "note": "prefill q/k/v projection GEMMs of one layer at S 1024, f16 weights"}
        if not args.no_stack:
            sec["stack_5"] = stack_case(sa, gen)
        if not args.no_decoder:
            msd, nbd, wb, kvb, (pre, gen) = decoder_case()
            sec["decoder_e2b_prefill"] = prefill_row(pre)
            sec["decoder_e2b_generate"] = generate_row(gen)
            sec["decoder_e2b"] = {"ms_per_token": round(msd, 4), "tokens/s": round(1e3 / msd, 1),
                                  "GB/s": round(nbd / msd / 1e6, 2), "hbm_frac": round(nbd / msd / 1e6 / HBM_PEAK_GBS, 4),
                                  "bytes_per_token": nbd, "weight_bytes": wb, "kv_bytes": kvb,
                                  "note": "whole decode step of an E2B-shaped synthetic model (35 layers, "
                                          "vocab 262144, random weights), greedy token resident on the GPU, "
                                          "32 steps at KV ~4096 in one HIP graph"}
        rec["secondary"] = sec
    if not args.no_cpu_baseline:
        if prefill_host is None:
            prefill_host = prefill_case(sa, 1024, 0, 1e6, 8, 2, gen)[2]
        rec["cpu_baseline"] = cpu_baseline(case, prefill_host)
    print(json.dumps(rec), flush=True)


if __name__ == "__main__":
    main()
