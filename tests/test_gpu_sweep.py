"""A seeded random sweep over the shapes the entry points accept, each case checked against
the CPU oracle at the contract tolerance (|d| <= 2e-3 + 1e-2|ref|): decode (single and
batched, global and windowed, f16 and f32 caches, with and without the fused KV write) and
prefill (start_pos > 0, ragged S, windows, group sizes 1-8, hd 256/512). The named tests
elsewhere pin specific cases; this one looks for combinations nobody wrote down. Sizes are
kept small so the oracle finishes in seconds on one host core."""
import numpy as np
import pytest
import torch

import oracle.attention as O
import slang_amd as sa
from helpers import contract_close

pytestmark = pytest.mark.gpu
DEV = "cuda"
WS = sa.Workspace(DEV)  # grows to the largest call; shared by the cases (one stream)
GROUPS = [(2, 2), (4, 1), (4, 2), (8, 2), (8, 1), (8, 8), (2, 1)]


def t(x):
    return torch.from_numpy(np.ascontiguousarray(x)).to(DEV)


def decode_cases(n=24, seed=2024):
    rng = np.random.default_rng(seed)
    for i in range(n):
        nH, kvH = GROUPS[rng.integers(len(GROUPS))]
        hd = int(rng.choice([256, 512]))
        B = int(rng.choice([1, 1, 2, 5]))
        lens = rng.integers(1, 1500, size=B).astype(np.int32)
        W = int(rng.choice([0, 0, 64, 333]))
        f32 = bool(rng.random() < 0.25)
        fused = bool(rng.random() < 0.4)
        yield pytest.param(i, nH, kvH, hd, lens, W, f32, fused, id=f"d{i}-{nH}/{kvH}-hd{hd}-B{B}-W{W}"
                           f"{'-f32' if f32 else ''}{'-kv' if fused else ''}")


@pytest.mark.parametrize("i,nH,kvH,hd,lens,W,f32,fused", list(decode_cases()))
def test_decode_sweep(i, nH, kvH, hd, lens, W, f32, fused):
    rng = np.random.default_rng(1000 + i)
    B, T = len(lens), int(lens.max()) + 2
    cdt = np.float32 if f32 else np.float16
    q = rng.standard_normal((B, nH, hd)).astype(np.float32)
    qg = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    kg = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    c, s = O.rope_tables(lens - 1, hd, 1e4)
    k = rng.standard_normal((B, T, kvH, hd)).astype(cdt)
    v = rng.standard_normal((B, T, kvH, hd)).astype(cdt)
    kw = dict(q_gain=t(qg), rope_cos=t(c), rope_sin=t(s))
    kraw = rng.standard_normal((B, kvH, hd)).astype(np.float32)
    vraw = rng.standard_normal((B, kvH, hd)).astype(np.float32)
    kc, vc = t(k), t(v)
    if fused:
        kw.update(k_new=t(kraw), v_new=t(vraw), k_gain=t(kg))
    got = sa.decode(t(q), kc, vc, t(lens), sa.AttnConfig(nH, kvH, hd, W), **kw)
    torch.cuda.synchronize()
    got = got.cpu().numpy()
    kn, vn = kc.float().cpu().numpy(), vc.float().cpu().numpy()
    for b in range(B):
        L = int(lens[b])
        if fused:  # the row the call wrote, against the oracle's kv_write
            kref, vref = O.kv_write(kraw[b:b + 1], vraw[b:b + 1], kg, c[b:b + 1], s[b:b + 1], cache_dtype=cdt)
            contract_close(kn[b, L - 1:L], kref.astype(np.float32), f"case {i} seq {b} k row")
            contract_close(vn[b, L - 1:L], vref.astype(np.float32), f"case {i} seq {b} v row")
        ref = O.decode_attention(q[b], kn[b, :L], vn[b, :L], L, kvH, q_gain=qg, cos=c[b], sin=s[b], window=W)
        contract_close(got[b], ref, f"case {i} seq {b} len {L}")


def prefill_cases(n=20, seed=77):
    rng = np.random.default_rng(seed)
    for i in range(n):
        nH, kvH = GROUPS[rng.integers(len(GROUPS))]
        hd = int(rng.choice([256, 256, 512]))
        S = int(rng.integers(1, 400))
        start = int(rng.choice([0, 0, rng.integers(1, 300)]))
        W = int(rng.choice([0, 0, 48, 257]))
        yield pytest.param(i, nH, kvH, hd, S, start, W, id=f"p{i}-{nH}/{kvH}-hd{hd}-S{S}-at{start}-W{W}")


@pytest.mark.parametrize("i,nH,kvH,hd,S,start,W", list(prefill_cases()))
def test_prefill_sweep(i, nH, kvH, hd, S, start, W):
    rng = np.random.default_rng(2000 + i)
    T = start + S
    q = rng.standard_normal((S, nH, hd)).astype(np.float32)
    qg = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    c, s = O.rope_tables(np.arange(start, T), hd, 1e6)
    k = rng.standard_normal((T + 3, kvH, hd)).astype(np.float16)  # rows past T are never attended
    v = rng.standard_normal((T + 3, kvH, hd)).astype(np.float16)
    cfg = sa.AttnConfig(nH, kvH, hd, W)
    q16 = sa.qprep(t(q), cfg, q_gain=t(qg), rope_cos=t(c), rope_sin=t(s))
    out = sa.prefill(t(q), t(k), t(v), start, cfg, q_gain=t(qg), rope_cos=t(c), rope_sin=t(s),
                     out_dtype=torch.float32, workspace=WS)
    torch.cuda.synchronize()
    ref = O.prefill_attention(q16.cpu().numpy().astype(np.float32), k, v, start, kvH, window=W)
    contract_close(out.cpu().numpy(), ref, f"case {i}")
