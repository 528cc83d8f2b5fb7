"""BASELINE config 5 at its full shape, one layer of each kind: a global layer (RoPE theta 1e6)
and a sliding-window-512 layer (theta 1e4), nH 8 / kvH 2, hd 256, f16 caches.

Per layer, as the stack runs it (bench.py stack_case; the reference's per-layer prefill is
prefill_gpu.py:335-354, its decode step runner.py:424-441):
  * prefill of S = 8192 tokens: the k/v rows (f16, kvnorm_b's input type) go through
    g4a_kv_write with a k gain ~N(1, 0.1) and RoPE, then g4a_prefill with a q gain
    ~N(1, 0.1) and RoPE;
  * 256 decode steps at T = 8193 .. 8448, each one g4a_decode_kv call: the step's raw k/v
    row (f32) is prepared and written at row T-1 inside the decode call.
q/k/v come from hidden states N(0,1) [tokens][1536] projected by f16 weights N(0, 0.02)
(the projection runs on the GPU in f32 and is test harness; both sides see its output).

Checked against the CPU oracle:
  * every cache row the prefill and the 256 steps wrote, within one f16 ulp of
    oracle.kv_write (the same inputs, rounded to the f16 cache; 1e-6 absolute where a RoPE
    pair nearly cancels);
  * >= 1024 prefill rows spread over the prompt: six 64-row runs (start, middle, end),
    every 32-position query-block edge, every 64-key tile edge (p = 64k - 1, 64k, 64k + 1) and every window edge (the window's
    first key p + 1 - 512 at 64k - 1, 64k, 64k + 1), at |d| <= 2e-3 + 1e-2|ref| against the
    oracle fed the kernel's f16 q (g4a_qprep, bit-identical to the prefill prologue), and
    tie-aware against the oracle's own rounding of q;
  * 26 of the 256 decode steps (the first and last, around T = 8192 + 64k and a spread), at the
    contract tolerance, against oracle.decode_attention on the caches as written.
"""
import numpy as np
import pytest
import torch

import oracle.attention as O
import slang_amd as sa
from helpers import contract_close, f16_ulp_close, tie_aware_e2e

pytestmark = pytest.mark.gpu
DEV = "cuda"
S, STEPS, NH, KVH, HD, H = 8192, 256, 8, 2, 256, 1536


def project(seed, n_tok):
    """q f32 [n][nH][hd], k/v f32 [n][kvH][hd] from h ~ N(0,1) and f16 W ~ N(0, 0.02)."""
    g = torch.Generator(device=DEV).manual_seed(seed)
    h = torch.randn(n_tok, H, device=DEV, generator=g)
    w = [(0.02 * torch.randn(n, H, device=DEV, generator=g)).half().float()
         for n in (NH * HD, KVH * HD, KVH * HD)]
    q = (h @ w[0].T).view(n_tok, NH, HD).contiguous()
    k = (h @ w[1].T).view(n_tok, KVH, HD).contiguous()
    v = (h @ w[2].T).view(n_tok, KVH, HD).contiguous()
    gains = [(1 + 0.1 * torch.randn(HD, device=DEV, generator=g)) for _ in range(2)]
    return q, k, v, gains[0], gains[1]


def check_rows(window):
    """Prefill rows checked: 64-row runs, every 32-position query-block edge, and every tile
    edge and window edge."""
    rows = set()
    for r0 in (0, 1000, 2048, 4096 - 32, 6000, S - 64):
        rows.update(range(r0, r0 + 64))
    for k in range(0, S + 64, 32):
        rows.update((k - 1, k))                # query-block edges (32 positions a block)
    for k in range(0, S + 64, 64):
        for d in (-1, 0, 1):
            rows.add(k + d)                    # the query's own key at a tile edge
            rows.add(k + d + 512 - 1)          # a window of 512 starting at a tile edge
    return np.array(sorted(r for r in rows if 0 <= r < S))


def runs(rows):
    """Contiguous runs [a, b) of a sorted row list."""
    out, a = [], rows[0]
    for i in range(1, len(rows) + 1):
        if i == len(rows) or rows[i] != rows[i - 1] + 1:
            out.append((a, rows[i - 1] + 1))
            if i < len(rows):
                a = rows[i]
    return out


@pytest.mark.parametrize("window,theta", [(0, 1e6), (512, 1e4)])
def test_config5_layer(window, theta):
    T = S + STEPS
    q, k, v, qg, kg = project(500 + window, T)
    cfg = sa.AttnConfig(NH, KVH, HD, window)
    kvcfg = sa.AttnConfig(KVH, KVH, HD)
    cos, sin = sa.rope_tables(np.arange(T), HD, theta)
    kc = torch.zeros(T, KVH, HD, device=DEV, dtype=torch.float16)
    vc = torch.zeros_like(kc)
    k16, v16 = k[:S].half(), v[:S].half()

    # ---- prefill: the cache write of the prompt, then attention
    sa.kv_write(k16, v16, kc, vc, 0, kvcfg, k_gain=kg, rope_cos=cos[:S], rope_sin=sin[:S])
    outp = sa.prefill(q[:S], kc, vc, 0, cfg, q_gain=qg, rope_cos=cos[:S], rope_sin=sin[:S],
                      workspace=sa.Workspace(DEV))
    q16 = sa.qprep(q[:S], cfg, q_gain=qg, rope_cos=cos[:S], rope_sin=sin[:S])
    # ---- 256 decode steps with the KV write fused in
    outd = torch.empty(STEPS, NH, HD, device=DEV)
    kl = torch.arange(S + 1, T + 1, dtype=torch.int32, device=DEV)
    ws = sa.DecodeWorkspace(DEV)
    for t in range(STEPS):
        p = S + t
        sa.decode(q[p], kc, vc, kl[t:t + 1], cfg, q_gain=qg, rope_cos=cos[p:p + 1], rope_sin=sin[p:p + 1],
                  out=outd[t:t + 1], workspace=ws, max_key_len=p + 1, k_new=k[p], v_new=v[p], k_gain=kg)
    torch.cuda.synchronize()

    qn, kn, vn = q.cpu().numpy(), k.cpu().numpy(), v.cpu().numpy()
    qgn, kgn = qg.cpu().numpy(), kg.cpu().numpy()
    cn, sn = cos.cpu().numpy(), sin.cpu().numpy()
    kcn, vcn = kc.cpu().numpy(), vc.cpu().numpy()

    # ---- every cache row the call chain wrote
    kref, vref = O.kv_write(k16.float().cpu().numpy(), v16.float().cpu().numpy(), kgn, cn[:S], sn[:S])
    # one f16 ulp, plus 1e-6 absolute where a RoPE pair nearly cancels (see f16_ulp_close)
    f16_ulp_close(kcn[:S], kref.astype(np.float32), "prefill k rows", slack=1e-6)
    f16_ulp_close(vcn[:S], vref.astype(np.float32), "prefill v rows", slack=1e-6)
    kref, vref = O.kv_write(kn[S:], vn[S:], kgn, cn[S:], sn[S:])
    f16_ulp_close(kcn[S:], kref.astype(np.float32), "decode-step k rows", slack=1e-6)
    f16_ulp_close(vcn[S:], vref.astype(np.float32), "decode-step v rows", slack=1e-6)

    # ---- prefill rows
    kf, vf = kcn.astype(np.float32), vcn.astype(np.float32)
    rows = check_rows(window)
    assert len(rows) >= 1024
    got = outp.float().cpu().numpy()
    q16n = q16.cpu().numpy()
    ref_k = np.empty((len(rows), NH, HD), np.float32)
    ref_o = np.empty_like(ref_k)
    i = 0
    for a, b in runs(rows):
        ref_k[i:i + b - a] = O.prefill_attention(q16n[a:b].astype(np.float32), kf, vf, a, KVH, window=window)
        ref_o[i:i + b - a] = O.prefill_attention(qn[a:b], kf, vf, a, KVH, q_gain=qgn, cos=cn[a:b], sin=sn[a:b],
                                                 window=window)
        i += b - a
    contract_close(got[rows], ref_k, f"S 8192 prefill W={window}")
    q_f32 = O.apply_rope(O.rms_norm(qn[rows], qgn), cn[rows][:, None, :], sn[rows][:, None, :])
    n_tie = tie_aware_e2e(got[rows], ref_o, ref_k, q16n[rows], q_f32, f"S 8192 prefill W={window} e2e")
    print(f"config5 W={window}: {len(rows)} prefill rows checked, {n_tie} (token, head) rows on the q tie allowance")

    # ---- decode steps
    steps = sorted({0, 1, 2, 3, STEPS - 2, STEPS - 1} | {s + d for s in range(64, STEPS, 64) for d in (-2, -1, 0, 1)}
                   | {17, 100, 150, 200, 222, 229, 240, 250})
    assert len(steps) >= 16
    gotd = outd.cpu().numpy()
    for t in steps:
        p = S + t
        ref = O.decode_attention(qn[p], kf, vf, p + 1, KVH, q_gain=qgn, cos=cn[p], sin=sn[p], window=window)
        contract_close(gotd[t], ref, f"decode step {t} (T {p + 1}) W={window}")
