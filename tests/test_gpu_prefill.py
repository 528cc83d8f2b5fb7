"""GPU parity of batched causal prefill attention (g4a_prefill) against the CPU oracle and
the golden vectors, at |d| <= 2e-3 + 1e-2|ref|; attended sets exact per query row.

The oracle consumes the same f16-rounded q the kernel feeds its MFMAs (qprep_b's rounding
point, kernels_dsl.py:1872-1873) and the same f16 caches. Cases
(S = 1024, global and window 512), the reference's S = 300 tile-crossing case
(gemma4_150/prefill_research/test_attn_prefill.py:17-27), continuation prefill
(start_pos > 0), ragged S, one-hot mask sets, and an S = 8192 layer (config 5).
"""
import numpy as np
import pytest
import torch

import oracle.attention as O
import slang_amd as sa
from helpers import contract_close, gold, srq_close

pytestmark = pytest.mark.gpu
DEV = "cuda"


def t(x):
    return torch.from_numpy(np.ascontiguousarray(x)).to(DEV)


def run(q, k, v, start, cfg, out_dtype=torch.float16, **kw):
    out = sa.prefill(t(q), t(k), t(v), start, cfg, out_dtype=out_dtype,
                     **{n: (t(a) if isinstance(a, np.ndarray) else a) for n, a in kw.items()})
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


def test_golden_prefill_core_exact_q():
    """Pre-rounded golden q (no prologue): the kernel's core against the f64 restatement."""
    z = gold("prefill.npz")
    for w in (0, 16):
        got = run(z["q16"].astype(np.float32), z["k"], z["v"], int(z["start_pos"]),
                  sa.AttnConfig(4, 2, 256, w), out_dtype=torch.float32)
        contract_close(got, z[f"expected_q16_w{w}"], f"golden core w={w}")


@pytest.mark.parametrize("window", [0, 16])
def test_golden_prefill_end_to_end(window):
    z = gold("prefill.npz")
    kw = dict(q_gain=z["w"], rope_cos=z["cos"], rope_sin=z["sin"])
    got = run(z["q"], z["k"], z["v"], int(z["start_pos"]), sa.AttnConfig(4, 2, 256, window), **kw)
    contract_close(got, z[f"expected_q16_w{window}"], f"golden e2e w={window}")
    ref = O.prefill_attention(z["q"], z["k"], z["v"], int(z["start_pos"]), 2, q_gain=z["w"],
                              cos=z["cos"], sin=z["sin"], window=window)
    contract_close(got, ref, f"oracle e2e w={window}")


def config3_inputs(S=1024, theta=1e6, seed=3, H=1536, nH=8, kvH=2, hd=256):
    """h ~ N(0,1) [S][H] projected by f16 Wq/Wk/Wv ~ N(0, 0.02); k/v through the cache write."""
    rng = np.random.default_rng(seed)
    h = rng.standard_normal((S, H)).astype(np.float32)
    wq = (0.02 * rng.standard_normal((nH * hd, H))).astype(np.float16).astype(np.float32)
    wk = (0.02 * rng.standard_normal((kvH * hd, H))).astype(np.float16).astype(np.float32)
    wv = (0.02 * rng.standard_normal((kvH * hd, H))).astype(np.float16).astype(np.float32)
    q = (h @ wq.T).reshape(S, nH, hd)
    kr = (h @ wk.T).reshape(S, kvH, hd)
    vr = (h @ wv.T).reshape(S, kvH, hd)
    qg = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    kg = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    cos, sin = O.rope_tables(np.arange(S), hd, theta)
    k, v = O.kv_write(kr, vr, kg, cos, sin)
    return q, qg, k, v, cos, sin


@pytest.mark.parametrize("window,theta", [(0, 1e6), (512, 1e4)])
def test_config3(window, theta):
    q, qg, k, v, cos, sin = config3_inputs(theta=theta)
    got = run(q, k, v, 0, sa.AttnConfig(8, 2, 256, window), q_gain=qg, rope_cos=cos, rope_sin=sin)
    ref = O.prefill_attention(q, k, v, 0, 2, q_gain=qg, cos=cos, sin=sin, window=window)
    contract_close(got, ref, f"config3 W={window}")


@pytest.mark.parametrize("hd", [256, 512])
@pytest.mark.parametrize("window", [0, 64])
def test_s300_crosses_tiles_with_srq(hd, window):
    """The reference's attn_prefill check: S = 300 (> one 256-key tile), inputs N(0,1)*0.5,
    seed 5, nH 8 kvH 1, output srq'd with o_in."""
    rng = np.random.default_rng(5)
    S, nH = 300, 8
    q = (0.5 * rng.standard_normal((S, nH, hd))).astype(np.float32)
    kr = (0.5 * rng.standard_normal((S, 1, hd))).astype(np.float32)
    vr = (0.5 * rng.standard_normal((S, 1, hd))).astype(np.float32)
    g = rng.standard_normal(hd).astype(np.float32)
    cos, sin = O.rope_tables(np.arange(S), hd, 1e4)
    k, v = O.kv_write(kr, vr, g, cos, sin)
    oq = 0.014886821620166302
    kw = dict(q_gain=g, rope_cos=cos, rope_sin=sin)
    ref = O.prefill_attention(q, k, v, 0, 1, q_gain=g, cos=cos, sin=sin, window=window)
    got = run(q, k, v, 0, sa.AttnConfig(nH, 1, hd, window), out_dtype=torch.float32, **kw)
    contract_close(got, ref, f"S300 hd={hd} W={window}")
    gq = run(q, k, v, 0, sa.AttnConfig(nH, 1, hd, window, out_q=oq), out_dtype=torch.float32, **kw)
    srq_close(gq, ref, oq, f"S300 srq hd={hd} W={window}")


@pytest.mark.parametrize("S,start,window", [(100, 700, 512), (37, 0, 0), (1, 0, 0), (1, 900, 0),
                                            (129, 383, 128), (250, 6, 5)])
@pytest.mark.parametrize("nH,kvH", [(8, 2), (4, 4), (8, 1), (4, 2)])
def test_continuation_and_ragged(S, start, window, nH, kvH):
    hd = 256
    T = start + S
    rng = np.random.default_rng(S + start + nH)
    q = rng.standard_normal((S, nH, hd)).astype(np.float32)
    qg = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    k = rng.standard_normal((T + 5, kvH, hd)).astype(np.float16)  # extra rows are never attended
    v = rng.standard_normal((T + 5, kvH, hd)).astype(np.float16)
    k, v = O.kv_write(k.astype(np.float32), v.astype(np.float32),
                      (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32))
    cos, sin = O.rope_tables(np.arange(start, T), hd, 1e4)
    got = run(q, k, v, start, sa.AttnConfig(nH, kvH, hd, window), q_gain=qg, rope_cos=cos, rope_sin=sin)
    ref = O.prefill_attention(q, k, v, start, kvH, q_gain=qg, cos=cos, sin=sin, window=window)
    contract_close(got, ref, f"S={S} start={start} W={window} nH={nH} kvH={kvH}")


@pytest.mark.parametrize("S,start", [(300, 0), (200, 100), (64, 447), (1, 0)])
@pytest.mark.parametrize("window", [0, 1, 63, 64, 65, 300])
def test_mask_sets_exact(S, start, window):
    """q = 0 weighs every attended key 1/n; one-hot V (v_j = e_j, hd 512) makes row s the
    indicator of its attended set, which must be exactly [max(0, p+1-W), p]."""
    hd, T = 512, start + S
    k = np.random.default_rng(S).standard_normal((T, 1, hd)).astype(np.float16)
    v = np.zeros((T, 1, hd), np.float16)
    v[np.arange(T), 0, np.arange(T)] = 1
    got = run(np.zeros((S, 2, hd), np.float32), k, v, start, sa.AttnConfig(2, 1, hd, window),
              out_dtype=torch.float32)
    for s in range(S):
        p = start + s
        lo = max(0, p + 1 - window) if window else 0
        assert set(np.nonzero(got[s, 0] > 1e-6)[0]) == set(range(lo, p + 1)), f"row {s}"
        assert set(np.nonzero(got[s, 1] > 1e-6)[0]) == set(range(lo, p + 1)), f"row {s}"


def test_f32_cache_and_mirror():
    """f32 caches (the reference's own cache type) through the attn_prefill slot drop-in."""
    z = gold("prefill.npz")
    S, start, hd, nH, kvH = 24, int(z["start_pos"]), 256, 4, 2
    cosT, sinT = O.rope_tables(np.arange(64), hd, 1e4)
    cosT[start:start + S], sinT[start:start + S] = z["cos"], z["sin"]
    out = torch.zeros(S * nH * hd, device=DEV, dtype=torch.float32)
    sa.attn_prefill(t(z["q"].reshape(-1)), t(z["w"]), t(cosT), t(sinT),
                    t(z["k"].astype(np.float32).reshape(-1)), t(z["v"].astype(np.float32).reshape(-1)),
                    out, (start, nH, kvH, 16, S), head_dim=hd)
    torch.cuda.synchronize()
    contract_close(out.cpu().numpy().reshape(S, nH, hd), z["expected_q16_w16"], "attn_prefill mirror")


@pytest.mark.parametrize("window", [0, 512])
def test_config5_layer_s8192(window):
    """One layer of config 5's prefill: S = 8192."""
    S, nH, kvH, hd = 8192, 8, 2, 256
    g = torch.Generator(device=DEV).manual_seed(8)
    q = torch.randn(S, nH, hd, device=DEV, generator=g)
    k = torch.randn(S, kvH, hd, device=DEV, generator=g).half()
    v = torch.randn(S, kvH, hd, device=DEV, generator=g).half()
    qg = torch.ones(hd, device=DEV)
    out = sa.prefill(q, k, v, 0, sa.AttnConfig(nH, kvH, hd, window), q_gain=qg)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    # check a spread of query rows (the oracle on all 8192 rows is slow on one host core)
    rows = np.r_[0:64, 1000:1064, 4090:4110, 8128:8192]
    qn, kn, vn = q.cpu().numpy(), k.cpu().numpy(), v.cpu().numpy()
    for s in rows:
        ref = O.prefill_attention(qn[s:s + 1], kn, vn, s, kvH, q_gain=np.ones(hd, np.float32),
                                  window=window)
        contract_close(got[s:s + 1], ref, f"S8192 row {s} W={window}")
