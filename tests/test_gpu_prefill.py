"""GPU parity of batched causal prefill attention (g4a_prefill) against the CPU oracle and
the golden vectors, at |d| <= 2e-3 + 1e-2|ref|; attended sets exact per query row.

Two q precisions. Default: q is rounded to f16 after RMSNorm+RoPE (qprep_b's rounding
point, kernels_dsl.py:1872-1873); the oracle is fed exactly that f16 q, taken from
g4a_qprep (bit-identical to the prefill prologue, checked below), because with scale 1.0
a one-ulp difference in a rounded q element moves scores by up to ~1e-2 and can push an
output past 2e-3. G4A_Q_HILO: q kept at f32 accuracy and compared with the f32-q oracle
(reference.py:150-151 semantics). Both modes see the same f16 caches. Cases
(S = 1024, global and window 512), the reference's S = 300 tile-crossing case
(gemma4_150/prefill_research/test_attn_prefill.py:17-27), continuation prefill
(start_pos > 0), ragged S and one-hot mask sets. Config 5 (S = 8192 and the decode steps
after it) is tests/test_gpu_config5.py.

End to end against the oracle's OWN f16 rounding of q (test_config3) the check is tie-aware,
as the reference's own prefill check is (gemma4_150/prefill_research/test_attn_prefill.py:
66-79): an element outside the contract is accepted only in a (token, head) row whose f16 q
differs from the oracle's rounding (by one ulp, from a value that straddles a rounding
boundary), and only if that row meets the contract when the oracle is given the kernel's
f16 q row.
"""
import ctypes

import numpy as np
import pytest
import torch

import oracle.attention as O
import slang_amd as sa
from helpers import contract_close, f16_ulp_close, gold, srq_close, tie_aware_e2e

pytestmark = pytest.mark.gpu
DEV = "cuda"
WS = sa.Workspace(DEV)  # grows to the largest call; the cases run one at a time on one stream


def t(x):
    return torch.from_numpy(np.ascontiguousarray(x)).to(DEV)


def run(q, k, v, start, cfg, out_dtype=torch.float16, q_hilo=False, **kw):
    out = sa.prefill(t(q), t(k), t(v), start, cfg, out_dtype=out_dtype, q_hilo=q_hilo, workspace=WS,
                     **{n: (t(a) if isinstance(a, np.ndarray) else a) for n, a in kw.items()})
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


def kernel_q16(q, cfg, q_gain=None, cos=None, sin=None):
    """The f16 q the prefill kernel feeds its MFMAs, via g4a_qprep."""
    out = sa.qprep(t(q), cfg, q_gain=None if q_gain is None else t(q_gain),
                   rope_cos=None if cos is None else t(cos), rope_sin=None if sin is None else t(sin))
    torch.cuda.synchronize()
    return out.cpu().numpy()


def check_both_modes(q, k, v, start, cfg, qg, cos, sin, what, out_q=0.0):
    """Default mode vs the oracle on the kernel's f16 q; HILO mode vs the f32-q oracle."""
    kvH, W = cfg.n_kv_heads, cfg.window
    kw = dict(q_gain=qg, rope_cos=cos, rope_sin=sin)
    q16 = kernel_q16(q, cfg, qg, cos, sin).astype(np.float32)
    ref16 = O.prefill_attention(q16, k, v, start, kvH, window=W, scale=cfg.scale)
    got = run(q, k, v, start, cfg, out_dtype=torch.float32, **kw)
    contract_close(got, ref16, f"{what} (f16 q)")
    ref32 = O.prefill_attention(q, k, v, start, kvH, q_gain=qg, cos=cos, sin=sin, window=W,
                                scale=cfg.scale, q_round_f16=False)
    got32 = run(q, k, v, start, cfg, out_dtype=torch.float32, q_hilo=True, **kw)
    contract_close(got32, ref32, f"{what} (hilo q)")
    return ref16, ref32


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


@pytest.mark.parametrize("window", [0, 16])
def test_golden_prefill_hilo(window):
    """G4A_Q_HILO against the float64 restatement with f32 q (reference.py's q precision)."""
    z = gold("prefill.npz")
    got = run(z["q"], z["k"], z["v"], int(z["start_pos"]), sa.AttnConfig(4, 2, 256, window),
              out_dtype=torch.float32, q_hilo=True, q_gain=z["w"], rope_cos=z["cos"], rope_sin=z["sin"])
    contract_close(got, z[f"expected_w{window}"], f"golden hilo w={window}")
    assert np.abs(got - z[f"expected_w{window}"]).max() < 5e-4


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
    cfg = sa.AttnConfig(8, 2, 256, window)
    ref16, _ = check_both_modes(q, k, v, 0, cfg, qg, cos, sin, f"config3 W={window}")
    # the product path (f16 q, f16 attnh output) end to end against the oracle's own q rounding
    got = run(q, k, v, 0, cfg, q_gain=qg, rope_cos=cos, rope_sin=sin)
    ref = O.prefill_attention(q, k, v, 0, 2, q_gain=qg, cos=cos, sin=sin, window=window)
    q_f32 = O.apply_rope(O.rms_norm(q, qg), cos[:, None, :], sin[:, None, :])
    n_tie = tie_aware_e2e(got, ref, ref16, kernel_q16(q, cfg, qg, cos, sin), q_f32, f"config3 W={window}")
    print(f"config3 W={window}: {n_tie} of {q.shape[0] * q.shape[1]} (token, head) rows needed the "
          f"one-ulp q tie allowance")


@pytest.mark.parametrize("window", [0, 512])
def test_qprep_is_the_prefill_prologue(window):
    """The f16 q every prefill path feeds its MFMAs is qprep's, bit for bit:
    * split path (q from qprep_kernel): prefill(raw q) == prefill(qprep(q)) with no prologue;
    * unsplit path (the q prologue fused into the attention kernel, which every call without
      a workspace and every long prompt takes): the same equality, so the fused prologue
      rounds exactly as qprep does (non-unit gain and RoPE);
    and qprep's f16 q matches the oracle's rounding except for rare one-ulp boundary cases."""
    q, qg, k, v, cos, sin = config3_inputs(S=256, seed=11, theta=1e4 if window else 1e6)
    cfg = sa.AttnConfig(8, 2, 256, window)
    c = cfg.c(0)
    assert sa._lib.load().g4a_prefill_ws_bytes(ctypes.byref(c), 256, 0) > 0, "S 256 should take the key split"
    q16 = kernel_q16(q, cfg, qg, cos, sin)
    for split in (True, False):
        a = run(q, k, v, 0, cfg, q_gain=qg, rope_cos=cos, rope_sin=sin, split=split)
        b = run(q16.astype(np.float32), k, v, 0, cfg, split=split)
        np.testing.assert_array_equal(a, b, err_msg=f"split={split}")
    ref = O.apply_rope(O.rms_norm(q, qg), cos[:, None, :], sin[:, None, :])
    assert (q16 != ref.astype(np.float16)).mean() < 0.01
    f16_ulp_close(q16, ref, "qprep vs oracle")


def test_qprep_b_mirror():
    rng = np.random.default_rng(2)
    S, nH, hd, start = 10, 8, 512, 5
    q = rng.standard_normal((S, nH, hd)).astype(np.float32)
    w = rng.standard_normal(hd).astype(np.float32)
    cosT, sinT = O.rope_tables(np.arange(32), hd, 1e6, cutoff=64)
    qf16 = torch.zeros(S * nH * hd, dtype=torch.float16, device=DEV)
    sa.qprep_b(t(q.reshape(-1)), t(w), t(cosT), t(sinT), qf16, (start, nH), S=S, head_dim=hd)
    torch.cuda.synchronize()
    ref = O.apply_rope(O.rms_norm(q, w), cosT[start:start + S, None, :], sinT[start:start + S, None, :])
    f16_ulp_close(qf16.cpu().numpy().reshape(S, nH, hd), ref, "qprep_b")


@pytest.mark.parametrize("hd", [256, 512])
@pytest.mark.parametrize("window", [0, 64])
def test_s300_crosses_tiles_with_srq(hd, window):
    """The reference's attn_prefill check: S = 300 (> one 256-key tile), inputs N(0,1)*0.5,
    seed 5, nH 8 kvH 1, gain ~N(0,1), output srq'd with o_in."""
    rng = np.random.default_rng(5)
    S, nH = 300, 8
    q = (0.5 * rng.standard_normal((S, nH, hd))).astype(np.float32)
    kr = (0.5 * rng.standard_normal((S, 1, hd))).astype(np.float32)
    vr = (0.5 * rng.standard_normal((S, 1, hd))).astype(np.float32)
    g = rng.standard_normal(hd).astype(np.float32)
    cos, sin = O.rope_tables(np.arange(S), hd, 1e4)
    k, v = O.kv_write(kr, vr, g, cos, sin)
    oq = 0.014886821620166302
    cfg = sa.AttnConfig(nH, 1, hd, window)
    ref16, ref32 = check_both_modes(q, k, v, 0, cfg, g, cos, sin, f"S300 hd={hd} W={window}")
    kw = dict(q_gain=g, rope_cos=cos, rope_sin=sin)
    cq = sa.AttnConfig(nH, 1, hd, window, out_q=oq)
    srq_close(run(q, k, v, 0, cq, out_dtype=torch.float32, **kw), ref16, oq, f"S300 srq hd={hd} W={window}")
    srq_close(run(q, k, v, 0, cq, out_dtype=torch.float32, q_hilo=True, **kw), ref32, oq,
              f"S300 srq hilo hd={hd} W={window}")


@pytest.mark.parametrize("S,start,window", [(1024, 0, 0), (1024, 0, 512), (2048, 0, 512), (600, 1500, 0),
                                            (333, 64, 100)])
def test_hd512_e2b_shape(S, start, window):
    """The Gemma 4 E2B global-layer shape (nH 8 / kvH 1, hd 512): f16 q on the 128-column
    kernel (every wave all 512 dims; key split at S 1024 global and at S 600 after 1500
    cached rows, unsplit one-workgroup-a-block grids at S 2048 W 512), f32 q on the
    dim-split wave-pair kernel, both against the oracle."""
    T = start + S
    q, qg, k, v, cos, sin = config3_inputs(S=T, theta=1e6 if window == 0 else 1e4, seed=S + window,
                                           nH=8, kvH=1, hd=512)
    q, cos, sin = q[start:], cos[start:], sin[start:]
    check_both_modes(q, k, v, start, sa.AttnConfig(8, 1, 512, window), qg, cos, sin,
                     f"hd512 S={S} start={start} W={window}")


@pytest.mark.parametrize("S,start,window", [(1024, 0, 0), (1024, 0, 512), (300, 600, 0)])
def test_hd512_unsplit_launch(S, start, window):
    """The hd-512 launches long prompts take, forced at test sizes (split=False: a workspace
    with only the f16 q rows): the causal one runs the 128-column kernel without q or output
    staging, the windowed one with output staging only. Both q modes against the oracle, and
    the f16-q result against the split call's within the contract."""
    T = start + S
    q, qg, k, v, cos, sin = config3_inputs(S=T, theta=1e6 if window == 0 else 1e4, seed=3 * S + window,
                                           nH=8, kvH=1, hd=512)
    q, cos, sin = q[start:], cos[start:], sin[start:]
    cfg = sa.AttnConfig(8, 1, 512, window)
    kw = dict(q_gain=qg, rope_cos=cos, rope_sin=sin)
    q16 = kernel_q16(q, cfg, qg, cos, sin).astype(np.float32)
    ref16 = O.prefill_attention(q16, k, v, start, 1, window=window, scale=cfg.scale)
    whole = run(q, k, v, start, cfg, out_dtype=torch.float32, split=False, **kw)
    contract_close(whole, ref16, f"hd512 unsplit S={S} start={start} W={window} (f16 q)")
    split = run(q, k, v, start, cfg, out_dtype=torch.float32, **kw)
    contract_close(split, whole, f"hd512 split vs unsplit S={S} W={window}")
    ref32 = O.prefill_attention(q, k, v, start, 1, q_gain=qg, cos=cos, sin=sin, window=window,
                                scale=cfg.scale, q_round_f16=False)
    whole32 = run(q, k, v, start, cfg, out_dtype=torch.float32, q_hilo=True, split=False, **kw)
    contract_close(whole32, ref32, f"hd512 unsplit S={S} W={window} (f32 q)")


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
    check_both_modes(q, k, v, start, sa.AttnConfig(nH, kvH, hd, window), qg, cos, sin,
                     f"S={S} start={start} W={window} nH={nH} kvH={kvH}")


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


def f32_caches(T, kvH, hd, seed):
    """f32 caches as the reference runners hold them (kvnorm's f32 rows): N(0,1) rows through
    the oracle's cache write, stored f32, so almost no value is an f16 grid point."""
    rng = np.random.default_rng(seed)
    kr = rng.standard_normal((T, kvH, hd)).astype(np.float32)
    vr = rng.standard_normal((T, kvH, hd)).astype(np.float32)
    kg = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    cos, sin = O.rope_tables(np.arange(T), hd, 1e4)
    k, v = O.kv_write(kr, vr, kg, cos, sin, cache_dtype=np.float32)
    assert (k != k.astype(np.float16).astype(np.float32)).mean() > 0.99
    return k, v


def test_f32_cache_and_mirror():
    """The attn_prefill and attn_gemm slot drop-ins on f32 caches (the reference runners' own
    cache type), each against the form it replaces: attn_prefill (kernels_dsl.py:1950-2098)
    reads f32 q and the f32 caches as they are; attn_gemm (prefill_gpu.py:259-313) rounds q
    (qprep_b) and both caches (srqh_b, :286-288) to f16 before its GEMMs."""
    z = gold("prefill.npz")
    S, start, hd, nH, kvH, W = 24, int(z["start_pos"]), 256, 4, 2, 16
    cosT, sinT = O.rope_tables(np.arange(64), hd, 1e4)
    cosT[start:start + S], sinT[start:start + S] = z["cos"], z["sin"]
    k32, v32 = f32_caches(start + S, kvH, hd, 17)
    out = torch.zeros(S * nH * hd, device=DEV, dtype=torch.float32)
    sa.attn_prefill(t(z["q"].reshape(-1)), t(z["w"]), t(cosT), t(sinT), t(k32.reshape(-1)), t(v32.reshape(-1)),
                    out, (start, nH, kvH, W, S), head_dim=hd, workspace=WS)
    torch.cuda.synchronize()
    ref = O.prefill_attention(z["q"], k32, v32, start, kvH, q_gain=z["w"], cos=z["cos"], sin=z["sin"], window=W,
                              q_round_f16=False)
    contract_close(out.cpu().numpy().reshape(S, nH, hd), ref, "attn_prefill mirror, f32 caches")
    out16 = torch.zeros(S * nH * hd, device=DEV, dtype=torch.float16)
    sa.attn_gemm(t(z["q"].reshape(-1)), t(z["w"]), t(cosT), t(sinT), t(k32.reshape(-1)), t(v32.reshape(-1)),
                 out16, S=S, start_pos=start, n_q_heads=nH, n_kv_heads=kvH, head_dim=hd, window=W, o_in=0.0,
                 workspace=WS)
    torch.cuda.synchronize()
    cfg = sa.AttnConfig(nH, kvH, hd, W)
    q16 = kernel_q16(z["q"], cfg, z["w"], z["cos"], z["sin"]).astype(np.float32)
    ref16 = O.prefill_attention(q16, k32, v32, start, kvH, window=W, kv_round_f16=True)
    contract_close(out16.float().cpu().numpy().reshape(S, nH, hd), ref16, "attn_gemm mirror, f32 caches")


@pytest.mark.parametrize("S,start,window,hd", [(1024, 0, 0, 256), (1024, 0, 512, 256), (700, 900, 512, 256),
                                               (300, 50, 0, 256), (300, 0, 0, 512), (257, 40, 64, 512)])
def test_f32_caches(S, start, window, hd):
    """f32 caches in both forms, against the oracle on the same unrounded f32 caches.
    * f32 q (attn_prefill's form, G4A_Q_HILO): K enters the score MFMAs as the f16 pair
      (k_hi, k_lo), so the scores are f32-accurate; the oracle reads q and the caches
      unrounded. (Rounding K to f16 instead puts thousands of these outputs beyond the
      contract: with scale 1.0 and |q.k| in the tens a 2^-11 relative error in k moves a
      score by ~0.1.)
    * f16 q (the GEMM form): the caches are rounded to f16 as its srqh_b does, so the output
      equals the call on f16-rounded caches bit for bit and meets the contract against the
      oracle with that rounding (kv_round_f16).
    * Without the workspace their f16 copy lives in, the C ABI refuses the call."""
    nH, kvH = (8, 2) if hd == 256 else (8, 1)
    T = start + S
    rng = np.random.default_rng(S + start + window + hd)
    q = rng.standard_normal((S, nH, hd)).astype(np.float32)
    qg = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    k32, v32 = f32_caches(T + 2, kvH, hd, S + window)  # rows past T are never attended
    cos, sin = O.rope_tables(np.arange(start, T), hd, 1e4 if window else 1e6)
    cfg = sa.AttnConfig(nH, kvH, hd, window)
    kw = dict(q_gain=qg, rope_cos=cos, rope_sin=sin)
    ref32 = O.prefill_attention(q, k32, v32, start, kvH, q_gain=qg, cos=cos, sin=sin, window=window,
                                q_round_f16=False)
    got32 = run(q, k32, v32, start, cfg, out_dtype=torch.float32, q_hilo=True, **kw)
    err = contract_close(got32, ref32, f"f32 q, f32 caches S={S} start={start} W={window} hd={hd}")
    print(f"f32 q on f32 caches: max |d| {err:.2e}")
    q16 = kernel_q16(q, cfg, qg, cos, sin).astype(np.float32)
    ref16 = O.prefill_attention(q16, k32, v32, start, kvH, window=window, kv_round_f16=True)
    got16 = run(q, k32, v32, start, cfg, out_dtype=torch.float32, **kw)
    contract_close(got16, ref16, f"f16 q, f32 caches S={S} start={start} W={window} hd={hd}")
    same = run(q, k32.astype(np.float16), v32.astype(np.float16), start, cfg, out_dtype=torch.float32, **kw)
    assert np.array_equal(got16, same), f"f16 q: f32 vs f16-rounded caches, max |d| {np.abs(got16 - same).max()}"
    lib = sa._lib.load()
    c = cfg.c(sa._lib.KV_F32 | sa._lib.OUT_F32 | sa._lib.Q_HILO)
    qd, kd, vd = t(q), t(k32), t(v32)
    o = torch.empty(S, nH, hd, device=DEV)
    rc = lib.g4a_prefill(ctypes.byref(c), S, start, ctypes.c_void_p(qd.data_ptr()), None, None, None,
                         ctypes.c_void_p(kd.data_ptr()), ctypes.c_void_p(vd.data_ptr()),
                         ctypes.c_void_p(o.data_ptr()), None, 0, None)
    assert rc == -3, f"f32 caches without a workspace: rc {rc}, expected G4A_EWORKSPACE"


def test_prefill_mirrors_allocate_nothing():
    """The runner-owned workspace contract (runner.py:102-109, prefill_gpu.py:229-256: every
    buffer persistent, kernels never allocate) for the attn_prefill / attn_gemm drop-ins: with
    the workspace reserved up front (the split partials and the f32 caches' f16 copy of an
    S 300 call), 10 calls in a row leave torch.cuda.memory_allocated() where it was, and a
    HIP graph captured over both calls replays -- several times, with the program's own
    eager work and synchronisations between the replays -- to the eager results bit for bit."""
    S, start, hd, nH, kvH, W = 300, 0, 256, 8, 2, 0
    rng = np.random.default_rng(31)
    q = t(rng.standard_normal((S * nH * hd,)).astype(np.float32))
    qg = t((1 + 0.1 * rng.standard_normal(hd)).astype(np.float32))
    cosT, sinT = (t(x) for x in O.rope_tables(np.arange(S), hd, 1e6))
    k32, v32 = (t(x.reshape(-1)) for x in f32_caches(S, kvH, hd, 5))
    cfg = sa.AttnConfig(nH, kvH, hd, W)
    need = max(sa.prefill_ws_bytes(S, start, cfg, kv_f32=True, q_hilo=True),
               sa.prefill_ws_bytes(S, start, cfg, kv_f32=True))
    assert need > 0
    ws = sa.Workspace(DEV).reserve(need)
    out = torch.empty(S * nH * hd, device=DEV)
    out16 = torch.empty(S * nH * hd, device=DEV, dtype=torch.float16)

    def calls():
        sa.attn_prefill(q, qg, cosT, sinT, k32, v32, out, (start, nH, kvH, W, S), head_dim=hd, workspace=ws)
        sa.attn_gemm(q, qg, cosT, sinT, k32, v32, out16, S=S, start_pos=start, n_q_heads=nH, n_kv_heads=kvH,
                     head_dim=hd, window=W, o_in=0.0, workspace=ws)

    calls()
    torch.cuda.synchronize()
    ref, ref16 = out.clone(), out16.clone()
    before = torch.cuda.memory_allocated()
    for _ in range(10):
        calls()
    torch.cuda.synchronize()
    assert torch.cuda.memory_allocated() == before, "an eager call allocated device memory"
    assert torch.equal(out, ref) and torch.equal(out16, ref16)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        calls()
    torch.cuda.synchronize()
    after_capture = torch.cuda.memory_allocated()
    for r in range(4):
        out.zero_()
        out16.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"replay {r}: attn_prefill output differs from the eager call"
        assert torch.equal(out16, ref16), f"replay {r}: attn_gemm output differs from the eager call"
    assert torch.cuda.memory_allocated() == after_capture, "a replay allocated device memory"
    with pytest.raises(RuntimeError, match="reserved"):
        ws.get(need + 1)


@pytest.mark.parametrize("S", [512, 1024, 2048])
@pytest.mark.parametrize("window", [0, 512])
def test_key_split_matches_unsplit(S, window):
    """Short prompts split long causal rows over workgroups (partials merged by a second
    kernel); the piece size grows with S (2, 3 and 5 key tiles at S 512, 1024, 2048 global).
    The split result equals the unsplit one (no workspace) up to summation order, and both
    meet the contract against the oracle."""
    q, qg, k, v, cos, sin = config3_inputs(S=S, seed=7, theta=1e4 if window else 1e6)
    cfg = sa.AttnConfig(8, 2, 256, window)
    kw = dict(q_gain=qg, rope_cos=cos, rope_sin=sin)
    q16 = kernel_q16(q, cfg, qg, cos, sin).astype(np.float32)
    ref = O.prefill_attention(q16, k, v, 0, 2, window=window)
    split = run(q, k, v, 0, cfg, out_dtype=torch.float32, **kw)
    whole = run(q, k, v, 0, cfg, out_dtype=torch.float32, split=False, **kw)
    contract_close(split, ref, f"split S={S} W={window}")
    contract_close(whole, ref, f"unsplit S={S} W={window}")
    # P is rounded to f16 against each piece's own running max
    contract_close(split, whole, f"split vs unsplit S={S} W={window}")
