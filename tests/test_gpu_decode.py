"""GPU parity of decode attention (libg4attn g4a_decode) against the CPU oracle and the
golden vectors, at the contract tolerance |d| <= 2e-3 + 1e-2|ref|; mask sets exact.

Cases follow the reference's own decode tests (tests/test_gemma3_kernels_gpu.py:372-395,
tests/test_gemma4_kernels_gpu.py:63-80, tests/test_kernels_dsl_parity.py:726-782) and
BASELINE configs 1, 2 (global and sliding) and 4.
"""
import ctypes

import numpy as np
import pytest
import torch

import oracle.attention as O
import slang_amd as sa
from helpers import contract_close, gold, srq_close

pytestmark = pytest.mark.gpu
DEV = "cuda"


def t(x, dtype=None):
    x = torch.from_numpy(np.ascontiguousarray(x))
    return (x if dtype is None else x.to(dtype)).to(DEV)


def run(q, k, v, key_len, cfg, **kw):
    out = sa.decode(t(q), t(k), t(v), key_len, cfg, **{n: (t(a) if isinstance(a, np.ndarray) else a)
                                                       for n, a in kw.items()})
    torch.cuda.synchronize()
    return out.cpu().numpy()


# ---------------------------------------------------------------- golden vectors
def test_golden_g3_fused_f32_cache():
    z = gold("g3_fused.npz")
    k32, v32 = z["k"].astype(np.float32), z["v"].astype(np.float32)
    for i, kl in enumerate(z["key_len"]):
        cfg = sa.AttnConfig(4, 1, 256, int(z["window"][i]), float(z["scale"]))
        got = run(z["q"], k32, v32, [int(kl)], cfg)
        contract_close(got, z["expected"][i], f"g3_fused kv_len={kl}")


@pytest.mark.parametrize("tag", ["hd256_s0", "hd512_s0", "hd256_s3", "hd512_s5"])
def test_golden_g4_fused(tag):
    z = gold("g4_fused.npz")
    hd = int(tag[2:5])
    cfg = sa.AttnConfig(8, 1, hd, int(z[f"{tag}_window"]))
    got = run(z[f"{tag}_q"], z[f"{tag}_k"], z[f"{tag}_v"], [int(z["key_len"])], cfg)
    contract_close(got, z[f"{tag}_expected"], tag)


@pytest.mark.parametrize("tag", ["hd256_len90", "hd512_len90"])
def test_golden_attn101(tag):
    """attn_101's own test case (q-norm, random gain and tables, G = 8) incl. the OUT_Q srq."""
    z = gold("attn101.npz")
    hd, kl = int(tag[2:5]), int(tag.split("len")[1])
    kw = dict(q_gain=z[f"{tag}_w"], rope_cos=z[f"{tag}_cos"][None], rope_sin=z[f"{tag}_sin"][None])
    got = run(z[f"{tag}_q"], z[f"{tag}_k"], z[f"{tag}_v"], [kl], sa.AttnConfig(8, 1, hd), **kw)
    contract_close(got, z[f"{tag}_expected"], tag)
    oq = float(z["out_q"])
    gq = run(z[f"{tag}_q"], z[f"{tag}_k"], z[f"{tag}_v"], [kl], sa.AttnConfig(8, 1, hd, out_q=oq), **kw)
    srq_close(gq, z[f"{tag}_expected"], oq, tag)


@pytest.mark.parametrize("window", [0, 40])
def test_golden_g4e2b(window):
    z = gold("g4e2b_decode.npz")
    got = run(z["q"], z["k"], z["v"], [int(z["key_len"])], sa.AttnConfig(8, 2, 256, window),
              q_gain=z["w"], rope_cos=z["cos"][None], rope_sin=z["sin"][None])
    contract_close(got, z[f"expected_w{window}"], f"g4e2b w={window}")


# ---------------------------------------------------------------- BASELINE configs
def config2_inputs(T, theta, seed=7, nH=8, kvH=2, hd=256):
    """Config 2: q, k, v ~ N(0,1); k RMSNorm*gain + RoPE and v RMSNorm written as f16 rows."""
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((nH, hd)).astype(np.float32)
    qg = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    kg = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    kr = rng.standard_normal((T, kvH, hd)).astype(np.float32)
    vr = rng.standard_normal((T, kvH, hd)).astype(np.float32)
    cos, sin = O.rope_tables(np.arange(T), hd, theta)
    k, v = O.kv_write(kr, vr, kg, cos, sin)
    return q, qg, k, v, cos[T - 1], sin[T - 1]


@pytest.mark.parametrize("window,theta", [(0, 1e6), (512, 1e4)])
def test_config2(window, theta):
    T = 4096
    q, qg, k, v, c, s = config2_inputs(T, theta)
    cfg = sa.AttnConfig(8, 2, 256, window)
    got = run(q, k, v, [T], cfg, q_gain=qg, rope_cos=c[None], rope_sin=s[None])
    ref = O.decode_attention(q, k, v, T, 2, q_gain=qg, cos=c, sin=s, window=window)
    contract_close(got, ref, f"config2 W={window}")


def test_config1_f32_cache_no_norm():
    rng = np.random.default_rng(1)
    q = rng.standard_normal((4, 256)).astype(np.float32)
    k = rng.standard_normal((1024, 1, 256)).astype(np.float32)
    v = rng.standard_normal((1024, 1, 256)).astype(np.float32)
    cfg = sa.AttnConfig(4, 1, 256, 0, 1 / 16)
    got = run(q, k, v, [1024], cfg)
    contract_close(got, O.decode_attention(q, k, v, 1024, 1, scale=1 / 16), "config1")


def test_config4_batched_long_context():
    """16 sequences, key lengths ~ U[1024, 32768], contiguous per-sequence caches."""
    B, nH, kvH, hd, Tmax = 16, 8, 2, 256, 32768
    lens = np.random.default_rng(4).integers(1024, 32769, size=B).astype(np.int32)
    g = torch.Generator(device=DEV).manual_seed(4)
    q = torch.randn(B, nH, hd, device=DEV, generator=g)
    k = torch.randn(B, Tmax, kvH, hd, device=DEV, generator=g).half()
    v = torch.randn(B, Tmax, kvH, hd, device=DEV, generator=g).half()
    out = sa.decode(q, k, v, t(lens), sa.AttnConfig(nH, kvH, hd))
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    qn = q.cpu().numpy()
    for b in range(B):
        L = int(lens[b])
        ref = O.decode_attention(qn[b], k[b, :L].cpu().numpy(), v[b, :L].cpu().numpy(), L, kvH)
        contract_close(got[b], ref, f"config4 seq {b} len {L}")


# ---------------------------------------------------------------- shapes and edges
@pytest.mark.parametrize("nH,kvH,hd", [(2, 2, 256), (4, 2, 256), (8, 1, 512), (4, 1, 512), (8, 8, 256)])
@pytest.mark.parametrize("T,window", [(1, 0), (17, 0), (300, 0), (1500, 0), (300, 64), (2049, 512)])
def test_group_sizes_and_lengths(nH, kvH, hd, T, window):
    rng = np.random.default_rng(T * 31 + nH)
    q = rng.standard_normal((nH, hd)).astype(np.float32)
    qg = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    k = rng.standard_normal((T, kvH, hd)).astype(np.float32)
    v = rng.standard_normal((T, kvH, hd)).astype(np.float32)
    k, v = O.kv_write(k, v, (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32))
    c, s = O.rope_tables([T - 1], hd, 1e4)
    got = run(q, k, v, [T], sa.AttnConfig(nH, kvH, hd, window), q_gain=qg, rope_cos=c, rope_sin=s)
    ref = O.decode_attention(q, k, v, T, kvH, q_gain=qg, cos=c[0], sin=s[0], window=window)
    contract_close(got, ref, f"nH={nH} kvH={kvH} hd={hd} T={T} W={window}")


def test_ragged_batch_with_window():
    B, nH, kvH, hd, Tmax = 5, 8, 2, 256, 700
    lens = np.array([1, 16, 17, 512, 700], np.int32)
    rng = np.random.default_rng(5)
    q = rng.standard_normal((B, nH, hd)).astype(np.float32)
    k = rng.standard_normal((B, Tmax, kvH, hd)).astype(np.float16)
    v = rng.standard_normal((B, Tmax, kvH, hd)).astype(np.float16)
    c, s = O.rope_tables(lens - 1, hd, 1e4)
    cfg = sa.AttnConfig(nH, kvH, hd, 300)
    got = run(q, k, v, t(lens), cfg, rope_cos=c, rope_sin=s)
    ref = O.decode_attention_batched(q, k, v, lens, kvH, cos=c, sin=s, window=300)
    contract_close(got, ref, "ragged batch")


@pytest.mark.parametrize("B,nH,kvH,hd,kv_dtype,window", [
    (80, 8, 2, 256, np.float16, 0),     # more than 64 sequences: the plan's multi-group passes
    (80, 8, 2, 256, np.float16, 96),
    (70, 4, 1, 512, np.float16, 0),     # hd 512: one resident workgroup per CU
    (67, 4, 2, 256, np.float32, 0),     # f32 caches
    (300, 8, 2, 256, np.float16, 0),    # more pairs than resident workgroups: the grid grows
])
def test_work_list_many_ragged_sequences(B, nH, kvH, hd, kv_dtype, window):
    """Several sequences run as one work list of equal-length units over all of them
    (sequence, kv head, split in order). Lengths include 0 (no unit, zero output), 1, and
    one sequence far longer than the rest, which takes most of the units."""
    rng = np.random.default_rng(B + hd)
    lens = rng.integers(0, 300, size=B).astype(np.int32)
    lens[:4] = [0, 1, 2900, 16]
    Tmax = int(lens.max())
    q = rng.standard_normal((B, nH, hd)).astype(np.float32)
    k = rng.standard_normal((B, Tmax, kvH, hd)).astype(kv_dtype)
    v = rng.standard_normal((B, Tmax, kvH, hd)).astype(kv_dtype)
    got = run(q, k, v, t(lens), sa.AttnConfig(nH, kvH, hd, window))
    for b in range(B):
        L = int(lens[b])
        if L == 0:
            assert np.array_equal(got[b], np.zeros_like(got[b])), f"seq {b} has no keys"
            continue
        ref = O.decode_attention(q[b], k[b, :L].astype(np.float32), v[b, :L].astype(np.float32), L, kvH,
                                 window=window)
        contract_close(got[b], ref, f"seq {b} len {L}")


def test_work_list_skewed_pair():
    """Two sequences, one 64x longer: the long one is cut into many units, the short one
    into one, and the merge finds each sequence's units."""
    lens = np.array([8192, 128], np.int32)
    rng = np.random.default_rng(21)
    q = rng.standard_normal((2, 8, 256)).astype(np.float32)
    k = rng.standard_normal((2, 8192, 2, 256)).astype(np.float16)
    v = rng.standard_normal((2, 8192, 2, 256)).astype(np.float16)
    got = run(q, k, v, t(lens), sa.AttnConfig(8, 2, 256))
    for b in range(2):
        L = int(lens[b])
        ref = O.decode_attention(q[b], k[b, :L].astype(np.float32), v[b, :L].astype(np.float32), L, 2)
        contract_close(got[b], ref, f"seq {b} len {L}")


@pytest.mark.parametrize("T", [1, 63, 64, 65, 255, 256, 257, 511])
@pytest.mark.parametrize("dw", [None, -1, 0, 1])
def test_mask_set_exact(T, dw):
    """q = 0 gives every attended key weight 1/n; one-hot V rows (v_j = e_j, hd 512) turn the
    output into the indicator of the attended set, which must be exactly [max(0,T-W), T)."""
    hd = 512
    window = 0 if dw is None else max(1, T + dw)
    k = np.random.default_rng(T).standard_normal((T, 1, hd)).astype(np.float16)
    v = np.zeros((T, 1, hd), np.float16)
    v[np.arange(T), 0, np.arange(T)] = 1
    got = run(np.zeros((2, hd), np.float32), k, v, [T], sa.AttnConfig(2, 1, hd, window))
    lo = max(0, T - window) if window else 0
    assert set(np.nonzero(got[0] > 1e-6)[0]) == set(range(lo, T))
    np.testing.assert_allclose(got[0][lo:T], 1.0 / (T - lo), rtol=1e-5)


@pytest.mark.parametrize("T,window", [(4096, 0), (4096, 512), (1000, 999), (1000, 1)])
def test_mask_leak_marker(T, window):
    """Keys outside the window score +8 and carry V = 1000; inside keys score 0, V = 1.
    Any leaked key pulls the output far above 1."""
    hd = 256
    lo = max(0, T - window) if window else 0
    q = np.zeros((4, hd), np.float32)
    q[:, 0] = 1.0
    k = np.zeros((T, 1, hd), np.float16)
    v = np.ones((T, 1, hd), np.float16)
    k[:lo, 0, 0] = 8.0
    v[:lo] = 1000.0
    got = run(q, k, v, [T], sa.AttnConfig(4, 1, hd, window))
    np.testing.assert_allclose(got, 1.0, atol=1e-5)


def test_deterministic_and_workspace_reuse():
    """Repeated calls are bit-identical, also when the workspace holds stale partials from a
    different call (the reference re-zeroes its ticket per call, kernels_dsl.py:1714-1715;
    this build keeps no state in the workspace between calls)."""
    T = 4096
    q, qg, k, v, c, s = config2_inputs(T, 1e6, seed=3)
    ws = sa.DecodeWorkspace(DEV)
    cfg = sa.AttnConfig(8, 2, 256)
    args = (t(q), t(k), t(v), [T], cfg)
    kw = dict(q_gain=t(qg), rope_cos=t(c[None]), rope_sin=t(s[None]), workspace=ws)
    a = sa.decode(*args, **kw).clone()
    ws.buf.fill_(0x7f)                      # garbage partials
    b = sa.decode(*args, **kw).clone()
    sa.decode(t(q), t(k), t(v), [1000], cfg, workspace=ws)   # a different split plan in between
    c2 = sa.decode(*args, **kw).clone()
    torch.cuda.synchronize()
    assert torch.equal(a, b) and torch.equal(a, c2)
    assert int(a.count_nonzero()) > 0


def test_stale_nan_workspace_and_empty_sequence():
    """Split slots past a sequence's live splits carry weightless (m = -inf, l = 0) markers:
    stale NaN partials left in the workspace must not leak into the merge, and a sequence
    with no keys gives zeros (the grid is sized for max_key_len = the cache length)."""
    B, nH, kvH, hd, T = 3, 8, 2, 256, 4096
    lens = np.array([T, 100, 0], np.int32)
    rng = np.random.default_rng(11)
    q = rng.standard_normal((B, nH, hd)).astype(np.float32)
    k = rng.standard_normal((B, T, kvH, hd)).astype(np.float16)
    v = rng.standard_normal((B, T, kvH, hd)).astype(np.float16)
    ws = sa.DecodeWorkspace(DEV)
    ws.get(1 << 24).fill_(0xFF)             # every f32 partial reads as NaN
    out = sa.decode(t(q), t(k), t(v), t(lens), sa.AttnConfig(nH, kvH, hd), workspace=ws)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    for b in range(2):
        ref = O.decode_attention(q[b], k[b, :lens[b]], v[b, :lens[b]], int(lens[b]), kvH)
        contract_close(got[b], ref, f"seq {b} len {lens[b]}")
    assert np.array_equal(got[2], np.zeros_like(got[2]))


def test_attn_101_mirror_matches_decode():
    """The reference-slot drop-in (params = (1, keyLen, pos, qH, kvH, W, 0, 0))."""
    z = gold("attn101.npz")
    tag, hd, kl = "hd256_len90", 256, 90
    maxseq = 128
    kc = np.zeros((maxseq, 1, hd), np.float16)
    vc = np.zeros((maxseq, 1, hd), np.float16)
    kc[:kl], vc[:kl] = z[f"{tag}_k"], z[f"{tag}_v"]
    out = torch.zeros(8 * hd, device=DEV)
    sa.attn_101(t(z[f"{tag}_q"].reshape(-1)), t(z[f"{tag}_w"]), t(z[f"{tag}_cos"]), t(z[f"{tag}_sin"]),
                t(kc.reshape(-1)), t(vc.reshape(-1)), sa.DecodeWorkspace(DEV), out,
                (1, kl, kl - 1, 8, 1, 0, 0, 0), head_dim=hd)
    torch.cuda.synchronize()
    contract_close(out.cpu().numpy().reshape(8, hd), z[f"{tag}_expected"], "attn_101 mirror")
    with pytest.raises(ValueError):
        sa.attn_101(t(z[f"{tag}_q"].reshape(-1)), None, None, None, t(kc.reshape(-1)),
                    t(vc.reshape(-1)), None, out, (1, kl, kl, 8, 1, 0, 0, 0), head_dim=hd)


# ---------------------------------------------------------------- fused KV write
@pytest.mark.parametrize("B,nH,kvH,hd,window,cache,k_in_q", [
    (1, 8, 2, 256, 0, torch.float16, 0.0),       # config 2 shape, one split per 64 keys
    (1, 8, 2, 256, 512, torch.float16, 0.02),    # sliding, srq'd inputs
    (1, 4, 1, 512, 0, torch.float16, 0.0),       # hd 512
    (1, 8, 2, 256, 0, torch.float32, 0.0),       # f32 caches
    (5, 8, 2, 256, 0, torch.float16, 0.0),       # a batch: the work list
    (3, 4, 1, 512, 96, torch.float16, 0.0),
])
def test_decode_kv_matches_kv_write_then_decode(B, nH, kvH, hd, window, cache, k_in_q):
    """g4a_decode_kv writes the same cache rows as g4a_kv_write (shared arithmetic, bit for
    bit) and returns the same output as g4a_kv_write followed by g4a_decode; both meet the
    contract against the oracle's kv_write + decode_attention."""
    rng = np.random.default_rng(B * 100 + hd + window)
    lens = np.array([rng.integers(1, 3000) for _ in range(B)], np.int32)
    lens[0] = 2049 if B == 1 else lens[0]
    Tmax = int(lens.max()) + 3
    q = t(rng.standard_normal((B, nH, hd)).astype(np.float32))
    qg = t((1 + 0.1 * rng.standard_normal(hd)).astype(np.float32))
    kg = t((1 + 0.1 * rng.standard_normal(hd)).astype(np.float32))
    kraw = t(rng.standard_normal((B, kvH, hd)).astype(np.float32))
    vraw = t(rng.standard_normal((B, kvH, hd)).astype(np.float32))
    c, s = O.rope_tables(lens - 1, hd, 1e4)
    c, s = t(c), t(s)
    base_k = torch.from_numpy(rng.standard_normal((B, Tmax, kvH, hd)).astype(np.float32)).to(DEV, cache)
    base_v = torch.from_numpy(rng.standard_normal((B, Tmax, kvH, hd)).astype(np.float32)).to(DEV, cache)
    cfg = sa.AttnConfig(nH, kvH, hd, window)
    kvcfg = sa.AttnConfig(kvH, kvH, hd)
    # separate: kv_write per sequence at its position, then decode
    k1, v1 = base_k.clone(), base_v.clone()
    for b in range(B):
        p = int(lens[b]) - 1
        sa.kv_write(kraw[b:b + 1], vraw[b:b + 1], k1[b], v1[b], p, kvcfg, k_gain=kg, rope_cos=c[b:b + 1],
                    rope_sin=s[b:b + 1], k_in_q=k_in_q, v_in_q=k_in_q)
    out1 = sa.decode(q, k1, v1, t(lens), cfg, q_gain=qg, rope_cos=c, rope_sin=s)
    # fused
    k2, v2 = base_k.clone(), base_v.clone()
    out2 = sa.decode(q, k2, v2, t(lens), cfg, q_gain=qg, rope_cos=c, rope_sin=s, k_new=kraw, v_new=vraw,
                     k_gain=kg, k_in_q=k_in_q, v_in_q=k_in_q)
    torch.cuda.synchronize()
    assert torch.equal(k1, k2) and torch.equal(v1, v2), "cache rows differ from g4a_kv_write's"
    assert torch.equal(out1, out2), "fused decode differs from kv_write + decode"
    # and against the oracle
    qn, kn, vn = q.cpu().numpy(), k2.float().cpu().numpy(), v2.float().cpu().numpy()
    cn, sn = c.cpu().numpy(), s.cpu().numpy()
    got = out2.cpu().numpy()
    for b in range(B):
        L = int(lens[b])
        kref, vref = O.kv_write(kraw[b:b + 1].cpu().numpy(), vraw[b:b + 1].cpu().numpy(), kg.cpu().numpy(),
                                cn[b:b + 1], sn[b:b + 1], k_in_q=k_in_q, v_in_q=k_in_q,
                                cache_dtype=np.float32 if cache == torch.float32 else np.float16)
        contract_close(kn[b, L - 1:L], kref.astype(np.float32), f"seq {b} k row")
        ref = O.decode_attention(qn[b], kn[b, :L], vn[b, :L], L, kvH, q_gain=qg.cpu().numpy(), cos=cn[b],
                                 sin=sn[b], window=window)
        contract_close(got[b], ref, f"seq {b} len {L}")


@pytest.mark.parametrize("B,window,fused", [(1, 0, False), (1, 512, False), (4, 0, False), (1, 0, True)])
def test_host_key_len_matches_device_key_len(B, window, fused):
    """A host-given length (key_len NULL at the C ABI, max_key_len exact) and the same length
    in a device array give bit-identical outputs (and cache rows, with the fused KV write)."""
    rng = np.random.default_rng(31 + B + window)
    T, nH, kvH, hd = 2049, 8, 2, 256
    q = t(rng.standard_normal((B, nH, hd)).astype(np.float32))
    qg = t((1 + 0.1 * rng.standard_normal(hd)).astype(np.float32))
    c, s = O.rope_tables([T - 1] * B, hd, 1e4)
    c, s = t(c), t(s)
    k = torch.from_numpy(rng.standard_normal((B, T + 7, kvH, hd)).astype(np.float16)).to(DEV)
    v = torch.from_numpy(rng.standard_normal((B, T + 7, kvH, hd)).astype(np.float16)).to(DEV)
    cfg = sa.AttnConfig(nH, kvH, hd, window)
    kw = dict(q_gain=qg, rope_cos=c, rope_sin=s)
    if fused:
        kw.update(k_new=t(rng.standard_normal((B, kvH, hd)).astype(np.float32)),
                  v_new=t(rng.standard_normal((B, kvH, hd)).astype(np.float32)), k_gain=qg)
    k1, v1, k2, v2 = k.clone(), v.clone(), k.clone(), v.clone()
    dev_len = torch.full((B,), T, dtype=torch.int32, device=DEV)
    a = sa.decode(q, k1, v1, dev_len, cfg, max_key_len=T, **kw)  # the same split plan
    b = sa.decode(q, k2, v2, [T] * B, cfg, **kw)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    assert torch.equal(k1, k2) and torch.equal(v1, v2)


# ---------------------------------------------------------------- f32-accurate scores
def test_decode_scores_are_f32_accurate():
    """The decode keeps q at f32 accuracy as an f16 high part plus an f16 low part. Both parts
    must come from one f32 value: a high part rounded from a different evaluation of q (a fused
    multiply-convert rounds once, a multiply then a convert twice) leaves hi + lo one f16 ulp
    off wherever q sits on an f16 rounding tie (about one element in 4096), a score error of up
    to ~1e-2 and an output error of several 1e-3 when such a key dominates.

    White-box: with every key of split d equal to e_d (a unit row), split d's score maximum,
    which the decode leaves in its workspace ((m, l) pairs [pair][split][G], m in log2 units),
    is exactly the kernel's q_d. 16 q rows with gain and RoPE (32,768 q elements): each must
    match the oracle's f32 q to a few f32 ulps."""
    T, nH, kvH, hd = 16384, 8, 2, 256        # 64 keys per split, 256 splits per kv head
    kc = torch.zeros(T, kvH, hd, device=DEV, dtype=torch.float16)
    for d in range(hd):
        kc[64 * d:64 * d + 64, :, d] = 1.0
    vc = torch.zeros_like(kc)
    cfg = sa.AttnConfig(nH, kvH, hd)
    rng = np.random.default_rng(77)
    lib = sa._lib.load()
    c = cfg.c(0)
    assert lib.g4a_decode_ws_bytes(ctypes.byref(c), 1, T) >= 2 * 256 * 4 * 8
    worst = 0.0
    for r in range(16):
        q = rng.standard_normal((nH, hd)).astype(np.float32)
        qg = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
        cos, sin = O.rope_tables([int(rng.integers(0, 1 << 20))], hd, 1e6 if r % 2 else 1e4)
        ws = sa.DecodeWorkspace(DEV)
        sa.decode(t(q), kc, vc, [T], cfg, q_gain=t(qg), rope_cos=t(cos), rope_sin=t(sin), workspace=ws)
        torch.cuda.synchronize()
        ml = ws.buf[:2 * 256 * 4 * 8].view(torch.float32).view(kvH, 256, nH // kvH, 2).cpu().numpy()
        q_kernel = (ml[..., 0].astype(np.float64) / np.log2(np.e)).transpose(0, 2, 1).reshape(nH, hd)
        q_ref = O._prep_q(q, qg, cos, sin, 1e-6).astype(np.float64)
        err = np.abs(q_kernel - q_ref) / np.maximum(np.abs(q_ref), 1.0)
        worst = max(worst, float(err.max()))
        assert err.max() < 2e-6, f"row {r}: kernel q off by {err.max():.2e} (relative) at {np.unravel_index(err.argmax(), err.shape)}"
    print(f"decode q vs oracle q: worst relative difference {worst:.2e}")
