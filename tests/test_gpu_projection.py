"""GPU parity of the q/k/v producer (g4a_dequant, g4a_qkv_gemv, g4a_srqh, g4a_gemm16) against the
projection oracle (oracle/projection.py), through the C ABI.

* dequant: bit-exact (the same f32 product rounded to f16), all widths, including the
  E2B q matrix [2048][1536];
* decode GEMV: the reference test's geometries (qd, hd) = (2048, 256) and (4096, 512)
  (tests/test_kernels_dsl_parity.py:658-700) plus BASELINE's kvH 2 shape (kv_dim 512),
  the KV-sharing q-only form and a hidden width past 2048; within 2e-3 + 1e-2|ref|
  unquantised, and on the srq grid within one step with srq scales;
* prefill GEMM: every f16 result within 2e-3 + 1e-2|ref| of the correctly rounded product,
  and within one f16 ulp of it wherever |ref| >= 0.25 (below that the f32 accumulation's
  own error over K = 1536, up to ~2e-5, can exceed an f16 ulp); f32 srq results within one
  grid step; at S = 1024 and ragged token counts.
"""
import numpy as np
import pytest
import torch

import oracle.projection as P
import slang_amd as sa
from helpers import contract_close, f16_ulp_close, srq_close

pytestmark = pytest.mark.gpu
DEV = "cuda"


def t(x):
    return torch.from_numpy(np.ascontiguousarray(x)).to(DEV)


def words(rng, n):
    return rng.integers(0, 2 ** 32, size=n, dtype=np.uint64).astype(np.uint32)


def dev_words(w):
    return t(w.view(np.int32))


def gemm_f16_close(got, ref, what):
    got = np.asarray(got, np.float16)
    err = contract_close(got.astype(np.float32), ref.astype(np.float32), what)
    big = np.abs(ref.astype(np.float32)) >= 0.25
    f16_ulp_close(got[big], ref[big], what + " (|ref| >= 0.25)")
    return err


@pytest.mark.parametrize("bits,n_in,n_out", [(2, 256, 64), (4, 256, 64), (8, 256, 64),
                                             (4, 1536, 2048), (2, 1536, 96)])
def test_dequant_bit_exact(bits, n_in, n_out):
    rng = np.random.default_rng(131 + bits)
    w = words(rng, n_out * n_in * bits // 32)
    sc = (rng.random(n_out).astype(np.float32) * 0.01 + 0.001)
    print(f"dequant bits {bits} [{n_out}x{n_in}]", flush=True)
    got = sa.dequant(dev_words(w), t(sc), n_in, n_out)
    assert sa.packed_bits(dev_words(w), n_in, n_out) == bits
    torch.cuda.synchronize()
    ref = P.dequant_f16(w, sc, n_in, n_out, bits)
    assert np.array_equal(got.cpu().numpy().view(np.uint16), ref.view(np.uint16))


def test_dq_f16_dropin_scale_offset():
    """_dq passes the k/v scales as an offset into qkv_scales (prefill_gpu.py:330-333)."""
    rng = np.random.default_rng(7)
    w = words(rng, 64 * 256 // 8)
    sc = rng.random(200).astype(np.float32) + 0.1
    out = torch.empty(64, 256, device=DEV, dtype=torch.float16)
    sa.dq_f16(dev_words(w), t(sc), out, (256, 64), scale_offset=128 * 4)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), P.dequant_f16(w, sc[128:], 256, 64, 4))


def gemv_case(seed, hidden, qd, kvd):
    rng = np.random.default_rng(seed)
    a = rng.standard_normal(hidden).astype(np.float32)
    wpr = hidden // 8
    qb, kb, vb = words(rng, qd * wpr), words(rng, kvd * wpr), words(rng, kvd * wpr)
    sc = (rng.random(qd + 2 * kvd).astype(np.float32) * 0.01 + 0.001)
    suma = np.array([a.sum(dtype=np.float64)], np.float32)
    return a, suma, qb, kb, vb, sc


@pytest.mark.parametrize("hidden,qd,kvd", [(1536, 2048, 256), (1536, 4096, 512), (1536, 2048, 512),
                                           (2560, 512, 256), (64, 8, 8)])
@pytest.mark.parametrize("scales", [(0.0, 0.0, 0.0), (0.03125, 0.0234375, 0.0156)])
def test_qkv_gemv_matches_oracle(hidden, qd, kvd, scales):
    a, suma, qb, kb, vb, sc = gemv_case(111, hidden, qd, kvd)
    print(f"qkv_gemv hidden {hidden} q {qd} kv {kvd} scales {scales}", flush=True)
    got = sa.qkv_gemv(t(a), t(suma), dev_words(qb), t(sc), qd, kvd, k_bits=dev_words(kb),
                      v_bits=dev_words(vb), q_out=scales[0], k_out=scales[1], v_out=scales[2])
    torch.cuda.synchronize()
    raw = P.qkv_gemv(a, suma[0], qb, kb, vb, sc, qd, kvd)  # unquantised
    for nm, g, r, s in zip("qkv", got, raw, scales):
        g = g.cpu().numpy()
        if s == 0.0:
            contract_close(g, r, f"out_{nm}")
        else:
            srq_close(g, r, s, f"out_{nm}")
        assert np.count_nonzero(g), f"out_{nm} empty"


@pytest.mark.parametrize("hidden,qd,kvd", [(1536, 2048, 256), (1536, 4096, 0), (2048, 512, 512), (256, 64, 8)])
def test_qkv_gemv_norm_prologue(hidden, qd, kvd):
    """g4a_qkv_gemv_norm: the previous layer's tail x = (x2 + rms(p) * w1) * mult and the input
    norm a = srq(rms(x) * w2, q2) made in the kernel. x against the oracle at the contract, a
    on its grid from the GPU's own x, sum_a against the sum of a, and q/k/v bit for bit equal
    to g4a_qkv_gemv run on the stored a and sum_a (the same arithmetic from memory)."""
    from oracle.decoder import rms_norm
    from slang_amd.decoder import norm_in
    rng = np.random.default_rng(hidden + qd)
    _, _, qb, kb, vb, sc = gemv_case(7, hidden, qd, kvd)
    p = (0.3 * rng.standard_normal(hidden)).astype(np.float32)
    x2 = rng.standard_normal(hidden).astype(np.float32)
    w1 = (1 + 0.1 * rng.standard_normal(hidden)).astype(np.float32)
    w2 = (1 + 0.1 * rng.standard_normal(hidden)).astype(np.float32)
    mult, q2 = 0.8125, 0.05
    print(f"qkv_gemv_norm hidden {hidden} q {qd} kv {kvd}", flush=True)
    x_out = torch.full((hidden,), 7.0, device=DEV)
    a_out = torch.full((hidden,), 7.0, device=DEV)
    s_out = torch.full((1,), 7.0, device=DEV)
    kw = dict(k_bits=dev_words(kb), v_bits=dev_words(vb), q_out=0.03125, k_out=0.0234375, v_out=0.0156)
    # the prologue struct holds raw pointers: its tensors must outlive the calls
    dp, dx2, dw1, dw2, dqb, dsc = t(p), t(x2), t(w1), t(w2), dev_words(qb), t(sc)
    pro = norm_in(dp, dx2, dw1, x_out, w2=dw2, q2=q2, mult=mult)
    got = sa.qkv_gemv(a_out, s_out, dqb, dsc, qd, kvd, pro=pro, hidden=hidden, **kw)
    torch.cuda.synchronize()
    x = x_out.cpu().numpy()
    contract_close(x, (x2 + rms_norm(p, w1)) * np.float32(mult), "x")
    a = a_out.cpu().numpy()
    srq_close(a, rms_norm(x, w2), q2, "a")
    assert abs(float(s_out.cpu()[0]) - a.sum(dtype=np.float64)) <= 1e-5 * np.abs(a).sum() + 1e-6
    ref = sa.qkv_gemv(a_out, s_out, dqb, dsc, qd, kvd, **kw)
    torch.cuda.synchronize()
    for nm, g, r in zip("qkv", got, ref):
        if r is not None:
            assert torch.equal(g, r), f"out_{nm} differs from g4a_qkv_gemv on the stored input"
    # the stores are optional: without them the outputs are the same
    pro = norm_in(dp, dx2, dw1, x_out, w2=dw2, q2=q2, mult=mult)
    pro.x_out = None
    again = sa.qkv_gemv(None, None, dqb, dsc, qd, kvd, pro=pro, hidden=hidden, **kw)
    torch.cuda.synchronize()
    for g, r in zip(again, ref):
        if r is not None:
            assert torch.equal(g, r)


def test_qkv_70_dropin_and_shared_layer():
    a, suma, qb, kb, vb, sc = gemv_case(5, 1536, 2048, 256)
    oq = torch.full((2048,), 7.0, device=DEV)
    ok = torch.full((256,), 7.0, device=DEV)
    ov = torch.full((256,), 7.0, device=DEV)
    sa.qkv_70(t(a), dev_words(qb), dev_words(kb), dev_words(vb), t(sc), t(suma), oq, ok, ov,
              (0.0, 0.0, 0.0, 0.0))
    torch.cuda.synchronize()
    rq, rk, rv = P.qkv_gemv(a, suma[0], qb, kb, vb, sc, 2048, 256)
    contract_close(oq.cpu().numpy(), rq, "q")
    contract_close(ok.cpu().numpy(), rk, "k")
    contract_close(ov.cpu().numpy(), rv, "v")
    # KV-sharing layer: q only, the k/v outputs untouched
    ok.fill_(7.0)
    ov.fill_(7.0)
    oq.zero_()
    sa.qkv_70(t(a), dev_words(qb), dev_words(qb), dev_words(qb), t(sc), t(suma), oq, ok, ov,
              (0.0, 0.0, 0.0, 0.0), shared=True)
    torch.cuda.synchronize()
    contract_close(oq.cpu().numpy(), rq, "q shared")
    assert (ok.cpu().numpy() == 7.0).all() and (ov.cpu().numpy() == 7.0).all()


def test_qkv_gemv_zero_point_and_one_hot():
    """Closed forms on the GPU: all values at the zero point give 0; a one-hot input picks
    out scale * (q - 8) of one column."""
    hidden, qd = 1536, 64
    rng = np.random.default_rng(9)
    a = rng.standard_normal(hidden).astype(np.float32)
    zp = np.full(qd * hidden // 8, 0x88888888, np.uint32)
    sc = np.ones(qd, np.float32)
    q, _, _ = sa.qkv_gemv(t(a), t(np.array([a.sum(dtype=np.float64)], np.float32)), dev_words(zp), t(sc), qd)
    torch.cuda.synchronize()
    assert np.abs(q.cpu().numpy()).max() < 1e-3
    vals = rng.integers(0, 16, size=(qd, hidden))
    wb = P.pack_values(vals, 4).reshape(-1)
    sc = rng.random(qd).astype(np.float32) + 0.5
    for j in (0, 1, 31, 32, 1535):
        e = np.zeros(hidden, np.float32)
        e[j] = 1.0
        q, _, _ = sa.qkv_gemv(t(e), t(np.ones(1, np.float32)), dev_words(wb), t(sc), qd)
        torch.cuda.synchronize()
        np.testing.assert_allclose(q.cpu().numpy(), sc * (vals[:, j] - 8), rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("M,N,K", [(1024, 2048, 1536), (1024, 512, 1536), (200, 256, 1536),
                                   (1, 128, 64), (129, 384, 192)])
def test_proj_gemm_matches_oracle(M, N, K):
    rng = np.random.default_rng(M + N + K)
    a = rng.standard_normal((M, K)).astype(np.float32)
    wb = words(rng, N * K // 8)
    sc = (rng.random(N).astype(np.float32) * 0.01 + 0.02)
    print(f"proj_gemm M {M} N {N} K {K}", flush=True)
    w16 = sa.dequant(dev_words(wb), t(sc), K, N)
    c16 = sa.proj(t(a), w16)
    cq = sa.proj(t(a), w16, out_f32=True, out_q=0.03125)
    torch.cuda.synchronize()
    wref = P.dequant_f16(wb, sc, K, N, 4)
    ref = P.proj_gemm(a, wref)
    err = gemm_f16_close(c16.cpu().numpy(), ref, "f16 out")
    print(f"max abs err {err:.2e}", flush=True)
    srq_close(cq.cpu().numpy(), ref.astype(np.float32), 0.03125, "q path srq")


@pytest.mark.parametrize("M,K,ns", [(1024, 1536, (2048, 512, 512)), (200, 1536, (256,)),
                                    (1, 64, (128, 128)), (129, 192, (384, 128, 256)),
                                    (1024, 768, (4096, 4096))])
def test_gemm16_grouped_matches_oracle(M, K, ns):
    """g4a_gemm16: up to three products over one f16 A in one launch, each f16 (gemm_tiled)
    or f32 srq'd (srq_b); ragged M (rows past M read as zeros, nothing stored past M).
    The last case has 512 tiles of 128 x 128 and runs on them; the others have fewer and run
    on 128 x 64 tiles."""
    rng = np.random.default_rng(M + K + len(ns))
    print(f"gemm16 M {M} K {K} n {ns}", flush=True)
    a = rng.standard_normal((M, K)).astype(np.float32)
    a16 = sa.srqh(t(a), 0.0625)
    ws = [(words(rng, n * K // 8), (rng.random(n).astype(np.float32) * 0.01 + 0.02)) for n in ns]
    w16 = [sa.dequant(dev_words(w), t(s), K, n) for (w, s), n in zip(ws, ns)]
    outs = [torch.full((M + 3, n), 7.0, device=DEV, dtype=torch.float32 if i == 0 else torch.float16)
            for i, n in enumerate(ns)]
    sa.gemm16(a16, [(w, o[:M], 0.03125 if i == 0 else None) for i, (w, o) in enumerate(zip(w16, outs))])
    torch.cuda.synchronize()
    a_q = P.srq(a, 0.0625)
    np.testing.assert_array_equal(a16.cpu().numpy(), a_q.astype(np.float16))  # srqh_b exactly
    for i, ((w, s), n, o) in enumerate(zip(ws, ns, outs)):
        ref = P.proj_gemm(a_q, P.dequant_f16(w, s, K, n, 4))
        got = o[:M].float().cpu().numpy()
        if i == 0:
            srq_close(got, ref.astype(np.float32), 0.03125, f"matrix {i} (q path)")
        else:
            gemm_f16_close(got, ref, f"matrix {i}")
        assert (o[M:] == 7.0).all(), "stores past M"


def test_prefill_qkv_block():
    """prefill_gpu.py:327-342 at BASELINE's shapes: q f32 srq'd, kraw/vraw f16, with an
    srqh_b input scale."""
    S, H, qd, kvd = 1024, 1536, 2048, 512
    rng = np.random.default_rng(3)
    a = rng.standard_normal((S, H)).astype(np.float32)
    ws = [(words(rng, n * H // 8), (rng.random(n).astype(np.float32) * 0.01 + 0.02)) for n in (qd, kvd, kvd)]
    w16 = [sa.dequant(dev_words(w), t(s), H, w.size * 8 // H) for w, s in ws]
    q, k, v = sa.prefill_qkv(t(a), *w16, a_in_q=0.0625, q_out=0.03125)
    torch.cuda.synchronize()
    a_q = P.srq(a, 0.0625)
    for got, (w, s), nm in ((k, ws[1], "k"), (v, ws[2], "v")):
        ref = P.proj_gemm(a_q, P.dequant_f16(w, s, H, w.size * 8 // H, 4))
        gemm_f16_close(got.cpu().numpy(), ref, nm)
    refq = P.proj_gemm(a_q, P.dequant_f16(ws[0][0], ws[0][1], H, qd, 4))
    srq_close(q.cpu().numpy(), refq.astype(np.float32), 0.03125, "q")


@pytest.mark.parametrize("M,K,ns", [(1024, 6144, (1536,)), (1024, 2048, (1536,)), (1024, 1536, (256,)),
                                    (200, 1536, (256,)), (512, 1536, (2048, 256, 256)), (77, 4096, (128, 384))])
def test_gemm16_split_k_matches_oracle(M, K, ns):
    """g4a_gemm16_ws: launches with few output tiles split K over several workgroups per tile
    and add the f32 partials in split order. The outputs meet the same bounds as the unsplit
    GEMM, a repeat call is bit-identical (the sum order does not depend on which workgroup
    finishes last), rows past M are not stored, and the tickets are left at zero."""
    rng = np.random.default_rng(M + K + 7 * len(ns))
    print(f"gemm16 split M {M} K {K} n {ns}", flush=True)
    a = rng.standard_normal((M, K)).astype(np.float32)
    a16 = sa.srqh(t(a), 0.0625)
    ws = [(words(rng, n * K // 8), (rng.random(n).astype(np.float32) * 0.01 + 0.02)) for n in ns]
    w16 = [sa.dequant(dev_words(w), t(s), K, n) for (w, s), n in zip(ws, ns)]
    alpha = 0.5
    outs = [torch.full((M + 3, n), 7.0, device=DEV, dtype=torch.float32 if i == 0 else torch.float16)
            for i, n in enumerate(ns)]
    mats = [(w, o[:M], 0.03125 if i == 0 else None, 1.0 if i == 0 else alpha)
            for i, (w, o) in enumerate(zip(w16, outs))]
    gws = sa.GemmWorkspace()
    _, _, tab = sa.projection._gemm_table(a16, mats)
    need = sa._lib.load().g4a_gemm16_ws_bytes(M, K, len(ns), tab)
    assert need > 0, "this shape should split K"
    sa.gemm16(a16, mats, gws)
    first = [o.clone() for o in outs]
    sa.gemm16(a16, mats, gws)
    torch.cuda.synchronize()
    for o, f in zip(outs, first):
        assert torch.equal(o, f), "a repeat call differs"
    assert not gws.buf[:sa._lib.GEMM_TICKET_BYTES].any(), "tickets left non-zero"
    a_q = P.srq(a, 0.0625)
    for i, ((w, s), n, o) in enumerate(zip(ws, ns, outs)):
        ref = P.proj_gemm(a_q, P.dequant_f16(w, s, K, n, 4))
        got = o[:M].float().cpu().numpy()
        if i == 0:
            srq_close(got, ref.astype(np.float32), 0.03125, f"matrix {i} (q path)")
        else:
            ref = (alpha * ref.astype(np.float64)).astype(np.float16)  # f16(alpha * sum)
            gemm_f16_close(got, ref, f"matrix {i}")
        assert (o[M:] == 7.0).all(), "stores past M"


def test_gemm16_split_k_workspace_checks():
    """A workspace shorter than g4a_gemm16_ws_bytes is refused before anything runs."""
    M, K, n = 1024, 2048, 1536
    a16 = torch.zeros(M, K, device=DEV, dtype=torch.float16)
    w = torch.zeros(n, K, device=DEV, dtype=torch.float16)
    o = torch.zeros(M, n, device=DEV, dtype=torch.float16)
    _, _, tab = sa.projection._gemm_table(a16, [(w, o, None)])
    lib = sa._lib.load()
    need = lib.g4a_gemm16_ws_bytes(M, K, 1, tab)
    assert need > sa._lib.GEMM_TICKET_BYTES
    short = torch.zeros(need - 256, device=DEV, dtype=torch.uint8)
    rc = lib.g4a_gemm16_ws(M, K, a16.data_ptr(), 1, tab, short.data_ptr(), short.numel(), None)
    assert rc == -3, "G4A_EWORKSPACE expected"


@pytest.mark.parametrize("M,K,n", [(1024, 1536, 6144), (77, 192, 128), (300, 512, 640)])
@pytest.mark.parametrize("out_q", [0.0, 0.05])
def test_gemm16_geglu_is_gemm16_then_geglu16(M, K, n, out_q):
    """g4a_gemm16_geglu: the gate/up GEMMs with geglu_b in their epilogue give exactly the codes
    of g4a_gemm16 on the two matrices followed by g4a_geglu16 (both against the oracle
    elsewhere), and store nothing past M."""
    from slang_amd.decoder import geglu16
    import oracle.decoder as OD
    rng = np.random.default_rng(M + K + n)
    print(f"gemm16_geglu M {M} K {K} n {n} out_q {out_q}", flush=True)
    a = rng.standard_normal((M, K)).astype(np.float32)
    a16 = sa.srqh(t(a), 0.0625)
    ws = [(words(rng, n * K // 8), (rng.random(n).astype(np.float32) * 0.01 + 0.02)) for _ in range(2)]
    wg, wu = [sa.dequant(dev_words(w), t(s), K, n) for w, s in ws]
    gq, uq = 0.05, 0.04
    out = torch.full((M + 2, n), 7.0, device=DEV, dtype=torch.float16)
    sa.gemm16_geglu(a16, wg, wu, gq, uq, out_q, out=out[:M])
    g16 = torch.empty(M, n, device=DEV, dtype=torch.float16)
    u16 = torch.empty_like(g16)
    sa.gemm16(a16, [(wg, g16, None), (wu, u16, None)])
    ref = geglu16(g16, u16, gq, uq, out_q)
    torch.cuda.synchronize()
    assert torch.equal(out[:M], ref), f"{(out[:M] != ref).sum().item()} codes differ from gemm16 + geglu16"
    assert (out[M:] == 7.0).all(), "stores past M"
    # and the unfused pair is the oracle's geglu_b of the GPU's f16 products (gelu's tanh in
    # another f32 implementation: codes at most one apart, values within the contract)
    want = OD.geglu_codes(g16.cpu().numpy(), u16.cpu().numpy(), gq, uq, out_q).astype(np.float32)
    got = ref.float().cpu().numpy()
    if out_q:
        d = np.abs(got - want)
        assert d.max() <= 1.0 and (d > 0).mean() <= 0.05, f"codes {d.max()} apart, {(d > 0).mean():.2%} off"
    else:
        contract_close(got, want, "geglu values")


def test_split_gemm_and_geglu_gemm_replay_in_a_graph():
    """The K-split GEMM (its tickets return to zero on every call) and the gate/up GEMM with
    geglu_b, captured in one HIP graph: every replay, with eager work and synchronisations
    between them, gives the eager results bit for bit."""
    rng = np.random.default_rng(5)
    M, K, n, K2 = 512, 2048, 1536, 1536
    a16 = sa.srqh(t(rng.standard_normal((M, K)).astype(np.float32)), 0.0625)
    b16 = sa.srqh(t(rng.standard_normal((M, K2)).astype(np.float32)), 0.0625)
    w = sa.dequant(dev_words(words(rng, n * K // 8)), t(rng.random(n).astype(np.float32) * 0.01 + 0.02), K, n)
    wg, wu = [sa.dequant(dev_words(words(rng, 640 * K2 // 8)), t(rng.random(640).astype(np.float32) * 0.01 + 0.02),
                         K2, 640) for _ in range(2)]
    gws = sa.GemmWorkspace()
    o1 = torch.empty(M, n, device=DEV, dtype=torch.float16)
    o2 = torch.empty(M, 640, device=DEV, dtype=torch.float16)

    def run():
        sa.gemm16(a16, [(w, o1, None, 0.5)], gws)
        sa.gemm16_geglu(b16, wg, wu, 0.05, 0.04, 0.05, out=o2)

    run()
    torch.cuda.synchronize()
    ref1, ref2 = o1.clone(), o2.clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        run()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        run()
    for rep in range(3):
        o1.fill_(float("nan"))
        o2.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(o1, ref1), f"replay {rep}: split GEMM differs"
        assert torch.equal(o2, ref2), f"replay {rep}: gate/up GEMM differs"
        assert not gws.buf[:sa._lib.GEMM_TICKET_BYTES].any(), "tickets left non-zero"
        _ = (a16.float() * 2).sum().item()  # eager work between replays


def test_split_gemm_workspace_shared_across_shapes():
    """One workspace for K-split launches of different tile counts and split counts in a row
    (the decoder prefill shares one): every result matches a fresh workspace's bit for bit and
    the tickets are zero after each call."""
    rng = np.random.default_rng(9)
    shared = sa.GemmWorkspace()
    for M, K, n in [(1024, 2048, 1536), (1024, 1536, 256), (512, 6144, 1536), (1024, 2048, 1536), (200, 1536, 256)]:
        a16 = sa.srqh(t(rng.standard_normal((M, K)).astype(np.float32)), 0.0625)
        w = sa.dequant(dev_words(words(rng, n * K // 8)), t(rng.random(n).astype(np.float32) * 0.01 + 0.02), K, n)
        o1 = torch.empty(M, n, device=DEV, dtype=torch.float16)
        o2 = torch.empty_like(o1)
        sa.gemm16(a16, [(w, o1, None)], shared)
        sa.gemm16(a16, [(w, o2, None)], sa.GemmWorkspace())
        torch.cuda.synchronize()
        assert torch.equal(o1, o2), f"M {M} K {K} n {n}: shared workspace result differs"
        assert not shared.buf[:sa._lib.GEMM_TICKET_BYTES].any(), "tickets left non-zero"


def test_norm_prologue_refuses_overlapping_outputs():
    """The norm prologues store x (and z) from workgroup 0 while every other workgroup still
    reads a, res and w1, so an output that overlaps one of them would race: g4a_qkv_gemv_norm
    and the fused GEMVs refuse it (G4A_EINVAL) before launching -- the residual ping-pong of
    the decode step makes it easy to pass res as x_out by mistake."""
    from slang_amd.decoder import norm_in, qgemv_gelu_mul
    hidden, qd, kvd = 256, 64, 8
    _, _, qb, kb, vb, sc = gemv_case(7, hidden, qd, kvd)
    rng = np.random.default_rng(3)
    dp, dx2 = t(rng.standard_normal(hidden).astype(np.float32)), t(rng.standard_normal(hidden).astype(np.float32))
    dw = t(np.ones(hidden, np.float32))
    dqb, dsc = dev_words(qb), t(sc)
    kw = dict(k_bits=dev_words(kb), v_bits=dev_words(vb), q_out=0.03125, k_out=0.0234375, v_out=0.0156)
    for x_out in (dx2, dp, dx2[8:]):
        pro = norm_in(dp, dx2, dw, x_out, w2=dw, q2=0.05)
        with pytest.raises(Exception, match="must not overlap"):
            sa.qkv_gemv(None, None, dqb, dsc, qd, kvd, pro=pro, hidden=hidden, **kw)
    z_out = torch.empty(hidden, device=DEV)
    pro = norm_in(dp, dx2, dw, z_out, w2=dw, z_out=dw, q2=0.05)
    with pytest.raises(Exception, match="must not overlap"):
        sa.qkv_gemv(None, None, dqb, dsc, qd, kvd, pro=pro, hidden=hidden, **kw)
    words = dev_words(rng.integers(0, 2**32, size=qd * hidden // 8, dtype=np.uint64).astype(np.uint32))
    pro = norm_in(dp, dx2, dw, dx2, q2=0.05)
    with pytest.raises(Exception, match="must not overlap"):
        qgemv_gelu_mul(None, words, t(np.ones(qd, np.float32)), t(np.ones(qd, np.float32)), hidden, qd, bits=4,
                       in_q=0.05, pro=pro)


@pytest.mark.parametrize("out_q", [0.0, 0.05])
def test_gelu_tables_give_the_oracles_codes_exactly(out_q):
    """With the exporter's GELU table of the gate grid (export.py:30-33) the prefill MLP tail is
    the runners' arithmetic exactly -- no f32 tanh on either side -- so the fused gate/up GEMM,
    geglu16 and plegate16 equal the oracle's geglu_b codes and plegate_b operands bit for bit
    on the GPU's own f16 products (geglu_b kernels_dsl.py:283, plegate_b :1785)."""
    from slang_amd.decoder import geglu16, plegate16
    import oracle.decoder as OD
    rng = np.random.default_rng(11)
    M, K, n, d = 300, 512, 640, 256
    a16 = sa.srqh(t(rng.standard_normal((M, K)).astype(np.float32)), 0.0625)
    wg, wu = [sa.dequant(dev_words(words(rng, n * K // 8)), t(rng.random(n).astype(np.float32) * 0.01 + 0.02),
                         K, n) for _ in range(2)]
    gq, uq = 0.05, 0.04
    lut = OD.gelu_lut(gq)
    fused = sa.gemm16_geglu(a16, wg, wu, gq, uq, out_q, gelu_lut=t(lut))
    g16 = torch.empty(M, n, device=DEV, dtype=torch.float16)
    u16 = torch.empty_like(g16)
    sa.gemm16(a16, [(wg, g16, None), (wu, u16, None)])
    unfused = geglu16(g16, u16, gq, uq, out_q, gelu_lut=t(lut))
    torch.cuda.synchronize()
    want = OD.geglu_codes(g16.cpu().numpy(), u16.cpu().numpy(), gq, uq, out_q, lut=lut)
    np.testing.assert_array_equal(unfused.cpu().numpy(), want)
    np.testing.assert_array_equal(fused.cpu().numpy(), want)
    lin = (0.3 * rng.standard_normal((M, d))).astype(np.float16)
    ple = rng.standard_normal((M, 3, d)).astype(np.float32)
    lq, oq = 0.03, 0.02
    lut_p = OD.gelu_lut(lq)
    got = plegate16(t(lin), lq, t(ple)[:, 1], 3 * d, oq, gelu_lut=t(lut_p))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(got.cpu().numpy(), OD.plegate_operand(lin, lq, ple[:, 1], oq, lut=lut_p))
