"""GPU parity of the decode step around the attention block (g4a_qgemv and its fused
gate/up and gelu-mul forms, g4a_gemv_f16, g4a_rms_norm, g4a_geglu, g4a_embed,
g4a_softcap_argmax and DecoderStack) against
oracle/decoder.py. SRQ'd outputs are checked on their grid, at most one step from the
oracle's unquantised value; every stage of a layer is checked from the GPU's own inputs."""
import numpy as np
import pytest
import torch

import oracle.decoder as OD
from helpers import chain_close, contract_close, qlin_codes, srq_close
from manifest_fixture import write_model
from oracle.projection import pack_values
from slang_amd import decoder as D
from slang_amd.manifest import load_manifest

pytestmark = pytest.mark.gpu
DEV = "cuda"


def host(t):
    return t.detach().float().cpu().numpy() if t.dtype != torch.int32 else t.cpu().numpy()


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


@pytest.mark.parametrize("bits,n_in,n_out,in_q,out_q", [
    (4, 2048, 1536, 0.01, 0.05),    # o_proj
    (4, 1536, 6144, 0.05, 0.02),    # gate / up
    (2, 1536, 12288, 0.05, 0.02),   # the 2-bit double-wide MLP
    (4, 6144, 1536, 0.01, 0.02),    # down
    (2, 12288, 1536, 0.01, 0.02),
    (2, 16384, 1000, 0.01, 0.02),   # the widest staged x: all four preloaded batches
    (4, 10240, 777, 0.01, 0.02),    # 2.5 batches; 320 chunks: some threads take two
    (8, 1536, 256, 0.05, 0.03),     # per-layer-embedding gate
    (8, 256, 1536, 0.03, 0.01),     # per-layer-embedding projection
    (2, 1536, 4099, 0.0, 0.0),      # lm_head rows (ragged count), no srq
    (8, 16, 3, 0.0, 0.0),           # one chunk per row, fewer rows than a workgroup
])
def test_qgemv_parity(bits, n_in, n_out, in_q, out_q):
    rng = np.random.default_rng(bits * 7 + n_out)
    words = pack_values(rng.integers(0, 1 << bits, size=(n_out, n_in)), bits)
    scale = (0.01 * (1 + rng.random(n_out))).astype(np.float32)
    x = (2 * rng.standard_normal(n_in)).astype(np.float32)
    got = host(D.qgemv(dev(x), dev(words).view(torch.int32).reshape(-1), dev(scale), n_in, n_out, in_q=in_q,
                       out_q=out_q, bits=bits))
    ref = OD.qlin(x, words, scale, n_in, bits, in_q, 0.0)
    if out_q:
        srq_close(got, ref, out_q, f"qgemv {bits}-bit {n_out}x{n_in}")
    else:
        contract_close(got, ref, f"qgemv {bits}-bit {n_out}x{n_in}")


@pytest.mark.parametrize("bits,n_in,n_out", [
    (4, 1536, 6144), (4, 2048, 1531), (8, 256, 1536), (8, 512, 77),
    (2, 1536, 12288),                  # the double-wide MLP's gate / up rows
    (2, 12288, 1536), (4, 6144, 1536),  # down projections: rows wider than a wave's chunks
    (4, 4096, 1536),                    # o_proj of an hd-512 layer
    (2, 16384, 1000), (4, 10240, 777),  # x staged in four / two and a half batches
])
def test_qgemv_integer_dot_is_exact(bits, n_in, n_out):
    """GEMVs with in_q > 0 sum codes times the int8 grid index k = srq's clamp(rint(x / in_q))
    in integers (v_dot4_i32_i8), x staged as k in LDS whether a row group covers the row in one
    pass or not. With out_q 0 the output is then exactly f32(f32(D * in_q) * scale),
    D = sum (c - zp) k over the row computed here in int64: a wrong 2-bit/nibble/byte order,
    zero point or index would change D."""
    rng = np.random.default_rng(bits * 31 + n_out)
    codes = rng.integers(0, 1 << bits, size=(n_out, n_in))
    words = pack_values(codes, bits)
    scale = (0.01 * (1 + rng.random(n_out))).astype(np.float32)
    x = (3 * rng.standard_normal(n_in)).astype(np.float32)  # some |x / in_q| past 127: clamped
    in_q = np.float32(0.03)
    got = host(D.qgemv(dev(x), dev(words).view(torch.int32).reshape(-1), dev(scale), n_in, n_out, in_q=float(in_q),
                       out_q=0.0, bits=bits))
    k = np.clip(np.rint(x / in_q), -128, 127).astype(np.int64)
    assert (np.abs(x / in_q) > 127.5).any()
    d = (codes.astype(np.int64) - (1 << (bits - 1))) @ k
    assert np.abs(d).max() < 1 << 24
    want = (d.astype(np.float32) * in_q).astype(np.float32) * scale
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("table", [False, True])
@pytest.mark.parametrize("bits,n_in,n_out", [(4, 1536, 6144), (2, 1536, 12288), (4, 256, 1024), (8, 512, 64)])
def test_qgemv_geglu_and_gelu_mul(bits, n_in, n_out, table):
    """The gate/up GEMV with its GeGLU and the per-layer-embedding gate GEMV with gelu * mul,
    with reference.py's f32 gelu_tanh, or (table) with GELU taken from the exporter's float64
    table of the gate's output grid by the srq code, as gateup_74/95 and plegate_76 do
    (kernels_dsl.py:867, 1292, 1373)."""
    rng = np.random.default_rng(bits + n_out)
    gw, uw = (pack_values(rng.integers(0, 1 << bits, size=(n_out, n_in)), bits) for _ in range(2))
    gs, us = ((0.01 * (1 + rng.random(n_out))).astype(np.float32) for _ in range(2))
    x = (2 * rng.standard_normal(n_in)).astype(np.float32)
    wd = lambda a: dev(a).view(torch.int32).reshape(-1)  # noqa: E731
    lut = OD.gelu_lut(0.02) if table else None
    got = host(D.qgemv_geglu(dev(x), (wd(gw), dev(gs), 0.05, 0.02), (wd(uw), dev(us), 0.04, 0.03), n_in, n_out,
                             out_q=0.01, bits=bits, gelu_lut=dev(lut) if table else None))
    g = qlin_codes(x, gw, gs, n_in, bits, 0.05, 0.02)
    u = qlin_codes(x, uw, us, n_in, bits, 0.04, 0.03)
    chain_close(got, lambda a, b: OD.gelu_of_srq(a, 0.02, lut) * b, [g, u], f"gate/up {bits}-bit", step=0.01)
    mul = rng.standard_normal(n_out).astype(np.float32)
    got = host(D.qgemv_gelu_mul(dev(x), wd(gw), dev(gs), dev(mul), n_in, n_out, in_q=0.05, out_q=0.02, bits=bits,
                                gelu_lut=dev(lut) if table else None))
    chain_close(got, lambda a: OD.gelu_of_srq(a, 0.02, lut) * mul, [g], f"gelu_mul {bits}-bit")


def test_gemv_f16_parity():
    rng = np.random.default_rng(3)
    w = (0.05 * rng.standard_normal((35 * 256, 1536))).astype(np.float16)
    x = rng.standard_normal(1536).astype(np.float32)
    contract_close(host(D.gemv_f16(dev(x), dev(w))), w.astype(np.float32) @ x, "gemv_f16")


def test_rms_norm_variants():
    rng = np.random.default_rng(4)
    for rows, n in ((1, 1536), (35, 256), (1, 12288), (3, 100)):
        x = (3 * rng.standard_normal((rows, n))).astype(np.float32)
        w = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
        res = rng.standard_normal((rows, n)).astype(np.float32)
        out, out2 = D.rms_norm(dev(x), dev(w), res=dev(res), pre=0.3, mult=0.7, q2=0.05, f16_2=True)
        sum2 = torch.empty(rows, device=DEV)
        D.rms_norm(dev(x), dev(w), out=torch.empty_like(out), q2=0.05, out2=torch.empty_like(out), sum2=sum2)
        ref = (res + OD.rms_norm(x * np.float32(0.3), w)) * np.float32(0.7)
        contract_close(host(out), ref, f"rms {rows}x{n}")
        # the second output from the GPU's own first one: exact
        o = host(out)
        want2 = OD.srq(o.astype(np.float16).astype(np.float32), 0.05).astype(np.float16).astype(np.float32)
        assert np.array_equal(host(out2), want2)
        plain = OD.srq(OD.rms_norm(x, w), 0.05)
        assert np.abs(host(sum2) - plain.sum(-1)).max() <= 0.05 * 3 + 1e-3 * n  # a few .5 flips at most
        # the second norm: out2 = srq(rms(out) * w2, q2), from the GPU's own out
        w2 = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
        out, out2 = D.rms_norm(dev(x), dev(w), res=dev(res), w2=dev(w2), q2=0.05)
        srq_close(host(out2), OD.rms_norm(host(out), w2), 0.05, f"rms second norm {rows}x{n}")
    # in place: out aliases res (the residual adds)
    x = rng.standard_normal(1536).astype(np.float32)
    r = dev(rng.standard_normal(1536).astype(np.float32))
    r0 = host(r)
    D.rms_norm(dev(x), None, res=r, out=r)
    contract_close(host(r), r0 + OD.rms_norm(x), "rms in place")


def test_geglu_and_embed():
    rng = np.random.default_rng(5)
    a = (2 * rng.standard_normal(6144)).astype(np.float32)
    b = rng.standard_normal(6144).astype(np.float32)
    srq_close(host(D.geglu(dev(a), dev(b), 0.01)), OD.gelu_tanh(a) * b, 0.01, "geglu")
    contract_close(host(D.geglu(dev(a), dev(b), 0.0)), OD.gelu_tanh(a) * b, "geglu no srq")
    vocab, H, nL, d = 300, 1536, 35, 256
    emb = rng.integers(0, 256, size=(vocab, H // 4), dtype=np.uint8)
    esc = rng.random(vocab).astype(np.float32)
    ple = rng.integers(0, 256, size=(vocab, nL * d // 2), dtype=np.uint8)
    psc = rng.random(vocab * nL).astype(np.float32)
    for t in (0, 7, vocab - 1):
        tok = torch.tensor([t], dtype=torch.int32, device=DEV)
        got = host(D.embed(dev(emb), tok, dev(esc), H, 2, H, 39.19))
        assert np.array_equal(got, OD.embed_row(emb, t, esc, H, 2, H, 39.19))
        got = host(D.embed(dev(ple), tok, dev(psc), nL * d, 4, d, 16.0))
        assert np.array_equal(got, OD.embed_row(ple, t, psc, nL * d, 4, d, 16.0))
    for t in (-1, vocab, 1 << 30):  # ids outside the table: zeros, no access outside it
        tok = torch.tensor([t], dtype=torch.int32, device=DEV)
        assert not host(D.embed(dev(emb), tok, dev(esc), H, 2, H, 1.0)).any()


def test_softcap_argmax():
    rng = np.random.default_rng(6)
    for n in (1, 1000, 262144):
        z = (5 * rng.standard_normal(n)).astype(np.float32)
        if n > 10:
            z[n // 3] = z[2 * n // 3] = z.max() + 1.0  # a tie: the first index wins
        lg = dev(z)
        tok = D.softcap_argmax(lg, 30.0)
        ref, t = OD.softcap_argmax(z, 30.0)
        contract_close(host(lg), ref, "softcap")
        assert int(host(tok)[0]) == t == int(np.argmax(z))
    lg = dev(np.array([3.0, 9.0, 9.0, -1.0], np.float32))
    assert int(host(D.softcap_argmax(lg, 0.0))[0]) == 1 and host(lg)[1] == 9.0


def _stage_checks(m, L, t, ple_in):
    """Each stage of layer L from the GPU's own inputs to it (trace t of DecoderStack.layer)."""
    s = m.layers[L]
    sc, H, inter, d = s.scales, m.hidden, s.intermediate, int(m.config["ple_d"])
    g = {k: host(v) for k, v in t.items()}
    w = lambda n: m.tensor(f"L{L}.{n}")  # noqa: E731
    o_w12, pl = w("o_w12"), w("pleproj_w12s")
    bits = lambda n, n_out, n_in: OD.bits_of(m, f"L{L}.{n}", n_out, n_in)  # noqa: E731
    what = f"layer {L}"
    srq_close(g["a"], OD.rms_norm(g["x0"], w("in_norm")), sc["qkv_in"], what + " a")
    srq_close(g["o"], OD.qlin(g["attn"], w("o_bits"), w("o_scale"), s.q_dim, bits("o_bits", H, s.q_dim), sc["o_in"]),
              sc["o_out"], what + " o_proj")
    contract_close(g["x1"], g["x0"] + OD.rms_norm(g["o"], o_w12[:H]), what + " x1")
    y2 = OD.srq(OD.rms_norm(g["x1"], o_w12[H:]).astype(np.float16).astype(np.float32), sc["gate_in"])
    assert np.abs(g["y2"] - y2).max() <= sc["gate_in"] * 1.001 and (g["y2"] != y2.astype(np.float16)).mean() < 0.05
    gb = bits("gate_bits", inter, H)
    gate = qlin_codes(g["y2"], w("gate_bits"), w("gate_scale"), H, gb, sc["gate_in"], sc["gate_out"])
    up = qlin_codes(g["y2"], w("up_bits"), w("up_scale"), H, gb, sc["up_in"], sc["up_out"])
    lut_g, lut_p = OD.layer_lut(m, L, "gate"), OD.layer_lut(m, L, "plegate")
    chain_close(g["geglu"], lambda a, b: OD.gelu_of_srq(a, sc["gate_out"], lut_g) * b, [gate, up],
                what + " gate/up/geglu", step=sc["down_in"])
    srq_close(g["down"], OD.qlin(g["geglu"], w("down_bits"), w("down_scale"), inter, bits("down_bits", H, inter),
                                 sc["down_in"]), sc["down_out"], what + " down")
    contract_close(g["x2"], g["x1"] + OD.rms_norm(g["down"], w("down_nw")), what + " x2")
    pgate = qlin_codes(g["x2"], w("plegate_codes"), w("plegate_rowscale"), H, 8, sc["plegate_in"], sc["plegate_out"])
    chain_close(g["pleg"], lambda a: OD.gelu_of_srq(a, sc["plegate_out"], lut_p) * ple_in[L], [pgate],
                what + " plegate")
    srq_close(g["pleproj"], OD.qlin(g["pleg"], w("pleproj_codes"), w("pleproj_rowscale"), d, 8, sc["pleproj_in"]),
              sc["pleproj_out"], what + " pleproj")
    contract_close(g["x3"], (g["x2"] + OD.rms_norm(g["pleproj"], pl[:H])) * pl[2 * H], what + " x3")
    if L + 1 < len(m.layers):
        srq_close(g["a_next"], OD.rms_norm(g["x3"], m.tensor(f"L{L + 1}.in_norm")),
                  m.layers[L + 1].scales["qkv_in"], what + " next input norm")
    else:
        contract_close(g["hf"], OD.rms_norm(g["x3"], m.tensor("final_norm")), what + " final norm")


@pytest.mark.parametrize("H,n_heads,ple_d,vocab,steps", [(256, 4, 32, 512, 3), (1536, 8, 256, 2048, 1)])
def test_decoder_steps_stage_by_stage(tmp_path, H, n_heads, ple_d, vocab, steps):
    """Resident steps of a four-layer model (sliding hd 256 / global hd 512 with partial
    RoPE, two KV-sharing layers, 4- and 2-bit MLPs): each step's token is the previous
    step's argmax, read on the device. The second case has E2B's widths (H 1536, 8 heads,
    intermediate 6144, per-layer inputs 256): the norm prologues at full width, the 128-
    and 256-thread GEMV row groups and the hd-512 o_proj rows."""
    write_model(tmp_path, full=True, seed=11, H=H, n_heads=n_heads, ple_d=ple_d, vocab=vocab)
    m = load_manifest(tmp_path)
    st = D.DecoderStack(m, max_seq=64, device=DEV)
    st.tok.fill_(5)
    prev = 5
    for pos in range(steps):
        trace = []
        st.step(pos, trace=trace)
        torch.cuda.synchronize()
        x = host(trace[0]["x"])
        assert np.array_equal(x, OD.embed_row(m.tensor("embed_q"), prev, m.tensor("embed_scale"), m.hidden, 2,
                                              m.hidden, m.config["embed_scale"]))
        ple_in = host(trace[0]["ple_in"])
        contract_close(ple_in, OD.ple_input(m, prev, x), f"step {pos} ple_in")
        for L in range(len(m.layers)):
            _stage_checks(m, L, trace[L + 1], ple_in)
        logits, t = OD.final_logits(m, host(trace[-1]["x3"]))
        got = host(st.logits)
        contract_close(got, logits, f"step {pos} logits")
        tok = int(host(st.tok)[0])
        assert got[tok] == got.max() and tok == int(np.argmax(got))
        top2 = np.sort(logits)[-2:]
        if top2[1] - top2[0] > 1e-2:
            assert tok == t
        prev = tok


def test_decoder_steps_graph_replays_match_eager(tmp_path):
    """Four resident steps captured as one HIP graph (the token only ever on the device),
    replayed three times with eager work and synchronisation between the replays: every
    replay gives the eager run's tokens and logits bit for bit (no atomics anywhere)."""
    write_model(tmp_path, full=True, seed=12)
    m = load_manifest(tmp_path)
    st = D.DecoderStack(m, max_seq=16, device=DEV)
    steps = 4

    def reset():
        for c in list(st.attn.kc.values()) + list(st.attn.vc.values()):
            c.zero_()
        st.tok.fill_(7)

    def run(rec):
        for p in range(steps):
            st.step(p)
            rec[0][p].copy_(st.tok)
            rec[1][p].copy_(st.logits)

    bufs = lambda: (torch.zeros(steps, 1, dtype=torch.int32, device=DEV),  # noqa: E731
                    torch.zeros(steps, st.vocab, device=DEV))
    eager = bufs()
    reset()
    run(eager)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):  # warm-up on the capture stream (workspaces sized)
        reset()
        run(bufs())
    torch.cuda.synchronize()
    got = bufs()
    g = torch.cuda.CUDAGraph()
    reset()
    torch.cuda.synchronize()
    with torch.cuda.graph(g, stream=s):
        run(got)
    for rep in range(3):
        reset()
        torch.cuda.synchronize()
        got[0].fill_(-1)
        got[1].fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(got[0], eager[0]), f"replay {rep}: tokens differ"
        assert torch.equal(got[1], eager[1]), f"replay {rep}: logits differ"
        _ = (st.x * 2).sum().item()  # eager work between replays
