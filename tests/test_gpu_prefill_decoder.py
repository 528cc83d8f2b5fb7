"""GPU parity of the layers-outer batched prefill of the whole decoder (DecoderStack.prefill;
the reference's PrefillGPU.prefill / _layer, gemma4_150/prefill_gpu.py:316-436) against the
oracle's restatement of its rounding points (oracle/decoder.py gemm16, rmsadd, tail_operand,
geglu_codes, plegate_operand, prefill_inputs) and the attention oracle, stage by stage on the
GPU's own intermediates, for a 512-token prompt through a four-layer model (a sliding hd-256
layer, a global hd-512 layer with partial RoPE, then a KV-sharing layer of each kind; 4- and
2-bit MLPs, int8 per-layer-embedding linears). Then the resident decode continues from the
prompt's caches (runner.py:542-569).

Tolerances: f16 GEMM products within one f16 ulp of the float64 product rounded to f16 plus
the f32 summation bound K * 2^-24 * sum |a_k w_k|; f32
row arithmetic at |d| <= 2e-3 + 1e-2|ref|; srq'd f16 operands equal to the oracle's code or,
for at most 5 % of them (a value on an srq midpoint), one grid step away.
"""
import numpy as np
import pytest
import torch

import oracle.attention as O
import oracle.decoder as OD
import oracle.projection as OP
from helpers import contract_close, f16_ulp_close, srq_close
from manifest_fixture import write_model
from slang_amd import decoder as D
from slang_amd.manifest import load_manifest

pytestmark = pytest.mark.gpu
DEV = "cuda"


def host(t):
    return t.cpu().numpy() if t.dtype in (torch.float16, torch.int32) else t.float().cpu().numpy()


def srq16_close(got16, ref_unq, step, what, frac=0.05):
    """f16(srq(z, step)) operands: each equal to the oracle's f16(srq(z_ref, step)), or one grid
    step away for at most `frac` of them (z on a midpoint, rounded the other way)."""
    got = np.asarray(got16, np.float16).astype(np.float64)
    ref = OD.srq(np.asarray(ref_unq, np.float32), step).astype(np.float16).astype(np.float64)
    d = np.abs(got - ref)
    ulp = np.spacing(np.abs(ref.astype(np.float16))).astype(np.float64)
    assert (d <= step * 1.001 + ulp).all(), f"{what}: a value {d.max() / step:.2f} grid steps off"
    assert (d > ulp).mean() <= frac, f"{what}: {(d > ulp).mean():.2%} of the values one step off"


def gemm_close(got16, a16, w16, what, alpha=1.0):
    """An f16 GEMM product against the oracle's: within one f16 ulp of the float64 product
    rounded to f16, plus the forward error bound of an f32 sum of K terms, K * 2^-24 *
    sum_k |a_k w_k| (a result that nearly cancels has a far smaller ulp than its terms)."""
    a = np.asarray(a16, np.float16).astype(np.float64)
    w = np.asarray(w16, np.float16).astype(np.float64)
    ref = OD.gemm16(a16, w16, alpha).astype(np.float64)
    bound = np.spacing(np.abs(ref.astype(np.float16))).astype(np.float64) + \
        a.shape[1] * 2.0 ** -24 * alpha * (np.abs(a) @ np.abs(w).T)
    d = np.abs(np.asarray(got16, np.float16).astype(np.float64) - ref)
    assert (d <= bound).all(), f"{what}: {int((d > bound).sum())} products beyond the bound, worst {(d / bound).max():.2f}x"


def codes_close(got16, ref16, what, frac=0.05):
    d = np.abs(np.asarray(got16, np.float32) - np.asarray(ref16, np.float32))
    assert d.max() <= 1.0, f"{what}: codes {d.max()} apart"
    assert (d > 0).mean() <= frac, f"{what}: {(d > 0).mean():.2%} of the codes one off"


def rope_rows(m, L, lo, hi):
    hd, theta, cutoff = m.rope_key(L)
    return O.rope_tables(np.arange(lo, hi), hd, theta, cutoff)


def layer_checks(m, st, L, g, prev_x3, ple_gpu, S):
    """Every stage of layer L from the GPU's own inputs to it (trace g of DecoderStack.prefill)."""
    s = m.layers[L]
    sc, H, it, d = s.scales, m.hidden, s.intermediate, int(m.config["ple_d"])
    w = lambda n: m.tensor(f"L{L}.{n}")  # noqa: E731
    bits = lambda n, n_out, n_in: OD.bits_of(m, f"L{L}.{n}", n_out, n_in)  # noqa: E731
    what = f"layer {L}"
    g = {k: host(v) for k, v in g.items() if v is not None}
    in_norm = w("in_norm")
    srq16_close(g["a16"], OD.rms_norm(prev_x3, in_norm), sc["qkv_in"], what + " input operand")
    # q / k / v GEMMs on the manifest's rows
    scales = w("q_scale") if s.shared else w("qkv_scales")
    wq = OP.dequant_f16(w("q_bits"), scales, H, s.q_dim, 4)
    srq_close(g["q"], OD.gemm16(g["a16"], wq).astype(np.float32), sc["q_out"], what + " q")
    if not s.shared:
        kv = m.kv_dim(L)
        wk = OP.dequant_f16(w("k_bits"), scales[s.q_dim:], H, kv, 4)
        wv = OP.dequant_f16(w("v_bits"), scales[s.q_dim + kv:], H, kv, 4)
        gemm_close(g["kraw"], g["a16"], wk, what + " k GEMM")
        gemm_close(g["vraw"], g["a16"], wv, what + " v GEMM")
        cos, sin = rope_rows(m, L, 0, S)
        kvH = m.n_kv_heads(L)
        kref, vref = O.kv_write(g["kraw"].astype(np.float32).reshape(S, kvH, s.head_dim),
                                g["vraw"].astype(np.float32).reshape(S, kvH, s.head_dim), w("k_norm"), cos, sin,
                                k_in_q=sc["k_out"], v_in_q=sc["v_out"])
        kc, vc = st.attn.caches(L)
        f16_ulp_close(host(kc[:S]), kref.astype(np.float32), what + " k cache rows", slack=1e-6)
        f16_ulp_close(host(vc[:S]), vref.astype(np.float32), what + " v cache rows", slack=1e-6)
    # attention over the source layer's caches
    cfg = m.attn_config(L)
    kc, vc = st.attn.caches(L)
    cos, sin = rope_rows(m, L, 0, S)
    ref = O.prefill_attention(g["q"].reshape(S, cfg.n_q_heads, s.head_dim), host(kc).astype(np.float32),
                              host(vc).astype(np.float32), 0, cfg.n_kv_heads, q_gain=w("q_norm"), cos=cos, sin=sin,
                              window=cfg.window)
    srq16_close(g["attn"].reshape(S, cfg.n_q_heads, s.head_dim), ref, sc["o_in"], what + " attention")
    # o_proj, residual add and the pre-FFN norm (rmsadd_b, rmssrqh_b)
    wo = OP.dequant_f16(w("o_bits"), w("o_scale"), s.q_dim, H, bits("o_bits", H, s.q_dim))
    gemm_close(g["o16"], g["attn"], wo, what + " o GEMM")
    o_w12 = w("o_w12")
    contract_close(g["x1"], OD.rmsadd(g["x0"], g["o16"], sc["o_out"], o_w12[:H]), what + " x1")
    z = OD.rms_norm(g["x1"], o_w12[H:]).astype(np.float16).astype(np.float32)
    srq16_close(g["y2"], z, sc["gate_in"], what + " MLP operand")
    # the MLP
    gb = bits("gate_bits", it, H)
    wg = OP.dequant_f16(w("gate_bits"), w("gate_scale"), H, it, gb)
    wu = OP.dequant_f16(w("up_bits"), w("up_scale"), H, it, gb)
    gemm_close(g["g16"], g["y2"], wg, what + " gate GEMM")
    gemm_close(g["u16"], g["y2"], wu, what + " up GEMM")
    codes_close(g["gg16"], OD.geglu_codes(g["g16"], g["u16"], sc["gate_out"], sc["up_out"], sc["down_in"],
                                          lut=OD.layer_lut(m, L, "gate")), what + " geglu codes")
    wd = OP.dequant_f16(w("down_bits"), w("down_scale"), it, H, bits("down_bits", H, it))
    gemm_close(g["d16"], g["gg16"], wd, what + " down GEMM", sc["down_in"])
    contract_close(g["x2"], OD.rmsadd(g["x1"], g["d16"], sc["down_out"], w("down_nw")), what + " x2")
    # the per-layer-embedding block
    srq16_close(g["hh"], g["x2"], sc["plegate_in"], what + " plegate operand")
    wpg = OP.dequant_f16(w("plegate_codes"), w("plegate_rowscale"), H, d, 8)
    gemm_close(g["plin"], g["hh"], wpg, what + " plegate GEMM")
    gate = OD.gelu_of_srq(OD.srq(g["plin"].astype(np.float32), sc["plegate_out"]), sc["plegate_out"],
                          OD.layer_lut(m, L, "plegate")) * ple_gpu[:, L]
    srq16_close(g["gph"], gate, sc["pleproj_in"], what + " pleproj operand")
    wpp = OP.dequant_f16(w("pleproj_codes"), w("pleproj_rowscale"), d, H, 8)
    gemm_close(g["pp16"], g["gph"], wpp, what + " pleproj GEMM")
    pl = w("pleproj_w12s")
    contract_close(g["x3"], OD.rmsadd(g["x2"], g["pp16"], sc["pleproj_out"], pl[:H], pl[2 * H]), what + " x3")
    return g["x3"]


def test_prefill_stage_by_stage_then_decode(tmp_path):
    write_model(tmp_path, full=True, seed=13, H=256, ple_d=128, vocab=512)
    m = load_manifest(tmp_path)
    S, nL, d = 512, len(m.layers), int(m.config["ple_d"])
    toks = np.random.default_rng(14).integers(0, 512, size=S + 1)
    st = D.DecoderStack(m, max_seq=S + 8, device=DEV)
    trace = []
    assert st.prefill(toks[:S], 0, trace=trace) == S
    torch.cuda.synchronize()
    # the prompt's start: token rows, per-layer projection, per-layer inputs
    g0 = {k: host(v) for k, v in trace[0].items()}
    hidden, _, table, _ = OD.prefill_inputs(m, toks[:S])
    np.testing.assert_array_equal(g0["hidden"], hidden)
    np.testing.assert_array_equal(g0["plegath"], table)
    gemm_close(g0["ctx"], g0["hidden"].astype(np.float16), m.tensor("pl_model_proj"), "per-layer projection")
    ple = (OD.rms_norm(g0["ctx"].reshape(S, nL, d) * np.float32(m.hidden ** -0.5), m.tensor("pl_proj_norm"))
           + g0["plegath"].reshape(S, nL, d)) * np.float32(2.0 ** -0.5)
    contract_close(g0["ple"], ple, "per-layer inputs")
    x = g0["hidden"]
    for L in range(nL):
        x = layer_checks(m, st, L, trace[L + 1], x, g0["ple"], S)

    # the resident decode continues at position S from the prompt's caches
    st.tok.fill_(int(toks[S]))
    tr = []
    st.step(S, trace=tr)
    torch.cuda.synchronize()
    for L, s in enumerate(m.layers):
        sc, cfg = s.scales, m.attn_config(L)
        a = host(tr[L + 1]["a"])
        q, _, _ = OP.qkv_gemv(a, float(a.sum()), m.tensor(f"L{L}.q_bits"), None, None,
                              m.tensor(f"L{L}.q_scale" if s.shared else f"L{L}.qkv_scales"), s.q_dim, 0,
                              q_out=sc["q_out"])
        kc, vc = st.attn.caches(L)
        cos, sin = rope_rows(m, L, S, S + 1)
        ref = O.decode_attention(q.reshape(cfg.n_q_heads, s.head_dim), host(kc).astype(np.float32),
                                 host(vc).astype(np.float32), S + 1, cfg.n_kv_heads, q_gain=m.tensor(f"L{L}.q_norm"),
                                 cos=cos[0], sin=sin[0], window=cfg.window)
        srq_close(host(tr[L + 1]["attn"]).reshape(cfg.n_q_heads, s.head_dim), ref, sc["o_in"],
                  f"layer {L} decode after the prefill")


def test_generate_is_prefill_then_resident_steps(tmp_path):
    """generate(ids, n) = prefill(ids[:-1]) then n resident steps from ids[-1]
    (runner.py:542-569), token for token."""
    write_model(tmp_path, full=True, seed=15, H=256, ple_d=128, vocab=512)
    m = load_manifest(tmp_path)
    ids = [int(t) for t in np.random.default_rng(16).integers(0, 512, size=40)]
    st = D.DecoderStack(m, max_seq=64, device=DEV)
    got = host(st.generate(ids, 6))
    st2 = D.DecoderStack(m, max_seq=64, device=DEV)
    pos = st2.prefill(ids[:-1], 0)
    st2.tok.fill_(ids[-1])
    want = []
    for i in range(6):
        st2.step(pos + i)
        want.append(int(host(st2.tok)[0]))
    assert got.tolist() == want
    # the token ids on the device (nothing through the host, as under graph capture)
    st3 = D.DecoderStack(m, max_seq=64, device=DEV)
    dev = torch.tensor(ids, dtype=torch.int32, device=DEV)
    assert host(st3.generate(dev, 6)).tolist() == want


def test_reserved_stack_replays_generate_in_a_graph(tmp_path):
    """DecoderStack.reserve(max_S) sizes and pins every buffer prefill/step use, so a HIP
    graph of a whole generate() call replays to the eager tokens -- several times, with eager
    work between the replays -- without allocating, and a longer prompt afterwards is refused
    instead of silently reallocating the buffers the graph points at."""
    write_model(tmp_path, full=True, seed=15, H=256, ple_d=128, vocab=512)
    m = load_manifest(tmp_path)
    ids = [int(t) for t in np.random.default_rng(16).integers(0, 512, size=40)]
    want = host(D.DecoderStack(m, max_seq=64, device=DEV).generate(ids, 6)).tolist()
    st = D.DecoderStack(m, max_seq=64, device=DEV).reserve(48)
    dev = torch.tensor(ids, dtype=torch.int32, device=DEV)
    assert host(st.generate(dev, 6)).tolist() == want  # eager, on the reserved buffers
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        toks = st.generate(dev, 6)
    torch.cuda.synchronize()
    mem = torch.cuda.memory_allocated()
    for r in range(3):
        toks.fill_(-1)
        st.tok.fill_(-1)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert host(toks).tolist() == want, f"replay {r}"
    assert torch.cuda.memory_allocated() == mem
    with pytest.raises(RuntimeError, match="reserved"):
        st.prefill(list(range(49)), 0)
