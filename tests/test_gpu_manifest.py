"""The attention block driven by an exported model's layer schedule (slang_amd.manifest.
AttentionStack) against the CPU oracle, stage by stage on the GPU's own intermediates:
q/k/v projections from the manifest's packed rows, the KV-cache rows each non-shared
layer writes (k RMSNorm + RoPE with the layer's partial cutoff, v norm), and attention
over the right cache (KV-sharing layers read their kv_source's), window and output srq
(o_in). Schedule: a sliding hd-256 layer, a global hd-512 layer with RoPE on 64 of 256
pairs, then a KV-sharing layer of each kind; a prefill of S tokens, then decode steps
(runner.py:373-441, prefill_gpu.py:327-354)."""
import numpy as np
import pytest
import torch

import oracle.attention as O
import oracle.projection as OP
import slang_amd as sa
import slang_amd.projection as P
from helpers import contract_close, srq_close
from manifest_fixture import write_model
from slang_amd.manifest import AttentionStack, load_manifest

pytestmark = pytest.mark.gpu
DEV = "cuda"


def host(t):
    return t.float().cpu().numpy() if t.dtype != torch.float16 else t.cpu().numpy()


def rope_rows(m, L, lo, hi):
    hd, theta, cutoff = m.rope_key(L)
    return O.rope_tables(np.arange(lo, hi), hd, theta, cutoff)


def check_cache_rows(st, m, L, lo, hi, k_in, v_in, k_in_q, v_in_q, what):
    """Cache rows [lo, hi) of layer L against the oracle's kv_write of the GPU's k/v."""
    s = m.layers[L]
    kvH, hd = m.n_kv_heads(L), s.head_dim
    cos, sin = rope_rows(m, L, lo, hi)
    kref, vref = O.kv_write(k_in.reshape(hi - lo, kvH, hd), v_in.reshape(hi - lo, kvH, hd),
                            m.tensor(f"L{L}.k_norm"), cos, sin, k_in_q=k_in_q, v_in_q=v_in_q,
                            cache_dtype=np.float32)
    kc, vc = st.caches(L)
    contract_close(host(kc[lo:hi]), kref, f"{what} k rows")
    contract_close(host(vc[lo:hi]), vref, f"{what} v rows")


def test_stack_prefill_then_decode(tmp_path):
    write_model(tmp_path, seed=3)
    m = load_manifest(tmp_path)
    H, S, steps = m.hidden, 96, 3
    st = AttentionStack(m, max_seq=S + steps, device=DEV)
    rng = np.random.default_rng(5)

    # ---- prefill: every layer in schedule order (shared layers after their source)
    for L, s in enumerate(m.layers):
        sc, cfg = s.scales, m.attn_config(L)
        a = OP.srq(rng.standard_normal((S, H)).astype(np.float32), sc["qkv_in"])
        at = torch.from_numpy(a).to(DEV)
        out = torch.empty(S, cfg.n_q_heads, s.head_dim, device=DEV)  # f32: srq grid checkable
        st.prefill_layer(L, 0, at, out=out)
        wq, wk, wv = st._dequant(L)
        q, kraw, vraw = P.prefill_qkv(at, wq, wk, wv, a_in_q=sc["qkv_in"], q_out=sc["q_out"])
        torch.cuda.synchronize()
        # projections from the manifest's packed rows
        scales = m.tensor(f"L{L}.q_scale" if s.shared else f"L{L}.qkv_scales")
        wq_ref = OP.dequant_f16(m.tensor(f"L{L}.q_bits"), scales, H, s.q_dim, 4)
        np.testing.assert_array_equal(host(wq), wq_ref)
        q_ref = OP.proj_gemm(a, wq_ref, sc["qkv_in"], out_f32=True, out_q=sc["q_out"])
        assert (np.abs(host(q) - q_ref) <= sc["q_out"] * 1.001).all()
        if not s.shared:
            kv = m.kv_dim(L)
            wk_ref = OP.dequant_f16(m.tensor(f"L{L}.k_bits"), scales[s.q_dim:], H, kv, 4)
            np.testing.assert_array_equal(host(wk), wk_ref)
            check_cache_rows(st, m, L, 0, S, host(kraw).astype(np.float32), host(vraw).astype(np.float32),
                             sc["k_out"], sc["v_out"], f"layer {L} prefill")
        # attention over the source layer's caches, on the kernel's own f16 q
        cos, sin = rope_rows(m, L, 0, S)
        qh = q.view(S, cfg.n_q_heads, s.head_dim)
        q16 = sa.qprep(qh, cfg, q_gain=st.w[L]["q_norm"], rope_cos=torch.from_numpy(cos).to(DEV),
                       rope_sin=torch.from_numpy(sin).to(DEV))
        kc, vc = st.caches(L)
        ref = O.prefill_attention(host(q16).astype(np.float32), host(kc), host(vc), 0, cfg.n_kv_heads,
                                  window=cfg.window)
        srq_close(host(out), ref, sc["o_in"], f"layer {L} prefill attention")

    # ---- decode steps
    for t in range(steps):
        pos = S + t
        for L, s in enumerate(m.layers):
            sc, cfg = s.scales, m.attn_config(L)
            a = OP.srq(rng.standard_normal(H).astype(np.float32), sc["qkv_in"])
            at = torch.from_numpy(a).to(DEV)
            sum_a = at.sum().reshape(1)
            out = st.decode_layer(L, pos, at, sum_a)
            w = st.w[L]
            kv = 0 if s.shared else m.kv_dim(L)
            q, k, v = P.qkv_gemv(at, sum_a, w["q_bits"], w["scales"], s.q_dim, kv, k_bits=w.get("k_bits"),
                                 v_bits=w.get("v_bits"), q_out=sc["q_out"], k_out=sc.get("k_out", 0.0),
                                 v_out=sc.get("v_out", 0.0))
            torch.cuda.synchronize()
            q_ref, _, _ = OP.qkv_gemv(a, float(host(sum_a)[0]), m.tensor(f"L{L}.q_bits"), None, None,
                                      host(w["scales"]), s.q_dim, 0, q_out=sc["q_out"])
            assert (np.abs(host(q) - q_ref) <= sc["q_out"] * 1.001).all()
            if not s.shared:
                check_cache_rows(st, m, L, pos, pos + 1, host(k), host(v), 0.0, 0.0, f"layer {L} step {t}")
            cos, sin = rope_rows(m, L, pos, pos + 1)
            kc, vc = st.caches(L)
            ref = O.decode_attention(host(q).reshape(cfg.n_q_heads, s.head_dim), host(kc), host(vc), pos + 1,
                                     cfg.n_kv_heads, q_gain=m.tensor(f"L{L}.q_norm"), cos=cos[0], sin=sin[0],
                                     window=cfg.window)
            srq_close(host(out), ref, sc["o_in"], f"layer {L} decode step {t}")


def test_shared_layers_write_no_cache(tmp_path):
    """Only the non-shared layers own caches; a shared layer's decode leaves them as they were."""
    write_model(tmp_path, seed=4)
    m = load_manifest(tmp_path)
    st = AttentionStack(m, max_seq=8, device=DEV)
    assert sorted(st.kc) == [0, 1]
    before = [st.kc[0].clone(), st.vc[0].clone()]
    a = torch.randn(m.hidden, device=DEV)
    st.decode_layer(2, 0, a, a.sum().reshape(1))
    torch.cuda.synchronize()
    assert torch.equal(st.kc[0], before[0]) and torch.equal(st.vc[0], before[1])
    with pytest.raises(ValueError):
        st.decode_layer(0, 8, a, a.sum().reshape(1))
