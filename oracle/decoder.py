"""CPU oracle for the decode step around the attention block (one token, every layer).

TEST INFRASTRUCTURE ONLY. Nothing in the product package (slang_amd/) imports
this module. It may be imported only by tests/, by __graft_entry__.smoke() and
by bench.py's cpu_baseline leg, and there only as the checker, never as a
fallback for the GPU path.

It restates gemma4_150/reference.py's ReferenceSRQ over the exported model format
(export.py:64-181) instead of the checkpoint:

  * gelu_tanh ........................................ reference.py:34-35
  * gelu_lut / gelu_of_srq: the runners' per-layer GELU table of an srq grid, looked up
    by the grid index ............................... export.py:30-33; kernels_dsl.py:283,
                                                       867, 1292, 1373, 1785
  * rms_norm (x / sqrt(mean(x^2) + eps) * w) .......... reference.py:38-43
  * _qlin: srq(W @ srq(x, in_s), out_s), W = (q - 2^(bits-1)) * row_scale
                                                       reference.py:96-101
  * _ilin_raw: the same with int8 rows; export.py:150-156 stores them biased by 128,
    which is the bits = 8 zero point ............... reference.py:103-111
  * embed (2-bit row * scale[tok] * sqrt(H)) ......... reference.py:114-121
  * ple_table (4-bit row, one scale per layer slice)  reference.py:123-131
  * ple_input ((rms(P x * H^-1/2, w) + ple) / sqrt 2)  reference.py:133-139
  * layer (sandwich norms, MLP with the f16 input rounding of :176-178, PLE block)
                                                       reference.py:141-191
  * forward's tail (final norm, 2-bit lm_head, softcap)  reference.py:193-207
  * lm_head rows from export.py's blocked [24][vocab][4] words  export.py:91-93
  * the layers-outer batched prefill's rounding points (f16 GEMM operands and products, the
    row tails rmsadd_b / rmssrqh_b / rmssrq_69 / srqh_b, geglu_b's codes, plegate_b,
    combine_b) ..................................... prefill_gpu.py:316-436

The attention block itself is oracle.attention's (q/k/v from oracle.projection).
`post_attention` and `ple_block` return every intermediate of a layer after its
attention; the GPU tests check each stage from the GPU's own inputs to that stage with
the primitives above (SRQ grids make a flipped code in one stage legitimately move every
later one).

Pinning (tests/test_oracle_decoder.py): gelu_tanh against the erf form of GELU and its
limits; gelu_lut against the identity gelu(x) - gelu(-x) = x, gelu(0) = 0, a float64 value
of math.tanh per entry and the f32 gelu_tanh of the grid values, and gelu_of_srq's index
(a shifted index is caught); rms_norm against a float64 loop and its scale invariance; qlin against a
pure-Python triple loop over unpacked codes, and against the zero-point closed form;
hand-packed embedding words; the lm_head block order against a row-major re-pack;
argmax ties. The batched prefill's stages: gemm16 against a float64 triple loop (with alpha,
and a transposed operand caught), rmsadd's closed forms (a constant row normalises to its
sign, a zero row adds nothing), a known answer where rmssrqh_b's double rounding and a single
rounding land on different srq codes, geglu_b's codes and clamp, and prefill_inputs against
the decode step's token row (exact) and per-layer inputs.
"""
from __future__ import annotations

import numpy as np

from .attention import srq
from .projection import unpack_values

EPS = 1e-6


def gelu_tanh(v):
    """reference.py:34-35."""
    v = np.asarray(v, np.float32)
    return (0.5 * v * (1.0 + np.tanh(np.float32(0.7978845608028654) * (v + np.float32(0.044715) * v ** 3)))
            ).astype(np.float32)


def gelu_lut(out_scale):
    """The runners' GELU table of one srq grid (export.py:30-33, written per layer for the gate
    and the per-layer-embedding gate, :150, :161): entry k + 128 is the tanh-form GELU of the
    grid value k * out_scale (k in [-128, 127]) evaluated in float64, then cast to f32."""
    g = (np.arange(256) - 128).astype(np.float64) * float(out_scale)
    return (0.5 * g * (1.0 + np.tanh(0.7978845608028654 * (g + 0.044715 * g ** 3)))).astype(np.float32)


def gelu_of_srq(v, s, lut=None):
    """GELU of values v already on the srq grid of step s, as the runner kernels form it
    (geglu_b kernels_dsl.py:283, plegate_76 :867, gateup_74/95 :1292/:1373, plegate_b :1785):
    lut[clamp(round(v / s), -128, 127) + 128] from the layer's table when there is one and
    s > 0, else gelu_tanh(v) in f32 (reference.py:34-35, and the runners when s is 0)."""
    if lut is None or s == 0.0:
        return gelu_tanh(v)
    k = np.clip(np.round(np.asarray(v, np.float32) / np.float32(s)), -128, 127).astype(np.int64)
    return np.asarray(lut, np.float32)[k + 128]


def layer_lut(man, L, which):
    """Layer L's exported table L{L}.gelu_gate / L{L}.gelu_plegate, or None when the model
    carries none (then GELU is reference.py's f32 gelu_tanh)."""
    name = f"L{L}.gelu_{which}"
    return man.tensor(name) if name in man.tensors else None


def rms_norm(x, w=None, eps=EPS):
    """reference.py:38-43 (w None: rms_norm_noscale); rows over the last axis."""
    x = np.asarray(x, np.float32)
    y = x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + np.float32(eps))
    return (y * w if w is not None else y).astype(np.float32)


def dequant_rows(words, scale, n_in, bits):
    """W [n_out][n_in] f32 = (q - 2^(bits-1)) * scale[o] (reference.py:99-100)."""
    codes = unpack_values(words, n_in, bits).astype(np.float32)
    return (codes - np.float32(1 << (bits - 1))) * np.asarray(scale, np.float32)[:, None]


def qlin(x, words, scale, n_in, bits, in_q=0.0, out_q=0.0):
    """reference.py:96-101 (_qlin) and :103-111 (_ilin_raw, bits 8 over biased codes)."""
    W = dequant_rows(words, scale, n_in, bits)
    return srq(W @ srq(np.asarray(x, np.float32), in_q), out_q).astype(np.float32)


def embed_row(table_u8, tok, scale, n, bits, group, mult):
    """reference.py:114-131: row tok of a packed u8 table -> mult * scale * (code - zp)."""
    row = np.ascontiguousarray(table_u8[tok]).view(np.uint32)
    codes = unpack_values(row.reshape(1, -1), n, bits)[0].astype(np.int64)
    sc = np.asarray(scale, np.float32).reshape(-1)[tok * (n // group) + np.arange(n) // group]
    return (np.float32(mult) * sc * (codes - (1 << (bits - 1))).astype(np.float32)).astype(np.float32)


def lmhead_rows(blk_words):
    """export.py:91-93 stores lm_head as [24][vocab][4] words; rows are [vocab][96]."""
    blk = np.asarray(blk_words, np.uint32)
    nb, vocab, four = blk.shape
    return np.ascontiguousarray(blk.transpose(1, 0, 2)).reshape(vocab, nb * four)


def softcap_argmax(logits, cap):
    """reference.py:207 softcap, then numpy's argmax (the first maximum)."""
    z = np.asarray(logits, np.float32)
    if cap:
        z = (np.float32(cap) * np.tanh(z / np.float32(cap))).astype(np.float32)
    return z, int(np.argmax(z))


def ple_input(man, tok, x):
    """reference.py:123-139 for token tok and its embedding x."""
    c = man.config
    H, nL, d = int(c["H"]), int(c["nL"]), int(c["ple_d"])
    ple = embed_row(man.tensor("ple_q"), tok, man.tensor("ple_scale"), nL * d, 4, d,
                    float(c["ple_scale"])).reshape(nL, d)
    proj = man.tensor("pl_model_proj").astype(np.float32) @ x
    ctx = proj.reshape(nL, d) * np.float32(H ** -0.5)
    ctx = rms_norm(ctx, man.tensor("pl_proj_norm"))
    return ((ctx + ple) * np.float32(2.0 ** -0.5)).astype(np.float32)


def bits_of(man, name, n_out, n_in):
    """Bit width of a packed [n_out][n_in] matrix from its word count (export.py:59-61)."""
    return 8 * int(man.tensors[name]["len"]) // (n_out * n_in)


def post_attention(man, L, x, attn):
    """The rest of layer L after its attention output attn (srq'd by o_in), stage by stage
    (reference.py:167-191). Returns a dict of every intermediate, each from its inputs."""
    s = man.layers[L]
    sc, H, inter = s.scales, man.hidden, s.intermediate
    t = lambda n: man.tensor(f"L{L}.{n}")  # noqa: E731
    o_w12, pl = t("o_w12"), t("pleproj_w12s")
    st = {}
    st["o"] = qlin(attn, t("o_bits"), t("o_scale"), s.q_dim, bits_of(man, f"L{L}.o_bits", H, s.q_dim),
                   sc["o_in"], sc["o_out"])
    st["x1"] = (x + rms_norm(st["o"], o_w12[:H])).astype(np.float32)
    h = rms_norm(st["x1"], o_w12[H:])
    st["y2"] = srq(h.astype(np.float16).astype(np.float32), sc["gate_in"]).astype(np.float16).astype(np.float32)
    gb = bits_of(man, f"L{L}.gate_bits", inter, H)
    st["gate"] = qlin(st["y2"], t("gate_bits"), t("gate_scale"), H, gb, sc["gate_in"], sc["gate_out"])
    st["up"] = qlin(st["y2"], t("up_bits"), t("up_scale"), H, gb, sc["up_in"], sc["up_out"])
    st["geglu"] = srq(gelu_of_srq(st["gate"], sc["gate_out"], layer_lut(man, L, "gate")) * st["up"],
                      sc["down_in"]).astype(np.float32)
    st["down"] = qlin(st["geglu"], t("down_bits"), t("down_scale"), inter,
                      bits_of(man, f"L{L}.down_bits", H, inter), sc["down_in"], sc["down_out"])
    st["x2"] = (st["x1"] + rms_norm(st["down"], t("down_nw"))).astype(np.float32)
    return st


def ple_block(man, L, x2, ple_in_L, gate_out=None, g=None, proj=None):
    """reference.py:185-191; each stage from the given previous stage when supplied."""
    s = man.layers[L]
    sc, H = s.scales, man.hidden
    d = int(man.config["ple_d"])
    t = lambda n: man.tensor(f"L{L}.{n}")  # noqa: E731
    pl = t("pleproj_w12s")
    st = {}
    st["plegate"] = qlin(x2, t("plegate_codes"), t("plegate_rowscale"), H, 8, sc["plegate_in"], sc["plegate_out"])
    st["pleg"] = (gelu_of_srq(st["plegate"] if gate_out is None else gate_out, sc["plegate_out"],
                              layer_lut(man, L, "plegate")) * ple_in_L).astype(np.float32)
    st["pleproj"] = qlin(st["pleg"] if g is None else g, t("pleproj_codes"), t("pleproj_rowscale"), d, 8,
                         sc["pleproj_in"], sc["pleproj_out"])
    st["x3"] = ((x2 + rms_norm(st["pleproj"] if proj is None else proj, pl[:H])) * pl[2 * H]).astype(np.float32)
    return st


def final_logits(man, x):
    """reference.py:200-207 (norm, 2-bit lm_head over the exported blocks, softcap)."""
    c = man.config
    H = man.hidden
    xn = rms_norm(x, man.tensor("final_norm"))
    rows = lmhead_rows(man.tensor("lmhead_blk"))
    W = dequant_rows(rows, man.tensor("lmhead_scale"), H, 2)
    return softcap_argmax(W @ xn, float(c["softcap"]))


# --------------------------------------------------------------------------
# the layers-outer batched prefill (prefill_gpu.py:316-436)
# --------------------------------------------------------------------------
# The same layer with the GPU runner's rounding points: every linear one f16 GEMM over the
# S rows (weights dq_f16'd, activations f16(srq(..)), products f16), the tails between them
# per row. `prefill_inputs` is the prompt's start (:412-431); the rest are the stages of
# _layer (:356-395), each from the previous stage's value so a test can feed the GPU's own.
def gemm16(a16, w16, alpha=1.0):
    """gemm_tiled (kernels_dsl.py:34-136, tr = 1): f16(alpha * (a16 . w16^T)); the product of the
    f16 operands accumulated in float64 (f32 on the GPU), scaled in f32 and rounded to f16."""
    c = np.asarray(a16, np.float16).astype(np.float64) @ np.asarray(w16, np.float16).astype(np.float64).T
    return (np.float32(alpha) * c.astype(np.float32)).astype(np.float16)


def rmsadd(hidden, x16, x_q, w1, mult=1.0):
    """rmsadd_b (kernels_dsl.py:622-657): hidden + rms(srq(f32(x16), x_q)) * w1, times mult."""
    d = srq(np.asarray(x16, np.float16).astype(np.float32), x_q)
    return ((np.asarray(hidden, np.float32) + rms_norm(d, w1)) * np.float32(mult)).astype(np.float32)


def tail_operand(hidden, mode, w2=None, q2=0.0):
    """The next GEMM's f16 operand from updated rows: "srq" = srqh_b (kernels_dsl.py:233-242),
    "norm" = rmssrq_69 then srqh_b (:158-206), "norm16" = rmssrqh_b's f16(srq(f32(f16(n)), q2))
    (:660-710: the normed value is narrowed to f16 before the srq as well as after)."""
    h = np.asarray(hidden, np.float32)
    z = h if mode == "srq" else rms_norm(h, w2)
    if mode == "norm16":
        z = z.astype(np.float16).astype(np.float32)
    return srq(z, q2).astype(np.float16)


def geglu_codes(g16, u16, gate_q, up_q, out_q, lut=None):
    """geglu_b (kernels_dsl.py:259-290): y = gelu(srq(f32(gate), gate_q)) * srq(f32(up), up_q),
    stored as its code on out_q's grid, f16(clamp(round(y / out_q), -128, 127)) (f16(y) when
    out_q is 0); the down GEMM scales it back with alpha = out_q (prefill_gpu.py:376-377).
    lut: the layer's GELU table (gelu_of_srq)."""
    y = (gelu_of_srq(srq(np.asarray(g16, np.float16).astype(np.float32), gate_q), gate_q, lut)
         * srq(np.asarray(u16, np.float16).astype(np.float32), up_q)).astype(np.float32)
    if out_q == 0.0:
        return y.astype(np.float16)
    return np.clip(np.round(y / np.float32(out_q)), -128.0, 127.0).astype(np.float16)


def plegate_operand(lin16, lin_q, ple_L, out_q, lut=None):
    """plegate_b then srqh_b (kernels_dsl.py:1767-1786, 233-242; prefill_gpu.py:381-384):
    f16(srq(gelu(srq(f32(lin), lin_q)) * ple, out_q)), ple the layer's per-layer inputs [S][d];
    lut: the layer's GELU table (gelu_of_srq)."""
    g = gelu_of_srq(srq(np.asarray(lin16, np.float16).astype(np.float32), lin_q), lin_q, lut)
    return srq((g * np.asarray(ple_L, np.float32)).astype(np.float32), out_q).astype(np.float16)


def prefill_inputs(man, toks):
    """The prompt's start (prefill_gpu.py:412-431): token rows (embed_00), the per-layer
    model projection as one GEMM over f16(h) with an f16 product (srqh_b, _gemm, srq_b with
    step 0), the per-layer table rows (plegather_01) and combine_b's
    ple = (rms(ctx * H^-1/2, pl_proj_norm) + table) / sqrt 2. Returns (hidden [S][H],
    ctx [S][nL*d], table [S][nL*d], ple [S][nL][d])."""
    c = man.config
    H, nL, d = int(c["H"]), int(c["nL"]), int(c["ple_d"])
    toks = [int(t) for t in toks]
    hidden = np.stack([embed_row(man.tensor("embed_q"), t, man.tensor("embed_scale"), H, 2, H,
                                 float(c["embed_scale"])) for t in toks])
    ctx = gemm16(hidden.astype(np.float16), man.tensor("pl_model_proj")).astype(np.float32)
    table = np.stack([embed_row(man.tensor("ple_q"), t, man.tensor("ple_scale"), nL * d, 4, d,
                                float(c["ple_scale"])) for t in toks])
    ple = ((rms_norm(ctx.reshape(-1, nL, d) * np.float32(H ** -0.5), man.tensor("pl_proj_norm"))
            + table.reshape(-1, nL, d)) * np.float32(2.0 ** -0.5)).astype(np.float32)
    return hidden, ctx, table, ple
