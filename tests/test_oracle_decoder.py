"""Pins of oracle/decoder.py (the decode step around attention) against what does not
restate it: the erf form of GELU, float64 loops, hand-packed words, closed forms."""
import math
import sys

import numpy as np

import oracle.decoder as OD
from oracle.projection import pack_values, unpack_values

sys.path.insert(0, __file__.rsplit("/", 1)[0])
from manifest_fixture import write_model  # noqa: E402


def test_gelu_tanh_against_erf_gelu_and_limits():
    v = np.linspace(-6, 6, 2001, dtype=np.float32)
    exact = np.array([0.5 * x * (1 + math.erf(x / math.sqrt(2))) for x in v.astype(np.float64)])
    assert np.abs(OD.gelu_tanh(v) - exact).max() < 1e-3       # the tanh form's known accuracy
    assert OD.gelu_tanh(np.float32(0.0)) == 0.0
    assert abs(OD.gelu_tanh(np.float32(10.0)) - 10.0) < 1e-5 and abs(OD.gelu_tanh(np.float32(-10.0))) < 1e-5
    assert OD.gelu_tanh(np.float32(1.0)) > 0.84 and OD.gelu_tanh(np.float32(-1.0)) < -0.15  # odd part


def test_gelu_lut_is_the_exporters_float64_table():
    """gelu_lut (export.py:30-33): every entry the float64 tanh-form GELU of the grid value
    k * s cast to f32 -- checked entry by entry with math.tanh, by the exact identity
    gelu(x) - gelu(-x) = x and gelu(0) = 0 of the float64 values, and within a few f32 ulps of
    reference.py's f32 gelu_tanh of the same grid values, over scales the runners use."""
    for s in (0.0017, 0.02, 0.0534, 0.25, 1.0 / 3):
        lut = OD.gelu_lut(s)
        assert lut.dtype == np.float32 and lut.shape == (256,) and lut[128] == 0.0
        for k in (-128, -77, -1, 1, 5, 64, 127):
            x = k * s
            want = np.float32(0.5 * x * (1.0 + math.tanh(0.7978845608028654 * (x + 0.044715 * x ** 3))))
            assert lut[k + 128] == want, (s, k)
        x = (np.arange(1, 128) * s).astype(np.float64)
        odd = lut[128 + np.arange(1, 128)].astype(np.float64) - lut[128 - np.arange(1, 128)].astype(np.float64)
        assert np.abs(odd - x).max() <= 4 * np.spacing(np.float32(x.max()))  # two f32 roundings
        grid = ((np.arange(256) - 128) * np.float32(s)).astype(np.float32)
        f32 = OD.gelu_tanh(grid)
        assert np.abs(f32 - lut).max() <= 8 * np.spacing(np.abs(lut).max())


def test_gelu_of_srq_indexes_the_grid():
    """gelu_of_srq looks up values already on the grid by their code (kernels_dsl.py:283);
    without a table, or on a zero step, it is gelu_tanh. An index shifted by one is caught."""
    s = np.float32(0.05)
    lut = OD.gelu_lut(s)
    k = np.arange(-128, 128)
    v = OD.srq((k * s).astype(np.float32), s)
    np.testing.assert_array_equal(OD.gelu_of_srq(v, s, lut), lut)
    assert OD.gelu_of_srq(np.float32(400.0), s, lut) == lut[255]   # clamped like srq
    np.testing.assert_array_equal(OD.gelu_of_srq(v, s, None), OD.gelu_tanh(v))
    np.testing.assert_array_equal(OD.gelu_of_srq(v, 0.0, lut), OD.gelu_tanh(v))
    shifted = np.asarray(lut)[np.clip(k + 129, 0, 255)]
    assert np.abs(shifted - OD.gelu_of_srq(v, s, lut)).max() > 10 * np.spacing(np.float32(1.0))


def test_rms_norm_against_float64_loop_and_invariants():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((3, 40)).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(40)).astype(np.float32)
    ref = np.empty_like(x, dtype=np.float64)
    for r in range(3):
        ms = sum(float(t) * float(t) for t in x[r]) / 40
        ref[r] = [float(t) / math.sqrt(ms + 1e-6) * float(g) for t, g in zip(x[r], w)]
    assert np.abs(OD.rms_norm(x, w) - ref).max() < 1e-5
    y = OD.rms_norm(x)
    assert np.allclose((y * y).mean(-1), 1.0, atol=1e-4)           # unit RMS
    assert np.allclose(OD.rms_norm(7.5 * x), y, atol=1e-5)         # scale invariance


def test_qlin_against_python_loop_all_widths():
    rng = np.random.default_rng(1)
    for bits in (2, 4, 8):
        n_in, n_out = 128 // bits * 2, 5
        codes = rng.integers(0, 1 << bits, size=(n_out, n_in))
        words = pack_values(codes, bits)
        scale = (0.01 * (1 + rng.random(n_out))).astype(np.float32)
        x = rng.standard_normal(n_in).astype(np.float32)
        in_q, out_q = 0.05, 0.02
        got = OD.qlin(x, words, scale, n_in, bits, in_q, out_q)
        zp = 1 << (bits - 1)
        xq = [min(max(round(float(np.float32(t) / np.float32(in_q))), -128), 127) * in_q for t in x]
        for o in range(n_out):
            acc = sum((int(codes[o][i]) - zp) * float(scale[o]) * xq[i] for i in range(n_in))
            want = min(max(round(acc / out_q), -128), 127) * out_q
            assert abs(got[o] - want) <= out_q * 1.001, (bits, o)   # a .5 tie may round either way
    # closed form: every value at the zero point gives 0 whatever the input
    words = pack_values(np.full((3, 64), 8), 4)
    assert not OD.qlin(rng.standard_normal(64).astype(np.float32), words, np.ones(3, np.float32), 64, 4).any()


def test_embed_row_hand_packed_words():
    # 2-bit row of 16 values 0,1,2,3,0,1,... in one word: value j at bits 2j
    word = sum((j % 4) << (2 * j) for j in range(16))
    table = np.frombuffer(np.array([[0] * 1, [word]], np.uint32).tobytes(), np.uint8).reshape(2, 4)
    got = OD.embed_row(table, 1, np.array([0.5, 2.0], np.float32), 16, 2, 16, 3.0)
    assert np.array_equal(got, 3.0 * 2.0 * (np.arange(16) % 4 - 2).astype(np.float32))
    # 4-bit, two slices of 8 values with their own scales
    word4 = [sum(((j + 8 * s) % 16) << (4 * j) for j in range(8)) for s in range(2)]
    table = np.frombuffer(np.array(word4, np.uint32).tobytes(), np.uint8).reshape(1, 8)
    got = OD.embed_row(table, 0, np.array([1.0, 0.25], np.float32), 16, 4, 8, 2.0)
    want = 2.0 * np.repeat([1.0, 0.25], 8) * (np.arange(16) % 16 - 8)
    assert np.array_equal(got, want.astype(np.float32))


def test_lmhead_block_order_and_argmax_ties():
    rng = np.random.default_rng(2)
    rows = pack_values(rng.integers(0, 4, size=(7, 128)), 2)            # [7][8] words
    blk = rows.reshape(7, 2, 4).transpose(1, 0, 2).copy()                 # export.py:91-93
    assert np.array_equal(OD.lmhead_rows(blk), rows)
    z, t = OD.softcap_argmax(np.array([1.0, 5.0, -2.0, 5.0], np.float32), 30.0)
    assert t == 1 and np.allclose(z, 30 * np.tanh(np.array([1, 5, -2, 5]) / 30))
    assert OD.softcap_argmax(np.array([0.0, 0.0], np.float32), 0.0)[1] == 0


def test_stage_functions_compose_to_reference_layer(tmp_path):
    """post_attention + ple_block == the reference layer's formula written out at once."""
    from slang_amd.manifest import load_manifest
    write_model(tmp_path, full=True, seed=4)
    m = load_manifest(tmp_path)
    rng = np.random.default_rng(3)
    H, L = m.hidden, 1
    s = m.layers[L]
    x = rng.standard_normal(H).astype(np.float32)
    attn = OD.srq(rng.standard_normal(s.q_dim).astype(np.float32), s.scales["o_in"])
    ple_in = rng.standard_normal(m.config["ple_d"]).astype(np.float32)
    st = OD.post_attention(m, L, x, attn)
    pb = OD.ple_block(m, L, st["x2"], ple_in)
    t = lambda n: m.tensor(f"L{L}.{n}")  # noqa: E731
    sc = s.scales
    W = lambda n, sname, n_in, bits: ((OD.unpack_values(t(n), n_in, bits) - (1 << (bits - 1)))  # noqa: E731
                                      * t(sname)[:, None].astype(np.float64))
    q = lambda v, step: np.clip(np.round(v / step), -128, 127) * step  # noqa: E731
    o = q(W("o_bits", "o_scale", s.q_dim, 4) @ q(attn, sc["o_in"]), sc["o_out"])
    assert np.abs(o - st["o"]).max() <= sc["o_out"] * 1.001
    assert s.intermediate == 4 * H and OD.bits_of(m, f"L{L}.gate_bits", 4 * H, H) == 2
    assert abs(pb["x3"] - (st["x2"] + OD.rms_norm(pb["pleproj"], t("pleproj_w12s")[:H])) * t("pleproj_w12s")[2 * H]
               ).max() < 1e-5


# ---------------------------------------------------------------- the batched prefill's stages
def test_prefill_gemm16_against_a_loop_and_alpha():
    """gemm_tiled's f16(alpha * A . W^T) against a pure-Python float64 loop on a tiny case."""
    rng = np.random.default_rng(21)
    a = rng.standard_normal((3, 5)).astype(np.float16)
    w = rng.standard_normal((4, 5)).astype(np.float16)
    for alpha in (1.0, 0.01):
        ref = np.empty((3, 4), np.float16)
        for m in range(3):
            for n in range(4):
                acc = sum(float(a[m, k]) * float(w[n, k]) for k in range(5))
                ref[m, n] = np.float16(np.float32(alpha) * np.float32(acc))
        np.testing.assert_array_equal(OD.gemm16(a, w, alpha), ref)
    # a transposed operand (A . W instead of A . W^T) is caught
    sq = rng.standard_normal((4, 4)).astype(np.float16)
    assert not np.array_equal(OD.gemm16(sq, sq.T.copy()), OD.gemm16(sq, sq))


def test_prefill_row_tails_closed_forms():
    """rmsadd_b: a constant row normalises to its sign times w1; a zero row adds nothing. The
    tail operands: srq grid codes; rmssrqh_b's double rounding differs from one rounding
    exactly where the f16 narrowing crosses an srq midpoint (kernels_dsl.py:667-671)."""
    H = 8
    hid = np.arange(H, dtype=np.float32)
    w1 = np.linspace(0.5, 1.5, H).astype(np.float32)
    x = np.full(H, -3.0, np.float16)
    np.testing.assert_allclose(OD.rmsadd(hid, x, 0.0, w1, 2.0), (hid - w1) * 2, rtol=1e-6)
    np.testing.assert_array_equal(OD.rmsadd(hid, np.zeros(H, np.float16), 0.0, w1), hid)
    # srq mode: codes of hidden on q2's grid
    h = np.array([[0.014, 0.016, -0.5, 2.0]], np.float32)
    np.testing.assert_array_equal(OD.tail_operand(h, "srq", q2=0.01), np.array([[0.01, 0.02, -0.5, 1.27]], np.float16))
    # norm vs norm16: z = 0.0150001 on a 0.01 grid: f16(z) = 0.0149994 rounds down, z itself up
    z = np.float32(0.0150001)
    w2 = np.full(4, z, np.float32)
    ones = np.ones((1, 4), np.float32)            # rms(ones) = 1, so the normed value is w2
    assert float(OD.tail_operand(ones, "norm", w2, 0.01)[0, 0]) == np.float16(0.02)
    assert float(OD.tail_operand(ones, "norm16", w2, 0.01)[0, 0]) == np.float16(0.01)


def test_geglu_codes_and_plegate_operand():
    """geglu_b stores the code of y on out_q's grid (gelu(0) = 0 gives code 0; y at k * out_q
    gives k; codes clamp to [-128, 127]); plegate_b + srqh_b is srq(gelu(srq(lin)) * ple)."""
    g = np.array([0.0, 0.5, 0.25, 40.0], np.float16)
    u = np.array([5.0, 1.0, 2.0, 1.0], np.float16)
    y = OD.gelu_tanh(g.astype(np.float32)) * u.astype(np.float32)
    codes = OD.geglu_codes(g, u, 0.0, 0.0, 0.01)
    assert codes[0] == 0 and codes[3] == 127
    np.testing.assert_array_equal(codes[1:3], np.round(y[1:3] / np.float32(0.01)).astype(np.float16))
    np.testing.assert_array_equal(OD.geglu_codes(g, u, 0.0, 0.0, 0.0), y.astype(np.float16))
    lin = np.array([[0.031, -0.2]], np.float16)
    ple = np.array([[2.0, -1.0]], np.float32)
    ref = OD.srq(OD.gelu_tanh(OD.srq(lin.astype(np.float32), 0.03)) * ple, 0.05).astype(np.float16)
    np.testing.assert_array_equal(OD.plegate_operand(lin, 0.03, ple, 0.05), ref)


def test_prefill_inputs_match_the_decode_step_inputs(tmp_path):
    """The batched start (embed_00, the per-layer projection as an f16 GEMM, combine_b) gives the
    decode step's token row exactly and its per-layer inputs (reference.py:133-139) up to the
    f16 rounding of the projection's operands and product."""
    from slang_amd.manifest import load_manifest
    write_model(tmp_path, full=True, seed=2, H=256, ple_d=128, vocab=64)
    m = load_manifest(tmp_path)
    toks = [3, 17, 63]
    hidden, ctx, table, ple = OD.prefill_inputs(m, toks)
    for i, t in enumerate(toks):
        x = OD.embed_row(m.tensor("embed_q"), t, m.tensor("embed_scale"), m.hidden, 2, m.hidden,
                         float(m.config["embed_scale"]))
        np.testing.assert_array_equal(hidden[i], x)
        ref = OD.ple_input(m, t, x)
        assert np.abs(ple[i] - ref).max() < 2e-2 * np.abs(ref).max()
        assert np.abs(ple[i] - ref).mean() < 2e-3 * np.abs(ref).mean()


def _qgemv_f32(x, words, scale, n_in, bits, in_q, out_q, drop_last=False, unq=False):
    """A quantised GEMV summed the way the decode kernels sum it, in f32: per-16-value chunk
    partial sums, the chunks added in order, the zero point times the sum of x subtracted,
    then the scale and srq -- a different order and precision than the oracle's."""
    codes = unpack_values(words, n_in, bits).astype(np.float32)
    xs = OD.srq(np.asarray(x, np.float32), in_q)
    if drop_last:
        xs = xs.copy()
        xs[-1] = 0
    prod = (codes * xs[None, :]).reshape(codes.shape[0], -1, 16)
    acc = np.zeros(codes.shape[0], np.float32)
    for c in range(prod.shape[1]):
        part = np.zeros(codes.shape[0], np.float32)
        for e in range(16):
            part = (part + prod[:, c, e]).astype(np.float32)
        acc = (acc + part).astype(np.float32)
    zsx = np.float32(1 << (bits - 1)) * np.float32(xs.sum(dtype=np.float32))
    v = (np.asarray(scale, np.float32) * (acc - zsx)).astype(np.float32)
    return v if unq else OD.srq(v, out_q)


def test_tie_aware_chain_check_accepts_f32_orders_and_rejects_mistakes():
    """The GPU decoder checks compare srq(gelu(srq(gate)) * srq(up)) chains against every choice
    of the operand codes whose sums sit on a rounding midpoint (helpers.qlin_codes/chain_close).
    An f32 GEMV in another summation order passes it; a dropped term, a swapped operand pair
    or a wrong sign fails it; and few codes have a second choice."""
    import pytest
    from helpers import chain_close, qlin_codes
    rng = np.random.default_rng(11)
    n_in, n_out, bits = 1536, 4096, 4
    gw, uw = (pack_values(rng.integers(0, 1 << bits, size=(n_out, n_in)), bits) for _ in range(2))
    gs, us = ((0.01 * (1 + rng.random(n_out))).astype(np.float32) for _ in range(2))
    x = (2 * rng.standard_normal(n_in)).astype(np.float32)
    g = qlin_codes(x, gw, gs, n_in, bits, 0.05, 0.02)
    u = qlin_codes(x, uw, us, n_in, bits, 0.04, 0.03)
    assert (g[0] != g[1]).mean() < 0.05 and (u[0] != u[1]).mean() < 0.05
    # the f32 order's error against the float64 sum, in units of 2^-24 * sum |terms|: a tenth
    # of the allowance qlin_codes makes (lam 4)
    codes = unpack_values(gw, n_in, bits).astype(np.float64)
    xs = OD.srq(x, 0.05).astype(np.float64)
    v64 = gs * ((codes - 8) @ xs)
    m = gs * (codes @ np.abs(xs) + 8 * np.abs(xs).sum())
    err = np.abs(_qgemv_f32(x, gw, gs, n_in, bits, 0.05, 0.0, unq=True) - v64) / (2.0 ** -24 * m)
    assert 0 < err.max() < 0.4
    fn = lambda a, b: OD.gelu_tanh(a) * b  # noqa: E731
    gk = _qgemv_f32(x, gw, gs, n_in, bits, 0.05, 0.02)
    uk = _qgemv_f32(x, uw, us, n_in, bits, 0.04, 0.03)
    chain_close(OD.srq(fn(gk, uk), 0.01), fn, [g, u], "f32 order", step=0.01)
    mul = rng.standard_normal(n_out).astype(np.float32)
    chain_close(OD.gelu_tanh(gk) * mul, lambda a: OD.gelu_tanh(a) * mul, [g], "gelu_mul f32 order")
    for bad in (OD.srq(fn(_qgemv_f32(x, gw, gs, n_in, bits, 0.05, 0.02, drop_last=True), uk), 0.01),
                OD.srq(fn(uk, gk), 0.01), OD.srq(fn(gk, -uk), 0.01)):
        with pytest.raises(AssertionError):
            chain_close(bad, fn, [g, u], "planted", step=0.01)
    with pytest.raises(AssertionError):
        chain_close(OD.gelu_tanh(gk) * mul[::-1], lambda a: OD.gelu_tanh(a) * mul, [g], "planted gelu_mul")
