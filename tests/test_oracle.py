"""Pin the CPU oracle (oracle/attention.py) before it is trusted as the GPU checker.

Three kinds of checks, chosen so that a plausible mistake (dropped gain, wrong
RoPE sign, off-by-one window edge, wrong GQA head map, wrong scale) fails one:
  1. golden vectors from an independent pure-Python float64 restatement on the
     reference tests' parameter sets (tests/golden/make_golden.py);
  2. closed forms and invariants (uniform attention = mean of attended rows,
     RoPE = complex rotation, split-KV merge identity, the helper invariants of
     the reference's tests/test_gemma4_reference.py:21-63);
  3. planted mistakes in the oracle (on the CPU) that the golden checks must catch.
"""
import math
import os

import numpy as np
import pytest

import oracle.attention as O

GOLD = os.path.join(os.path.dirname(__file__), "golden")
TOL = dict(atol=1e-4, rtol=1e-4)          # oracle (f32) vs float64 restatement


def load(name):
    return np.load(os.path.join(GOLD, name))


# ---------------------------------------------------------------- golden
def test_golden_g3_fused():
    z = load("g3_fused.npz")
    for i, kl in enumerate(z["key_len"]):
        got = O.decode_attention(z["q"], z["k"], z["v"], int(kl), 1, window=int(z["window"][i]),
                                 scale=float(z["scale"]))
        np.testing.assert_allclose(got, z["expected"][i], **TOL)


@pytest.mark.parametrize("tag", ["hd256_s0", "hd512_s0", "hd256_s3", "hd512_s5"])
def test_golden_g4_fused(tag):
    z = load("g4_fused.npz")
    got = O.decode_attention(z[f"{tag}_q"], z[f"{tag}_k"], z[f"{tag}_v"], int(z["key_len"]), 1,
                             window=int(z[f"{tag}_window"]), scale=1.0)
    np.testing.assert_allclose(got, z[f"{tag}_expected"], **TOL)


@pytest.mark.parametrize("tag", ["hd256_len90", "hd512_len90"])
def test_golden_attn101(tag):
    z = load("attn101.npz")
    kl = int(tag.split("len")[1])
    got = O.decode_attention(z[f"{tag}_q"], z[f"{tag}_k"], z[f"{tag}_v"], kl, 1,
                             q_gain=z[f"{tag}_w"], cos=z[f"{tag}_cos"], sin=z[f"{tag}_sin"])
    np.testing.assert_allclose(got, z[f"{tag}_expected"], **TOL)
    # with attn_101's OUT_Q epilogue: every element on the SRQ grid, at most one step
    # away from srq(expected) (a value on a .5 boundary may round either way)
    oq = float(z["out_q"])
    gq = O.decode_attention(z[f"{tag}_q"], z[f"{tag}_k"], z[f"{tag}_v"], kl, 1,
                            q_gain=z[f"{tag}_w"], cos=z[f"{tag}_cos"], sin=z[f"{tag}_sin"], out_q=oq)
    steps = gq / np.float32(oq)
    np.testing.assert_allclose(steps, np.round(steps), atol=1e-3)
    d = np.abs(gq - O.srq(z[f"{tag}_expected"].astype(np.float32), oq))
    assert (d <= oq * 1.001).all()
    assert np.count_nonzero(d) <= 2


@pytest.mark.parametrize("window", [0, 40])
def test_golden_g4e2b_decode(window):
    z = load("g4e2b_decode.npz")
    got = O.decode_attention(z["q"], z["k"], z["v"], int(z["key_len"]), int(z["n_kv_heads"]),
                             q_gain=z["w"], cos=z["cos"], sin=z["sin"], window=window)
    np.testing.assert_allclose(got, z[f"expected_w{window}"], **TOL)


@pytest.mark.parametrize("window", [0, 16])
def test_golden_prefill(window):
    z = load("prefill.npz")
    kw = dict(q_gain=z["w"], cos=z["cos"], sin=z["sin"], window=window)
    got = O.prefill_attention(z["q"], z["k"], z["v"], int(z["start_pos"]), int(z["n_kv_heads"]),
                              q_round_f16=False, block=7, **kw)
    np.testing.assert_allclose(got, z[f"expected_w{window}"], **TOL)
    # qprep_b's rounding point (q -> f16 after norm+RoPE, kernels_dsl.py:1872-1873).
    # (a) the oracle's f16 q equals the golden pipeline's, except where the f32 and f64
    #     values straddle a rounding boundary (then one f16 ulp apart);
    qn = O.apply_rope(O.rms_norm(z["q"], z["w"]), z["cos"][:, None, :], z["sin"][:, None, :])
    q16 = qn.astype(np.float16)
    diff = q16 != z["q16"]
    assert diff.mean() < 0.01
    np.testing.assert_allclose(q16.astype(np.float32), z["q16"].astype(np.float32), rtol=1e-3)
    # (b) fed the golden f16 q itself, the oracle's core matches the f64 restatement;
    got16 = O.prefill_attention(z["q16"].astype(np.float32), z["k"], z["v"], int(z["start_pos"]),
                                int(z["n_kv_heads"]), window=window, q_round_f16=True)
    np.testing.assert_allclose(got16, z[f"expected_q16_w{window}"], **TOL)
    # (c) end to end the boundary cases stay inside the contract tolerance, but the f16
    #     rounding of q alone moves outputs past 2e-3 (scale 1.0, unit-RMS q and k give
    #     scores with std ~16), so the oracle has to mirror the rounding point.
    e2e = O.prefill_attention(z["q"], z["k"], z["v"], int(z["start_pos"]), int(z["n_kv_heads"]),
                              q_round_f16=True, **kw)
    np.testing.assert_allclose(e2e, z[f"expected_q16_w{window}"], atol=2e-3, rtol=1e-2)
    assert np.abs(e2e - z[f"expected_w{window}"]).max() > 2e-3


def test_golden_kv_write():
    z = load("kv_write.npz")
    for tag, kq, vq in (("plain", 0.0, 0.0), ("srq", float(z["k_in_q"]), float(z["v_in_q"]))):
        k, v = O.kv_write(z["k"], z["v"], z["g"], z["cos"], z["sin"], k_in_q=kq, v_in_q=vq,
                          cache_dtype=np.float32)
        np.testing.assert_allclose(k, z[f"k_{tag}"], atol=1e-5, rtol=1e-5)
        np.testing.assert_allclose(v, z[f"v_{tag}"], atol=1e-5, rtol=1e-5)
        k16, _ = O.kv_write(z["k"], z["v"], z["g"], z["cos"], z["sin"], k_in_q=kq, v_in_q=vq)
        assert k16.dtype == np.float16
        np.testing.assert_allclose(k16.astype(np.float32), z[f"k_{tag}"], rtol=1e-3, atol=1e-4)


# ---------------------------------------------------------------- closed forms
def test_rms_norm_scales_by_w_not_1_plus_w():       # reference tests/test_gemma4_reference.py:22-28
    x = np.random.default_rng(0).standard_normal(64).astype(np.float32)
    w = np.full(64, 2.0, np.float32)
    np.testing.assert_allclose(O.rms_norm(x, w), x / np.sqrt(np.mean(x * x) + 1e-6) * 2.0, rtol=1e-6)


def test_rms_norm_noscale_is_unit_gain():           # reference tests/test_gemma4_reference.py:30-35
    x = np.random.default_rng(1).standard_normal(64).astype(np.float32)
    np.testing.assert_allclose(O.rms_norm_noscale(x), O.rms_norm(x, np.ones(64, np.float32)), rtol=1e-6)
    r = O.rms_norm_noscale(np.random.default_rng(2).standard_normal((5, 256)).astype(np.float32) * 7)
    np.testing.assert_allclose(np.sqrt(np.mean(r.astype(np.float64) ** 2, -1)), 1.0, rtol=1e-5)


def test_rope_is_complex_rotation():
    rng = np.random.default_rng(3)
    hd, pos, theta = 256, 37, 1e4
    x = rng.standard_normal((4, hd)).astype(np.float32)
    c, s = O.rope_tables([pos], hd, theta)
    got = O.apply_rope(x, c[0], s[0]).astype(np.float64)
    half = hd // 2
    ang = pos * theta ** (-2.0 * np.arange(half) / hd)
    z = (x[:, :half] + 1j * x[:, half:]).astype(np.complex128) * np.exp(1j * ang)
    np.testing.assert_allclose(got[:, :half], z.real, atol=1e-5)
    np.testing.assert_allclose(got[:, half:], z.imag, atol=1e-5)
    # pair norms preserved
    np.testing.assert_allclose(np.hypot(got[:, :half], got[:, half:]),
                               np.hypot(x[:, :half], x[:, half:]), rtol=1e-5)


def test_rope_tables_match_math_and_reference_formula():
    hd, theta = 256, 1e6
    pos = [0, 1, 4095, 8191]
    c, s = O.rope_tables(pos, hd, theta)
    for r, p in enumerate(pos):
        for i in (0, 1, 63, 127):
            a = p * theta ** (-2.0 * i / hd)
            assert abs(c[r, i] - math.cos(a)) < 1e-7 and abs(s[r, i] - math.sin(a)) < 1e-7
    # reference.py:46-55 (f32 angles) agrees at small positions
    x = np.random.default_rng(4).standard_normal((2, hd)).astype(np.float32)
    c7, s7 = O.rope_tables([7], hd, theta)
    np.testing.assert_allclose(O.rope(x, 7, theta, hd // 2), O.apply_rope(x, c7[0], s7[0]), atol=1e-5)


def test_rope_partial_identity_beyond_cutoff():     # reference tests/test_gemma4_reference.py:46-55
    x = np.random.default_rng(3).standard_normal((8, 512)).astype(np.float32)
    got = O.rope(x, 100, 1e6, 64)
    np.testing.assert_array_equal(got[:, 64:256], x[:, 64:256])
    np.testing.assert_array_equal(got[:, 256 + 64:], x[:, 256 + 64:])
    assert not np.allclose(got[:, :64], x[:, :64])


def test_srq_grid_clamp_and_ties():
    s = 0.25
    x = np.array([0.125, 0.375, -0.125, 100.0, -100.0, 0.3], np.float32)
    np.testing.assert_array_equal(O.srq(x, s), np.array([0.0, 0.5, -0.0, 31.75, -32.0, 0.25], np.float32))
    np.testing.assert_array_equal(O.srq(x, 0.0), x)


@pytest.mark.parametrize("T,window", [(1, 0), (64, 0), (65, 64), (64, 64), (63, 64), (257, 256),
                                      (256, 256), (255, 256), (300, 37)])
def test_uniform_attention_is_mean_of_attended_rows(T, window):
    """q = 0 makes every attended key weigh 1/n: output = mean of exactly the attended V rows.
    One-hot V rows (v_j = e_j) turn the output into the indicator of the attended set."""
    hd = 512
    v = np.zeros((T, 1, hd), np.float32)
    v[np.arange(T), 0, np.arange(T) % hd] = 1.0
    k = np.random.default_rng(T).standard_normal((T, 1, hd)).astype(np.float32)
    out = O.decode_attention(np.zeros((2, hd), np.float32), k, v, T, 1, window=window)
    lo, hi = (max(0, T - window) if window else 0), T
    want = np.zeros(hd, np.float32)
    for j in range(lo, hi):
        want[j % hd] += 1.0 / (hi - lo)
    np.testing.assert_allclose(out[0], want, atol=1e-6)
    assert set(np.nonzero(out[0])[0]) == {j % hd for j in range(lo, hi)}


def test_prefill_mask_sets_exact():
    """Per query row: attended set == [max(0, p+1-W), p] via one-hot V and q = 0."""
    S, start, hd = 40, 23, 128
    T = start + S
    for window in (0, 1, 8, 24, 63, 64):
        v = np.zeros((T, 1, hd), np.float32)
        v[np.arange(T), 0, np.arange(T) % hd] = 1.0
        out = O.prefill_attention(np.zeros((S, 1, hd), np.float32), v, v, start, 1,
                                  window=window, q_round_f16=False, block=16)
        for s in range(S):
            p = start + s
            lo = max(0, p + 1 - window) if window else 0
            assert set(np.nonzero(out[s, 0] > 1e-6)[0]) == {j % hd for j in range(lo, p + 1)}


def test_gqa_head_map():
    rng = np.random.default_rng(9)
    nH, kvH, hd, T = 8, 2, 64, 20
    q = rng.standard_normal((nH, hd)).astype(np.float32)
    k = rng.standard_normal((T, kvH, hd)).astype(np.float32)
    v = rng.standard_normal((T, kvH, hd)).astype(np.float32)
    full = O.decode_attention(q, k, v, T, kvH)
    for h in range(nH):
        kh = h // 4
        one = O.decode_attention(q[h:h + 1], k[:, kh:kh + 1], v[:, kh:kh + 1], T, 1)
        np.testing.assert_allclose(full[h], one[0], atol=1e-6)


def test_split_kv_merge_identity():
    rng = np.random.default_rng(11)
    hd, T = 256, 1000
    q = rng.standard_normal(hd)
    k = rng.standard_normal((T, hd)) * 0.3
    v = rng.standard_normal((T, hd))
    whole = O.merge_partials([O.partial_attention(q, k, v)])
    for cuts in ([0, 1000], [0, 1, 1000], [0, 64, 128, 500, 999, 1000], list(range(0, 1001, 37)) + [1000]):
        cuts = sorted(set(cuts))
        parts = [O.partial_attention(q, k[a:b], v[a:b]) for a, b in zip(cuts[:-1], cuts[1:])]
        np.testing.assert_allclose(O.merge_partials(parts), whole, rtol=1e-12, atol=1e-12)
    direct = O.decode_attention(q[None].astype(np.float32), k[:, None].astype(np.float32),
                                v[:, None].astype(np.float32), T, 1)
    np.testing.assert_allclose(direct[0], whole, atol=1e-5)


def test_scale_is_applied_to_scores():
    rng = np.random.default_rng(12)
    q = rng.standard_normal((4, 256)).astype(np.float32)
    k = rng.standard_normal((30, 1, 256)).astype(np.float32)
    v = rng.standard_normal((30, 1, 256)).astype(np.float32)
    np.testing.assert_allclose(O.decode_attention(q, k, v, 30, 1, scale=1 / 16),
                               O.decode_attention(q / 16, k, v, 30, 1), atol=1e-6)


def test_batched_decode_matches_per_sequence():
    rng = np.random.default_rng(13)
    B, nH, kvH, hd, T = 3, 8, 2, 64, 50
    q = rng.standard_normal((B, nH, hd)).astype(np.float32)
    k = rng.standard_normal((B, T, kvH, hd)).astype(np.float32)
    v = rng.standard_normal((B, T, kvH, hd)).astype(np.float32)
    lens = [50, 7, 33]
    got = O.decode_attention_batched(q, k, v, lens, kvH)
    for b in range(B):
        np.testing.assert_allclose(got[b], O.decode_attention(q[b], k[b], v[b], lens[b], kvH))


def test_prefill_last_row_equals_decode():
    """The last prefill row is a decode query at p = T-1 (q rounding off)."""
    z = load("prefill.npz")
    S, start = z["q"].shape[0], int(z["start_pos"])
    pre = O.prefill_attention(z["q"], z["k"], z["v"], start, 2, q_gain=z["w"], cos=z["cos"],
                              sin=z["sin"], window=16, q_round_f16=False)
    dec = O.decode_attention(z["q"][-1], z["k"], z["v"], start + S, 2, q_gain=z["w"],
                             cos=z["cos"][-1], sin=z["sin"][-1], window=16)
    np.testing.assert_allclose(pre[-1], dec, atol=1e-6)


def test_prefill_cache_rounding_is_the_gemm_forms():
    """kv_round_f16 (the GEMM form's srqh_b on both caches, prefill_gpu.py:286-288) is a no-op
    on f16 caches, equals the oracle on explicitly f16-rounded f32 caches, and moves the
    output well beyond the contract with scale 1.0 -- why the fused form (which reads its f32
    caches as they are) must not round K."""
    z = load("prefill.npz")
    S, start = z["q"].shape[0], int(z["start_pos"])
    kw = dict(q_gain=z["w"], cos=z["cos"], sin=z["sin"], window=16, q_round_f16=False)
    k16, v16 = z["k"], z["v"]
    assert k16.dtype == np.float16
    np.testing.assert_array_equal(O.prefill_attention(z["q"], k16, v16, start, 2, kv_round_f16=True, **kw),
                                  O.prefill_attention(z["q"], k16, v16, start, 2, **kw))
    rng = np.random.default_rng(3)
    k32 = (k16.astype(np.float32) * (1 + 2e-3 * rng.standard_normal(k16.shape))).astype(np.float32)
    v32 = (v16.astype(np.float32) * (1 + 2e-3 * rng.standard_normal(v16.shape))).astype(np.float32)
    rounded = O.prefill_attention(z["q"], k32, v32, start, 2, kv_round_f16=True, **kw)
    np.testing.assert_array_equal(
        rounded, O.prefill_attention(z["q"], k32.astype(np.float16), v32.astype(np.float16), start, 2, **kw))
    exact = O.prefill_attention(z["q"], k32, v32, start, 2, **kw)
    assert np.abs(rounded - exact).max() > 2e-3


# ---------------------------------------------------------------- planted mistakes
def _g4e2b_err(window):
    z = load("g4e2b_decode.npz")
    got = O.decode_attention(z["q"], z["k"], z["v"], int(z["key_len"]), int(z["n_kv_heads"]),
                             q_gain=z["w"], cos=z["cos"], sin=z["sin"], window=window)
    return np.abs(got - z[f"expected_w{window}"]).max()


@pytest.mark.parametrize("mistake", ["window_off_by_one", "gqa_modulo", "no_gain", "rope_sign"])
def test_planted_mistakes_are_caught(monkeypatch, mistake):
    assert _g4e2b_err(40) < 1e-4
    if mistake == "window_off_by_one":
        monkeypatch.setattr(O, "attended_range",
                            lambda p, w: ((max(0, p + 2 - w) if w > 0 else 0), p + 1))
    elif mistake == "gqa_modulo":
        monkeypatch.setattr(O, "kv_head_of", lambda h, nh, nkv: h % nkv)
    elif mistake == "no_gain":
        monkeypatch.setattr(O, "rms_norm", lambda x, w, eps=1e-6: O.rms_norm_noscale(x, eps))
    elif mistake == "rope_sign":
        orig = O.apply_rope
        monkeypatch.setattr(O, "apply_rope", lambda x, c, s: orig(x, c, -s))
    assert _g4e2b_err(40) > 2e-3      # the contract tolerance would flag it
