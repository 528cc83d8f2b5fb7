"""Pin the projection oracle (oracle/projection.py) before it checks the GPU kernels.

The reference holds no stored vectors for these kernels: its own tests compare two GPU
translations of the same kernel bit for bit and check dq_f16 exactly against a float64
reconstruction (tests/test_kernels_dsl_parity.py:658-700, 785-829). The oracle is pinned
here by:
  1. known-answer words whose values are written out by hand (value order, all widths);
  2. the float64 reconstruction of dq_f16, as the reference's test does;
  3. a pure-Python restatement of qkv_70's loop (lo/hi nibble vec4 dots, kernels_dsl.py:
     1417-1428) on small sizes, so a wrong interleave in the vectorised oracle fails;
  4. closed forms: values at the zero point give 0, a one-hot input picks one column,
     an identity input reproduces the dequantised weights;
  5. a planted mistake (nibbles swapped) that check 3 must catch.
"""
import numpy as np
import pytest

import oracle.projection as P


# ---------------------------------------------------------------- 1. known answers
def test_unpack_known_words():
    w4 = np.array([[0x76543210, 0xFEDCBA98]], np.uint32)
    assert P.unpack_values(w4, 16, 4).tolist() == [list(range(16))]
    # 2-bit: byte 0b11100100 holds 0, 1, 2, 3 from the low bits up
    w2 = np.array([[0xE4E4E4E4]], np.uint32)
    assert P.unpack_values(w2, 16, 2).tolist() == [[0, 1, 2, 3] * 4]
    w8 = np.array([[0x04030201, 0xFF00807F]], np.uint32)
    assert P.unpack_values(w8, 8, 8).tolist() == [[1, 2, 3, 4, 0x7F, 0x80, 0x00, 0xFF]]


@pytest.mark.parametrize("bits", [2, 4, 8])
def test_pack_roundtrip(bits):
    rng = np.random.default_rng(5)
    vals = rng.integers(0, 1 << bits, size=(7, 96))
    words = P.pack_values(vals, bits)
    assert words.shape == (7, 96 * bits // 32)
    assert np.array_equal(P.unpack_values(words, 96, bits), vals)


# ---------------------------------------------------------------- 2. float64 reconstruction
@pytest.mark.parametrize("bits", [2, 4, 8])
def test_dequant_float64_reconstruction(bits):
    """tests/test_kernels_dsl_parity.py:785-829's check, on every row."""
    n_in, n_out = 256, 64
    vpw, per_byte = 32 // bits, 8 // bits
    rng = np.random.default_rng(131)
    words = rng.integers(0, 2 ** 32, size=n_out * (n_in // vpw), dtype=np.uint64).astype(np.uint32)
    scale = (rng.random(n_out).astype(np.float32) * 0.01 + 0.001)
    got = P.dequant_f16(words, scale, n_in, n_out, bits)
    raw = words.reshape(n_out, -1).astype(np.uint64)
    sh = np.array([8 * (i // per_byte) + bits * (i % per_byte) for i in range(vpw)], np.uint64)
    q = ((raw[:, :, None] >> sh[None, None, :]) & np.uint64((1 << bits) - 1)).astype(np.float64)
    exact = scale.astype(np.float64)[:, None] * (q.reshape(n_out, -1) - (1 << (bits - 1)))
    ref = exact.astype(np.float16)
    for o in (0, 1, n_out - 1):  # the rows the reference's test compares exactly
        assert np.array_equal(got[o], ref[o]), f"row {o}"
    # elsewhere the kernel's f32 product rounded to f16 may differ from the float64 product
    # rounded to f16 only where the f32 product is inexact (double rounding), by one ulp
    diff = got != ref
    f32_inexact = exact.astype(np.float32).astype(np.float64) != exact
    assert not (diff & ~f32_inexact).any()
    ulp = np.spacing(np.abs(ref)).astype(np.float64)
    assert (np.abs(got.astype(np.float64) - ref.astype(np.float64)) <= ulp).all()


# ---------------------------------------------------------------- 3. qkv_70's loop
def _qkv70_loop(a, sum_a, words, scales, n_rows):
    """qkv_70's per-row loop as written (kernels_dsl.py:1417-1436), float64."""
    out = []
    wpr = len(a) // 8
    for o in range(n_rows):
        acc = 0.0
        for w in range(wpr):
            p = int(words[o * wpr + w])
            lo = [(p >> (8 * j)) & 0x0F for j in range(4)]
            hi = [(p >> (8 * j + 4)) & 0x0F for j in range(4)]
            v0 = (lo[0], hi[0], lo[1], hi[1])
            v1 = (lo[2], hi[2], lo[3], hi[3])
            acc += sum(x * float(a[8 * w + i]) for i, x in enumerate(v0))
            acc += sum(x * float(a[8 * w + 4 + i]) for i, x in enumerate(v1))
        out.append(float(scales[o]) * (acc - 8.0 * float(sum_a)))
    return np.array(out)


def _qkv_case(seed=111, hidden=64, qd=24, kvd=8):
    rng = np.random.default_rng(seed)
    a = rng.standard_normal(hidden).astype(np.float32)
    wpr = hidden // 8
    qb = rng.integers(0, 2 ** 32, size=qd * wpr, dtype=np.uint64).astype(np.uint32)
    kb = rng.integers(0, 2 ** 32, size=kvd * wpr, dtype=np.uint64).astype(np.uint32)
    vb = rng.integers(0, 2 ** 32, size=kvd * wpr, dtype=np.uint64).astype(np.uint32)
    sc = (rng.random(qd + 2 * kvd).astype(np.float32) * 0.01 + 0.001)
    return a, np.float32(a.sum(dtype=np.float64)), qb, kb, vb, sc


def test_qkv_gemv_matches_kernel_loop():
    a, sa, qb, kb, vb, sc = _qkv_case()
    q, k, v = P.qkv_gemv(a, sa, qb, kb, vb, sc, 24, 8)
    np.testing.assert_allclose(q, _qkv70_loop(a, sa, qb, sc, 24), rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(k, _qkv70_loop(a, sa, kb, sc[24:], 8), rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(v, _qkv70_loop(a, sa, vb, sc[32:], 8), rtol=1e-6, atol=1e-7)
    q_only, kn, vn = P.qkv_gemv(a, sa, qb, None, None, sc, 24, 0)
    assert kn is None and vn is None and np.array_equal(q_only, q)


def test_qkv_gemv_srq_grid():
    a, sa, qb, kb, vb, sc = _qkv_case(seed=3)
    q, k, v = P.qkv_gemv(a, sa, qb, kb, vb, sc, 24, 8, 0.03125, 0.0234375, 0.0156)
    for x, s in ((q, 0.03125), (k, 0.0234375), (v, 0.0156)):
        n = x / np.float32(s)
        assert np.allclose(n, np.round(n), atol=1e-3) and np.abs(n).max() <= 128


# ---------------------------------------------------------------- 4. closed forms
def test_zero_point_gives_zero():
    rng = np.random.default_rng(9)
    a = rng.standard_normal(64).astype(np.float32)
    words = np.full(16 * 8, 0x88888888, np.uint32)  # every value 8 = the zero point
    q, _, _ = P.qkv_gemv(a, a.sum(dtype=np.float64), words, None, None, np.ones(16, np.float32), 16, 0)
    assert np.abs(q).max() < 1e-5


def test_one_hot_input_picks_a_column():
    rng = np.random.default_rng(10)
    vals = rng.integers(0, 16, size=(12, 64))
    words = P.pack_values(vals, 4)
    sc = rng.random(12).astype(np.float32) + 0.5
    for j in (0, 1, 7, 8, 63):
        a = np.zeros(64, np.float32)
        a[j] = 1.0
        q, _, _ = P.qkv_gemv(a, 1.0, words, None, None, sc, 12, 0)
        np.testing.assert_allclose(q, sc * (vals[:, j] - 8), rtol=1e-6)


@pytest.mark.parametrize("bits", [2, 4, 8])
def test_identity_input_reproduces_weights(bits):
    rng = np.random.default_rng(11)
    n, k = 16, 64
    words = rng.integers(0, 2 ** 32, size=n * k * bits // 32, dtype=np.uint64).astype(np.uint32)
    w = P.dequant_f16(words, rng.random(n).astype(np.float32) * 0.1, k, n, bits)
    c = P.proj_gemm(np.eye(k, dtype=np.float32), w)
    assert np.array_equal(c, w.T)


def test_gemm_rows_match_gemv():
    """A GEMM row over dequantised weights equals the GEMV up to the f16 roundings."""
    a, sa, qb, kb, vb, sc = _qkv_case(seed=12, hidden=128, qd=32, kvd=8)
    a16 = a.astype(np.float16).astype(np.float32)  # f16-exact input: srqh_b is lossless
    q, _, _ = P.qkv_gemv(a16, a16.sum(dtype=np.float64), qb, None, None, sc, 32, 0)
    w = P.dequant_f16(qb, sc, 128, 32, 4)
    c = P.proj_gemm(a16[None, :], w)[0].astype(np.float64)
    np.testing.assert_allclose(c, q, rtol=2e-3, atol=2e-3)
    cq = P.proj_gemm(a16[None, :], w, out_f32=True, out_q=0.03125)[0]
    assert np.allclose(cq / 0.03125, np.round(cq / 0.03125), atol=1e-3)


# ---------------------------------------------------------------- 5. planted mistake
def test_swapped_nibbles_are_caught(monkeypatch):
    real = P.unpack_values

    def swapped(words, n_in, bits):
        v = real(words, n_in, bits)
        return v.reshape(v.shape[0], -1, 2)[:, :, ::-1].reshape(v.shape)

    monkeypatch.setattr(P, "unpack_values", swapped)
    a, sa, qb, kb, vb, sc = _qkv_case()
    q, _, _ = P.qkv_gemv(a, sa, qb, kb, vb, sc, 24, 8)
    assert not np.allclose(q, _qkv70_loop(a, sa, qb, sc, 24), rtol=1e-6, atol=1e-7)
