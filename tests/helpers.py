"""Shared test helpers: the parity bar and input builders."""
import itertools
import os

import numpy as np

# max-abs 2e-3 and relative 1e-2 (f16 inputs, f32 accumulation)
ATOL, RTOL = 2e-3, 1e-2
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def gold(name):
    return np.load(os.path.join(GOLD, name))


def contract_close(got, ref, what=""):
    """|got - ref| <= 2e-3 + 1e-2 |ref| elementwise; also returns the max abs error."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, f"{what}: shape {got.shape} vs {ref.shape}"
    assert np.isfinite(got).all(), f"{what}: non-finite output"
    err = np.abs(got - ref)
    bad = err > ATOL + RTOL * np.abs(ref)
    assert not bad.any(), (f"{what}: {int(bad.sum())}/{bad.size} beyond 2e-3+1e-2|ref| "
                           f"(max abs err {err.max():.3e} at {np.unravel_index(err.argmax(), err.shape)})")
    return float(err.max())


def srq_close(got, ref_unquantised, step, what="", max_flip_frac=0.05):
    """SRQ'd outputs: on the grid, and at most one grid step from srq(ref) (a value near a
    .5 boundary may round either way, as the reference's own tie-aware check allows,
    gemma4_150/prefill_research/test_attn_prefill.py:68-79)."""
    got = np.asarray(got, np.float64)
    k = got / step
    assert np.abs(k - np.round(k)).max() < 1e-3, f"{what}: output off the SRQ grid"
    s = np.float32(step)
    ref_q = np.clip(np.round(np.asarray(ref_unquantised, np.float32) / s), -128, 127) * s
    d = np.abs(got - ref_q)
    assert (d <= step * 1.001).all(), f"{what}: a difference beyond one SRQ step ({d.max():.3e})"
    assert (d > 0).mean() <= max_flip_frac, f"{what}: {(d > 0).mean():.3%} of elements one step off"


def f16_ulp_close(got, ref, what="", ulps=1, slack=1e-7):
    """f16 results within `ulps` units in the last place of the f16 reference, plus an absolute
    `slack` for values the f32 arithmetic before the rounding leaves a few f32 ulps of their
    O(1) inputs apart (a RoPE pair that nearly cancels gives a tiny value whose f16 ulp is
    smaller than that)."""
    got = np.asarray(got, np.float16).astype(np.float64)
    ref16 = np.asarray(ref, np.float16)
    ulp = np.spacing(np.abs(ref16)).astype(np.float64)
    d = np.abs(got - ref16.astype(np.float64))
    bad = d > ulps * ulp + slack
    assert not bad.any(), (f"{what}: {int(bad.sum())} elements beyond {ulps} ulp + {slack:g}, e.g. got "
                           f"{got[bad][:3]} vs {ref16[bad][:3]}")


def tie_aware_e2e(got, ref_own, ref_kernel_q, q16, q_f32, what):
    """End-to-end check against the oracle's own f16 rounding of q (ref_own), tie-aware.

    q_f32 [S][nH][hd] is the oracle's normalised, rotated q before rounding and q16 the
    kernel's f16 q. Every element of `got` outside 2e-3 + 1e-2|ref_own| must lie in a
    (token, head) row where q16 differs from the oracle's rounding, every such difference
    must be one f16 ulp of a value that straddles a rounding boundary, and those rows must
    meet the contract against ref_kernel_q (the oracle fed the kernel's q16). Returns the
    number of (token, head) rows that needed the tie allowance."""
    oq16 = q_f32.astype(np.float16)
    f16_ulp_close(q16, q_f32, f"{what}: kernel q16 vs the oracle's unrounded q", slack=4e-6)
    diff = q16 != oq16
    if diff.any():
        # a differing element sits on a rounding boundary: the kernel's f32 value and the
        # oracle's straddle it, and they differ only by the f32 arithmetic before the rounding
        # (norm, gain, RoPE: a few f32 ulps of values below 8, so within 4e-6)
        mid = (q16[diff].astype(np.float64) + oq16[diff].astype(np.float64)) / 2
        ulp = np.abs(q16[diff].astype(np.float64) - oq16[diff].astype(np.float64))
        dist = np.abs(q_f32[diff].astype(np.float64) - mid)
        assert (dist <= ulp / 64 + 4e-6).all(), \
            f"{what}: a q16 difference that is not a rounding tie (max distance {dist.max():.2e}, ulp {ulp.max():.2e})"
    row_diff = diff.any(axis=-1)                          # [S][nH]
    err = np.abs(got.astype(np.float64) - ref_own)
    bad_rows = (err > ATOL + RTOL * np.abs(ref_own)).any(axis=-1)
    stray = bad_rows & ~row_diff
    assert not stray.any(), (f"{what}: {int(stray.sum())} rows outside the contract with the "
                             f"same f16 q as the oracle, e.g. {np.argwhere(stray)[:4].tolist()}")
    if bad_rows.any():
        contract_close(got[bad_rows], ref_kernel_q[bad_rows], f"{what}: tie rows on the kernel's q")
    return int(bad_rows.sum())


def qlin_codes(x, words, scale, n_in, bits, in_q, out_q, lam=4.0):
    """The values srq(qlin(x)) may take when the GEMV sums in f32 (oracle.decoder.qlin is
    W @ srq(x, in_q), then srq(., out_q)). Returns (code, alt): code is the oracle's value
    computed in float64, alt the grid value on the other side of the rounding midpoint where
    the exact sum lies within the f32 sum's error of that midpoint (else alt == code).

    The error allowed is lam * 2^-24 * m, m the sum of |terms| the kernels add (the raw codes
    times x, and the zero point times the sum of x, subtracted once per row), plus 2^-21
    |value| for the scale product and the division by out_q. Terms of random sign make an f32
    sum's error grow like 2^-24 m, not n 2^-24 m (the probabilistic analyses of Higham and
    Mary, SIAM J. Sci. Comput. 2019 and 2020); a sequential f32 sum of these tests' data
    reaches 0.37 of 2^-24 m, so lam 4 leaves a factor ten."""
    from oracle.projection import unpack_values
    from oracle.attention import srq
    codes = unpack_values(words, n_in, bits).astype(np.float64)
    zp = float(1 << (bits - 1))
    xs = srq(np.asarray(x, np.float32), in_q).astype(np.float64)
    sc = np.abs(np.asarray(scale, np.float64))
    v = np.asarray(scale, np.float64) * ((codes - zp) @ xs)
    mag = sc * (codes @ np.abs(xs) + zp * np.abs(xs).sum())
    err = lam * 2.0 ** -24 * mag + 2.0 ** -21 * np.abs(v)
    k = v / out_q
    base = np.clip(np.round(k), -128, 127)
    other = np.clip(base + np.where(k >= base, 1.0, -1.0), -128, 127)
    near = np.abs(np.abs(k - base) - 0.5) * out_q <= err
    return (base * out_q).astype(np.float32), (np.where(near, other, base) * out_q).astype(np.float32)


def chain_close(got, fn, operands, what="", step=None, max_flip_frac=0.05):
    """got = fn(*operands), each operand a (code, alt) pair from qlin_codes: every element must
    match fn for SOME choice of its operands' codes -- within one grid step of srq(fn, step)
    (at most max_flip_frac of them a step off: a midpoint of the last rounding), or with
    step None within 2e-3 + 1e-2 |fn|. An operand code only has a second choice where its own
    sum sits on a rounding midpoint, so a wrong term, sign or index fails."""
    from oracle.attention import srq
    got = np.asarray(got, np.float64)
    if step is not None:
        assert np.abs(got / step - np.round(got / step)).max() < 1e-3, f"{what}: off the SRQ grid"
    best = np.full(got.shape, np.inf)
    n_alt = [int((a != c).sum()) for c, a in operands]
    for choice in itertools.product(*[(0, 1)] * len(operands)):
        ref = fn(*[operands[i][ch] for i, ch in enumerate(choice)]).astype(np.float32)
        if step is not None:
            d = np.abs(got - srq(ref, step)) / (step * 1.001)
        else:
            d = np.abs(got - ref) / (ATOL + RTOL * np.abs(ref.astype(np.float64)))
        best = np.minimum(best, d)
    bad = best > 1.0
    assert not bad.any(), (f"{what}: {int(bad.sum())}/{bad.size} elements match no choice of operand codes "
                           f"(worst {best.max():.2f}x the bound; operands with a second code: {n_alt})")
    if step is not None:
        assert (best > 0).mean() <= max_flip_frac, f"{what}: {(best > 0).mean():.2%} of elements a step off"
