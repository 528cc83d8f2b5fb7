"""Shared test helpers: the parity bar and input builders."""
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


def f16_ulp_close(got, ref, what="", ulps=1):
    """f16 results within `ulps` units in the last place of the f16 reference."""
    got = np.asarray(got, np.float16).astype(np.float64)
    ref16 = np.asarray(ref, np.float16)
    ulp = np.spacing(np.abs(ref16)).astype(np.float64)
    d = np.abs(got - ref16.astype(np.float64))
    assert (d <= ulps * ulp + 1e-7).all(), f"{what}: {int((d > ulps * ulp).sum())} elements beyond {ulps} ulp"
