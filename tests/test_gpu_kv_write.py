"""GPU parity of the KV-cache write (g4a_kv_write; kvnorm / kvnorm_b semantics).

f16 cache rows must be within one f16 ulp of the oracle's (the kernel and numpy round
the same f32 value, which may differ in its last f32 bit); f32 rows within 1e-5.
Mirrors tests/test_kernels_dsl_parity.py:319-356 (write at row 3, hd 256 and 512).
"""
import numpy as np
import pytest
import torch

import oracle.attention as O
import slang_amd as sa
from helpers import f16_ulp_close, gold

pytestmark = pytest.mark.gpu
DEV = "cuda"


def t(x):
    return torch.from_numpy(np.ascontiguousarray(x)).to(DEV)


def test_golden_kv_write():
    z = gold("kv_write.npz")
    S, kvH, hd = z["k"].shape
    start = int(z["start_pos"])
    for tag, kq, vq in (("plain", 0.0, 0.0), ("srq", float(z["k_in_q"]), float(z["v_in_q"]))):
        for cache_dtype in (torch.float32, torch.float16):
            kc = torch.zeros(start + S + 2, kvH, hd, dtype=cache_dtype, device=DEV)
            vc = torch.zeros_like(kc)
            sa.kv_write(t(z["k"]), t(z["v"]), kc, vc, start, sa.AttnConfig(kvH, kvH, hd),
                        k_gain=t(z["g"]), rope_cos=t(z["cos"]), rope_sin=t(z["sin"]), k_in_q=kq, v_in_q=vq)
            torch.cuda.synchronize()
            kg, vg = kc.cpu().float().numpy(), vc.cpu().float().numpy()
            assert not kg[:start].any() and not kg[start + S:].any(), "wrote outside its rows"
            if cache_dtype == torch.float32:
                np.testing.assert_allclose(kg[start:start + S], z[f"k_{tag}"], atol=1e-5, rtol=1e-5)
                np.testing.assert_allclose(vg[start:start + S], z[f"v_{tag}"], atol=1e-5, rtol=1e-5)
            else:
                f16_ulp_close(kg[start:start + S], z[f"k_{tag}"], f"k {tag}")
                f16_ulp_close(vg[start:start + S], z[f"v_{tag}"], f"v {tag}")


@pytest.mark.parametrize("hd", [256, 512])
@pytest.mark.parametrize("in_dtype", [np.float32, np.float16])
def test_kv_write_matches_oracle(hd, in_dtype):
    """Config-2/3 style: 4096 tokens, kvH 2, gains ~N(1,0.1), RoPE theta 1e6, f16 caches;
    f16 inputs with srq scales (kvnorm_b) and f32 inputs (kvnorm)."""
    rng = np.random.default_rng(hd)
    S, kvH = 4096, 2
    k = rng.standard_normal((S, kvH, hd)).astype(in_dtype)
    v = rng.standard_normal((S, kvH, hd)).astype(in_dtype)
    g = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    cos, sin = O.rope_tables(np.arange(S), hd, 1e6)
    kq, vq = (0.0, 0.0) if in_dtype == np.float32 else (0.02, 0.03)
    kc = torch.zeros(S, kvH, hd, dtype=torch.float16, device=DEV)
    vc = torch.zeros_like(kc)
    sa.kv_write(t(k), t(v), kc, vc, 0, sa.AttnConfig(kvH, kvH, hd), k_gain=t(g), rope_cos=t(cos),
                rope_sin=t(sin), k_in_q=kq, v_in_q=vq)
    torch.cuda.synchronize()
    rk, rv = O.kv_write(k, v, g, cos, sin, k_in_q=kq, v_in_q=vq)
    f16_ulp_close(kc.cpu().numpy(), rk, "k")
    f16_ulp_close(vc.cpu().numpy(), rv, "v")


def test_kvnorm_mirror_decode_step():
    """kvnorm slot drop-in: one token written at pkv = pos*hd (test_kvnorm_bit_exact writes row 3)."""
    hd, pos = 256, 3
    rng = np.random.default_rng(51)
    k = rng.standard_normal(hd).astype(np.float32)
    v = rng.standard_normal(hd).astype(np.float32)
    g = rng.standard_normal(hd).astype(np.float32)
    c, s = O.rope_tables([pos], hd, 1e4)
    kc = torch.zeros(16 * hd, dtype=torch.float16, device=DEV)
    vc = torch.zeros_like(kc)
    sa.kvnorm(t(k), t(v), t(g), t(c[0]), t(s[0]), kc, vc, (pos * hd, 0, 0, 0), head_dim=hd)
    torch.cuda.synchronize()
    rk, rv = O.kv_write(k[None, None], v[None, None], g, c, s)
    kg, vg = kc.cpu().numpy().reshape(16, hd), vc.cpu().numpy().reshape(16, hd)
    f16_ulp_close(kg[pos], rk[0, 0], "k row")
    f16_ulp_close(vg[pos], rv[0, 0], "v row")
    assert np.count_nonzero(kg[np.arange(16) != pos]) == 0


def test_no_v_norm_and_no_gain():
    hd, kvH, S = 256, 1, 8
    rng = np.random.default_rng(2)
    k = rng.standard_normal((S, kvH, hd)).astype(np.float32)
    v = rng.standard_normal((S, kvH, hd)).astype(np.float32)
    kc = torch.zeros(S, kvH, hd, dtype=torch.float32, device=DEV)
    vc = torch.zeros_like(kc)
    sa.kv_write(t(k), t(v), kc, vc, 0, sa.AttnConfig(1, 1, hd), v_norm=False)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(kc.cpu().numpy(), k)
    np.testing.assert_array_equal(vc.cpu().numpy(), v)
