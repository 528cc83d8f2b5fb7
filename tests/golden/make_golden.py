"""Write the golden attention fixtures under tests/golden/.

    python tests/golden/make_golden.py

The reference ships no golden vectors: every attention test in it computes its
expectation live on an Apple GPU. These fixtures therefore come from an
independent restatement of the textbook definitions in pure Python float64
(`math` only -- no numpy arithmetic touches the expected values), evaluated on
the parameter sets of the reference's own attention tests:

  g3_fused      tests/test_gemma3_kernels_gpu.py:372-395  nH 4, hd 256, scale 1/sqrt(hd),
                (kv_len, start) in {(10,0),(100,0),(100,37),(1,0)}
  g4_fused      tests/test_gemma4_kernels_gpu.py:63-80    nH 8, kv_len 11, scale 1.0,
                (hd, start) in {(256,0),(512,0),(256,3),(512,5)}
  attn101       tests/test_kernels_dsl_parity.py:726-741  seed 121, nH 8, kvH 1, q-norm with
                random gain and random cos/sin tables, (hd, key_len) in {(256,90),(512,90)}
  g4e2b_decode  BASELINE config 2 shape at small T: nH 8, kvH 2, hd 256, gains ~N(1,0.1),
                RoPE theta 1e4 at p = T-1, window 40 and global
  prefill       BASELINE config 3 shape at small S with start_pos > 0 (continuation),
                nH 4, kvH 2, window 16 and global
  kv_write      kvnorm / kvnorm_b rows (kernels_dsl.py:573-618, 1789-1834) incl. input srq

numpy is used only to draw inputs and to store arrays. Input caches are stored
as float16 (values exactly representable), which is the build's cache type.
"""
from __future__ import annotations

import math
import os
import struct

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
EPS = 1e-6


# ---------------- pure-Python float64 restatement -------------------------
def py_rms(x, eps=EPS):
    return 1.0 / math.sqrt(sum(v * v for v in x) / len(x) + eps)


def py_norm(x, w=None, eps=EPS):
    r = py_rms(x, eps)
    return [x[i] * r * (1.0 if w is None else w[i]) for i in range(len(x))]


def py_rope(x, c, s):
    half = len(x) // 2
    a, b = x[:half], x[half:]
    return [a[i] * c[i] - b[i] * s[i] for i in range(half)] + \
           [b[i] * c[i] + a[i] * s[i] for i in range(half)]


def py_attend(qv, keys, vals, lo, hi, scale):
    """softmax over keys j in [lo, hi) of scale*q.k_j, then sum p_j v_j (float64)."""
    sc = [scale * sum(qv[d] * keys[j][d] for d in range(len(qv))) for j in range(lo, hi)]
    m = max(sc)
    e = [math.exp(v - m) for v in sc]
    z = sum(e)
    hd = len(vals[0])
    out = [0.0] * hd
    for t, j in enumerate(range(lo, hi)):
        p = e[t] / z
        vj = vals[j]
        for d in range(hd):
            out[d] += p * vj[d]
    return out


def py_f16(x):
    """IEEE binary16 round-to-nearest-even via struct's 'e' format (no numpy)."""
    return [struct.unpack("<e", struct.pack("<e", val))[0] for val in x]


def py_range(p, window):
    hi = p + 1
    return (max(0, hi - window) if window > 0 else 0), hi


def py_tables(positions, hd, theta, cutoff=None):
    half = hd // 2
    cutoff = half if cutoff is None else cutoff
    cs, ss = [], []
    for p in positions:
        c, s = [], []
        for i in range(half):
            inv = theta ** (-2.0 * i / hd) if i < cutoff else 0.0
            c.append(math.cos(p * inv))
            s.append(math.sin(p * inv))
        cs.append(c)
        ss.append(s)
    return cs, ss


def tl(a):
    return np.asarray(a, np.float64).tolist()


# ---------------- cases ----------------------------------------------------
def case_g3_fused():
    rng = np.random.default_rng(1234)
    nH, hd, T = 4, 256, 100
    q = rng.standard_normal((nH, hd), dtype=np.float32)
    k = rng.standard_normal((T, 1, hd), dtype=np.float32).astype(np.float16)
    v = rng.standard_normal((T, 1, hd), dtype=np.float32).astype(np.float16)
    K, V, Q = [r[0] for r in tl(k)], [r[0] for r in tl(v)], tl(q)
    cases = [(10, 0), (100, 0), (100, 37), (1, 0)]
    exp = np.zeros((len(cases), nH, hd), np.float64)
    for ci, (kv_len, start) in enumerate(cases):
        for h in range(nH):
            exp[ci, h] = py_attend(Q[h], K, V, start, kv_len, 1.0 / math.sqrt(hd))
    window = np.array([(kv_len - start) if start > 0 else 0 for kv_len, start in cases], np.int32)
    np.savez(os.path.join(HERE, "g3_fused.npz"), q=q, k=k, v=v,
             key_len=np.array([c[0] for c in cases], np.int32), window=window,
             scale=np.float64(1.0 / math.sqrt(hd)), expected=exp.astype(np.float32))


def case_g4_fused():
    rng = np.random.default_rng(1234)
    nH, T = 8, 11
    out = {}
    for hd, start in [(256, 0), (512, 0), (256, 3), (512, 5)]:
        q = rng.standard_normal((nH, hd), dtype=np.float32)
        k = rng.standard_normal((16, 1, hd), dtype=np.float32).astype(np.float16)
        v = rng.standard_normal((16, 1, hd), dtype=np.float32).astype(np.float16)
        K, V, Q = [r[0] for r in tl(k)], [r[0] for r in tl(v)], tl(q)
        exp = [py_attend(Q[h], K, V, start, T, 1.0) for h in range(nH)]
        tag = f"hd{hd}_s{start}"
        out.update({f"{tag}_q": q, f"{tag}_k": k, f"{tag}_v": v,
                    f"{tag}_window": np.int32(T - start if start else 0),
                    f"{tag}_expected": np.asarray(exp, np.float32)})
    np.savez(os.path.join(HERE, "g4_fused.npz"), key_len=np.int32(T), **out)


def case_attn101():
    out = {}
    for hd, key_len in [(256, 90), (512, 90)]:
        rng = np.random.default_rng(121)
        nH, half = 8, hd // 2
        q = rng.standard_normal((nH, hd)).astype(np.float32)
        w = rng.standard_normal(hd).astype(np.float32)
        cos = rng.standard_normal(half).astype(np.float32)
        sin = rng.standard_normal(half).astype(np.float32)
        k = rng.standard_normal((key_len, 1, hd)).astype(np.float32).astype(np.float16)
        v = rng.standard_normal((key_len, 1, hd)).astype(np.float32).astype(np.float16)
        K, V, W, C, S = [r[0] for r in tl(k)], [r[0] for r in tl(v)], tl(w), tl(cos), tl(sin)
        exp = []
        for h in range(nH):
            qh = py_rope(py_norm(tl(q[h]), W), C, S)
            exp.append(py_attend(qh, K, V, 0, key_len, 1.0))
        tag = f"hd{hd}_len{key_len}"
        out.update({f"{tag}_q": q, f"{tag}_w": w, f"{tag}_cos": cos, f"{tag}_sin": sin,
                    f"{tag}_k": k, f"{tag}_v": v, f"{tag}_expected": np.asarray(exp, np.float32)})
    np.savez(os.path.join(HERE, "attn101.npz"), out_q=np.float64(0.014886821620166302), **out)


def case_g4e2b_decode():
    rng = np.random.default_rng(2)
    nH, kvH, hd, T = 8, 2, 256, 96
    q = rng.standard_normal((nH, hd)).astype(np.float32)
    w = (1.0 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    k = rng.standard_normal((T, kvH, hd)).astype(np.float32).astype(np.float16)
    v = rng.standard_normal((T, kvH, hd)).astype(np.float32).astype(np.float16)
    cs, ss = py_tables([T - 1], hd, 1e4)
    cos, sin = np.asarray(cs[0], np.float32), np.asarray(ss[0], np.float32)
    W, C, S = tl(w), tl(cos), tl(sin)
    out = {}
    for window in (0, 40):
        lo, hi = py_range(T - 1, window)
        exp = []
        for h in range(nH):
            kh = h // (nH // kvH)
            K = [row[kh] for row in tl(k)]
            V = [row[kh] for row in tl(v)]
            qh = py_rope(py_norm(tl(q[h]), W), C, S)
            exp.append(py_attend(qh, K, V, lo, hi, 1.0))
        out[f"expected_w{window}"] = np.asarray(exp, np.float32)
    np.savez(os.path.join(HERE, "g4e2b_decode.npz"), q=q, w=w, k=k, v=v, cos=cos, sin=sin,
             key_len=np.int32(T), n_kv_heads=np.int32(kvH), **out)


def case_prefill():
    rng = np.random.default_rng(5)
    S, start, nH, kvH, hd = 24, 8, 4, 2, 256
    T = start + S
    q = (0.5 * rng.standard_normal((S, nH, hd))).astype(np.float32)
    w = (1.0 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    k = rng.standard_normal((T, kvH, hd)).astype(np.float32).astype(np.float16)
    v = rng.standard_normal((T, kvH, hd)).astype(np.float32).astype(np.float16)
    cs, ss = py_tables(range(start, T), hd, 1e4)
    cos, sin = np.asarray(cs, np.float32), np.asarray(ss, np.float32)
    W = tl(w)
    Kh = [[row[kh] for row in tl(k)] for kh in range(kvH)]
    Vh = [[row[kh] for row in tl(v)] for kh in range(kvH)]
    out = {}
    for window in (0, 16):
        exp = np.zeros((S, nH, hd), np.float64)
        exp16 = np.zeros((S, nH, hd), np.float64)
        q16 = np.zeros((S, nH, hd), np.float64)
        for s in range(S):
            p = start + s
            lo, hi = py_range(p, window)
            C, Sn = tl(cos[s]), tl(sin[s])
            for h in range(nH):
                kh = h // (nH // kvH)
                qh = py_rope(py_norm(tl(q[s, h]), W), C, Sn)
                exp[s, h] = py_attend(qh, Kh[kh], Vh[kh], lo, hi, 1.0)
                # qprep_b's rounding point: normalised, rotated q stored as f16
                q16[s, h] = py_f16(qh)
                exp16[s, h] = py_attend(list(q16[s, h]), Kh[kh], Vh[kh], lo, hi, 1.0)
        out[f"expected_w{window}"] = exp.astype(np.float32)
        out[f"expected_q16_w{window}"] = exp16.astype(np.float32)
        out["q16"] = q16.astype(np.float16)
    np.savez(os.path.join(HERE, "prefill.npz"), q=q, w=w, k=k, v=v, cos=cos, sin=sin,
             start_pos=np.int32(start), n_kv_heads=np.int32(kvH), **out)


def case_kv_write():
    rng = np.random.default_rng(51)
    S, kvH, hd, start = 4, 2, 256, 3
    k = rng.standard_normal((S, kvH, hd)).astype(np.float32)
    v = rng.standard_normal((S, kvH, hd)).astype(np.float32)
    g = (1.0 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    cs, ss = py_tables(range(start, start + S), hd, 1e6)
    cos, sin = np.asarray(cs, np.float32), np.asarray(ss, np.float32)
    k_in_q, v_in_q = 0.03125, 0.0625

    def srq_py(x, sc):
        if sc == 0.0:
            return x
        # round-half-to-even, as numpy's np.round and the GPU's rint
        return [max(-128.0, min(127.0, float(round(val / sc)))) * sc for val in x]

    out = {}
    for tag, kq, vq in (("plain", 0.0, 0.0), ("srq", k_in_q, v_in_q)):
        ek = np.zeros((S, kvH, hd)); ev = np.zeros((S, kvH, hd))
        for s in range(S):
            for kh in range(kvH):
                kk = srq_py(tl(k[s, kh]), kq)
                vv = srq_py(tl(v[s, kh]), vq)
                ek[s, kh] = py_rope(py_norm(kk, tl(g)), tl(cos[s]), tl(sin[s]))
                ev[s, kh] = py_norm(vv)
        out[f"k_{tag}"] = ek.astype(np.float32)
        out[f"v_{tag}"] = ev.astype(np.float32)
    np.savez(os.path.join(HERE, "kv_write.npz"), k=k, v=v, g=g, cos=cos, sin=sin,
             start_pos=np.int32(start), k_in_q=np.float64(k_in_q), v_in_q=np.float64(v_in_q), **out)


def main():
    for f in (case_g3_fused, case_g4_fused, case_attn101, case_g4e2b_decode, case_prefill,
              case_kv_write):
        f()
        print("wrote", f.__name__)


if __name__ == "__main__":
    main()
