"""CPU oracle for the Gemma 4 E2B attention hot path.

TEST INFRASTRUCTURE ONLY. Nothing in the product package (slang_amd/) imports
this module. It may be imported only by tests/, by __graft_entry__.smoke() and
by bench.py's cpu_baseline leg, and there only as the checker or the timed CPU
baseline, never as a fallback for the GPU path.

It restates the attention block of the reference's numpy SRQ oracle and the
semantics of the kernels the reference runners dispatch:

  * srq / rms_norm / rms_norm_noscale / rope ... gemma4_150/reference.py:30-55
  * decode attention (scale 1.0, sliding start) . gemma4_150/reference.py:146-168
  * Gemma 3 scale 1/sqrt(query_pre_attn_scalar)  gemma3/reference.py:73-86
  * GQA head map hKv = h // (nH // kvH) ......... gemma4_150/kernels_dsl.py:1581, 1985
  * attended set [max(0, p+1-W), p] ............. kernels_dsl.py:1582-1589 (decode),
                                                  :1986-1992 (attn_prefill), :1898-1908 (smax_b)
  * k RMSNorm*gain + RoPE, v RMSNorm (no gain) .. kernels_dsl.py:573-618 (kvnorm),
                                                  :1789-1834 (kvnorm_b, with srq of the inputs)
  * q -> f16 rounding before the score GEMM ..... kernels_dsl.py:1837-1873 (qprep_b)
  * RoPE tables, f64 angles cast to f32 ......... gemma4_150/runner.py:283-289,
                                                  prefill_wgpu.py:142-153

Generalisations the reference lacks but BASELINE's configs need (documented in
the build's design notes): kvH > 1, several sequences with their own key
lengths, key lengths beyond the reference's 2048 cap.

Pinning (tests/test_oracle.py): golden vectors from an independent pure-Python
float64 restatement (tests/golden/make_golden.py) on the parameter sets of the
reference's own attention tests, closed forms (uniform attention = mean of the
attended V rows, RoPE as complex rotation, softmax/merge identities) and the
invariants of tests/test_gemma4_reference.py:21-63.
"""
from __future__ import annotations

import numpy as np

EPS = 1e-6


# --------------------------------------------------------------------------
# elementwise helpers (gemma4_150/reference.py:30-55)
# --------------------------------------------------------------------------
def srq(x, s):
    """Static-range quantisation, identity when s == 0 (reference.py:30-31)."""
    if s == 0.0:
        return x
    s = np.float32(s)
    return (np.clip(np.round(x / s), -128.0, 127.0) * s).astype(np.float32)


def rms_norm(x, w, eps=EPS):
    """x / sqrt(mean(x^2) + eps) * w -- Gemma 4 scales by w, not (1 + w) (reference.py:38-39)."""
    x = np.asarray(x, np.float32)
    return (x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + np.float32(eps)) * w).astype(np.float32)


def rms_norm_noscale(x, eps=EPS):
    """RMSNorm without a gain, used on v (reference.py:42-43)."""
    x = np.asarray(x, np.float32)
    return (x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + np.float32(eps))).astype(np.float32)


def rope_inv_freq(head_dim, theta, cutoff=None, dtype=np.float64):
    """inv_i = theta^(-2i/hd) for i < half; 0 for i >= cutoff (identity pairs).

    reference.py:50-51 computes it in f32; runner.py:285-286 and
    prefill_wgpu.py:150-151 in f64. Both are offered.
    """
    half = head_dim // 2
    cutoff = half if cutoff is None else cutoff
    i = np.arange(half, dtype=dtype)
    inv = (1.0 / np.asarray(theta, dtype) ** (2.0 * i / head_dim)).astype(dtype)
    inv[cutoff:] = 0.0
    return inv


def rope_tables(positions, head_dim, theta, cutoff=None, exact=True):
    """cos/sin tables f32 [len(positions)][half].

    exact=True follows the runners (angles in f64, then cast; runner.py:283-289,
    metal_runner.py:268-283, prefill_wgpu.py:142-153) -- what the kernels are fed.
    exact=False follows reference.py:50-53 (f32 angle pos*inv).
    """
    pos = np.asarray(positions)
    if exact:
        ang = np.outer(pos.astype(np.float64), rope_inv_freq(head_dim, theta, cutoff, np.float64))
        return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    inv = rope_inv_freq(head_dim, theta, cutoff, np.float32)
    ang = pos.astype(np.float32)[:, None] * inv[None, :]
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


def apply_rope(x, cos, sin):
    """Split-half RoPE with pairs (i, i+half): [a*c - b*s, b*c + a*s] (reference.py:54-55).

    x [..., hd]; cos/sin broadcastable to [..., half].
    """
    x = np.asarray(x, np.float32)
    half = x.shape[-1] // 2
    a, b = x[..., :half], x[..., half:]
    return np.concatenate([a * cos - b * sin, b * cos + a * sin], axis=-1).astype(np.float32)


def rope(x, pos, theta, cutoff):
    """reference.py:46-55 verbatim semantics: split-half RoPE at one position, f32 angles."""
    c, s = rope_tables([pos], x.shape[-1], theta, cutoff, exact=False)
    return apply_rope(x, c[0], s[0])


# --------------------------------------------------------------------------
# mask / index logic (integer, exact)
# --------------------------------------------------------------------------
def attended_range(p, window):
    """Keys attended by the query at absolute position p: [lo, hi) = [max(0, p+1-W), p+1).

    W == 0 means global. reference.py:160-161 (start = max(0, kv_len - W) with
    kv_len = p+1); kernels_dsl.py:1582-1589, 1986-1992, 1898-1908.
    """
    hi = p + 1
    lo = max(0, hi - window) if window > 0 else 0
    return lo, hi


def kv_head_of(h, n_q_heads, n_kv_heads):
    """GQA map hKv = h / (qHeads / kvHeads) (kernels_dsl.py:1581, 1985)."""
    return h // (n_q_heads // n_kv_heads)


# --------------------------------------------------------------------------
# KV write (kvnorm / kvnorm_b)
# --------------------------------------------------------------------------
def kv_write(k, v, k_gain=None, cos=None, sin=None, *, k_in_q=0.0, v_in_q=0.0,
             v_norm=True, eps=EPS, cache_dtype=np.float16):
    """Rows a KV-cache write stores for S new tokens.

    k, v: [S][kvH][hd] (f32, or f16 as kvnorm_b reads them). cos/sin: [S][half]
    rows for the tokens' absolute positions, or None for no RoPE.
    k <- rope(rms_norm(srq(k, k_in_q)) * gain); v <- rms_norm_noscale(srq(v, v_in_q)).
    kernels_dsl.py:573-618 (decode kvnorm), :1789-1834 (kvnorm_b: srq first);
    reference.py:155-156. Returns (k_rows, v_rows) cast to cache_dtype.
    """
    k = srq(np.asarray(k, np.float32), k_in_q)
    v = srq(np.asarray(v, np.float32), v_in_q)
    if k_gain is not None:
        k = rms_norm(k, np.asarray(k_gain, np.float32), eps)
    if cos is not None:
        k = apply_rope(k, np.asarray(cos, np.float32)[:, None, :], np.asarray(sin, np.float32)[:, None, :])
    if v_norm:
        v = rms_norm_noscale(v, eps)
    return k.astype(cache_dtype), v.astype(cache_dtype)


# --------------------------------------------------------------------------
# attention cores
# --------------------------------------------------------------------------
def _prep_q(q, q_gain, cos, sin, eps):
    """q RMSNorm * gain then RoPE (reference.py:150-151; kernels_dsl.py:1593-1615)."""
    q = np.asarray(q, np.float32)
    if q_gain is not None:
        q = rms_norm(q, np.asarray(q_gain, np.float32), eps)
    if cos is not None:
        q = apply_rope(q, cos, sin)
    return q


def _softmax_pv(scores, vals):
    """max-subtracted softmax then P.V, f32 (reference.py:165-167)."""
    scores = scores - scores.max(-1, keepdims=True)
    probs = np.exp(scores)
    probs /= probs.sum(-1, keepdims=True)
    return (probs @ vals).astype(np.float32)


def decode_attention(q, k_cache, v_cache, key_len, n_kv_heads, *, q_gain=None, cos=None,
                     sin=None, window=0, scale=1.0, eps=EPS, out_q=0.0):
    """One decode query at position p = key_len-1 against a KV cache.

    q [nH][hd] f32 (raw: q RMSNorm*gain and RoPE are applied here, as attn_101
    does, kernels_dsl.py:1593-1615). k_cache/v_cache [>=key_len][kvH][hd] in the
    stored dtype (upcast to f32). cos/sin [half] for position p, or None.
    Masked scores (-1e9 before key `start`) follow reference.py:159-167; the
    optional output SRQ is attn_101's OUT_Q (kernels_dsl.py:1749; reference.py:168).
    Returns [nH][hd] f32.
    """
    q = _prep_q(q, q_gain, None if cos is None else np.asarray(cos, np.float32)[None, :],
                None if sin is None else np.asarray(sin, np.float32)[None, :], eps)
    nH, hd = q.shape
    lo, hi = attended_range(key_len - 1, window)
    out = np.empty((nH, hd), np.float32)
    for h in range(nH):
        kh = kv_head_of(h, nH, n_kv_heads)
        keys = np.asarray(k_cache[:hi, kh], np.float32)
        vals = np.asarray(v_cache[:hi, kh], np.float32)
        scores = (keys @ q[h]) * np.float32(scale)
        if lo > 0:
            scores[:lo] = -1e9
        out[h] = _softmax_pv(scores[None, :], vals)[0]
    return srq(out, out_q)


def decode_attention_batched(q, k_caches, v_caches, key_lens, n_kv_heads, **kw):
    """Several independent sequences: q [B][nH][hd]; caches [B][T][kvH][hd].

    Per-sequence cos/sin may be passed as [B][half] arrays.
    """
    cos, sin = kw.pop("cos", None), kw.pop("sin", None)
    outs = []
    for b in range(len(key_lens)):
        outs.append(decode_attention(q[b], k_caches[b], v_caches[b], int(key_lens[b]), n_kv_heads,
                                     cos=None if cos is None else cos[b],
                                     sin=None if sin is None else sin[b], **kw))
    return np.stack(outs)


def prefill_attention(q, k_cache, v_cache, start_pos, n_kv_heads, *, q_gain=None, cos=None,
                      sin=None, window=0, scale=1.0, eps=EPS, out_q=0.0, q_round_f16=True,
                      kv_round_f16=False, block=256):
    """Batched causal attention for S prompt tokens at positions start_pos..start_pos+S-1.

    q [S][nH][hd] f32 raw; cos/sin [S][half] rows for those absolute positions
    (attn_prefill indexes its tables by absolute position, kernels_dsl.py:2007-2014).
    k_cache/v_cache [>= start_pos+S][kvH][hd] already hold every token's k/v.
    q_round_f16 mirrors qprep_b's f16 rounding of the normalised, rotated q
    (kernels_dsl.py:1872-1873), which is also what the MFMA kernel consumes.
    kv_round_f16 mirrors the GEMM form's conversion of the caches to f16 before its
    products (srqh_b with step 0 on kc and vc, prefill_gpu.py:286-288; kernels_dsl.py:
    232-242): a no-op on f16 caches, round-to-nearest-even on f32 ones. The fused form
    (attn_prefill, kernels_dsl.py:1950-2098) reads its f32 caches as they are: both
    roundings off.
    Each query attends [max(0, p+1-W), p] (kernels_dsl.py:1986-1992).
    Query rows are processed in blocks to bound memory at long S. Returns [S][nH][hd] f32.
    """
    q = np.asarray(q, np.float32)
    S, nH, hd = q.shape
    qn = _prep_q(q, q_gain, None if cos is None else np.asarray(cos, np.float32)[:, None, :],
                 None if sin is None else np.asarray(sin, np.float32)[:, None, :], eps)
    if q_round_f16:
        qn = qn.astype(np.float16).astype(np.float32)
    T = start_pos + S
    out = np.empty((S, nH, hd), np.float32)
    G = nH // n_kv_heads
    for kh in range(n_kv_heads):
        keys = np.asarray(k_cache[:T, kh], np.float32)
        vals = np.asarray(v_cache[:T, kh], np.float32)
        if kv_round_f16:
            keys = keys.astype(np.float16).astype(np.float32)
            vals = vals.astype(np.float16).astype(np.float32)
        for s0 in range(0, S, block):
            s1 = min(S, s0 + block)
            pos = start_pos + np.arange(s0, s1)
            k_lo = attended_range(int(pos[0]), window)[0]
            k_hi = int(pos[-1]) + 1
            kk = keys[k_lo:k_hi]
            vv = vals[k_lo:k_hi]
            j = np.arange(k_lo, k_hi)
            lo = np.array([attended_range(int(p), window)[0] for p in pos])
            allowed = (j[None, :] <= pos[:, None]) & (j[None, :] >= lo[:, None])
            for hh in range(G):
                h = kh * G + hh
                sc = (qn[s0:s1, h] @ kk.T) * np.float32(scale)
                sc = np.where(allowed, sc, np.float32(-1e9)).astype(np.float32)
                out[s0:s1, h] = _softmax_pv(sc, vv)
    return srq(out, out_q)


# --------------------------------------------------------------------------
# split-KV merge identity (kernels_dsl.py:1717-1749)
# --------------------------------------------------------------------------
def partial_attention(q_prepped, keys, vals, scale=1.0):
    """(m, l, o) of one key chunk for one head: m = max s, l = sum e^(s-m), o = sum e^(s-m) v."""
    s = (np.asarray(keys, np.float64) @ np.asarray(q_prepped, np.float64)) * scale
    m = s.max()
    e = np.exp(s - m)
    return m, e.sum(), e @ np.asarray(vals, np.float64)


def merge_partials(parts):
    """Flash-decoding merge: m = max m_c, l = sum l_c e^(m_c-m), o = sum o_c e^(m_c-m) / l."""
    m = max(p[0] for p in parts)
    l = sum(p[1] * np.exp(p[0] - m) for p in parts)
    o = sum(p[2] * np.exp(p[0] - m) for p in parts)
    return o / l
