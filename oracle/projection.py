"""CPU oracle for the q/k/v producer in front of the attention path.

TEST INFRASTRUCTURE ONLY. Nothing in the product package (slang_amd/) imports
this module. It may be imported only by tests/, by __graft_entry__.smoke() and
by bench.py's cpu_baseline leg, and there only as the checker, never as a
fallback for the GPU path.

It restates the reference's QAT projection kernels:

  * packed weights, value order and zero point .. dq_f16, gemma4_150/kernels_dsl.py:2101-2138
      value i of a row sits at bit 8*(i // (8/bits)) + bits*(i % (8/bits)) of the
      row's little-endian bytes; w = row_scale * (q - 2**(bits-1)) rounded to f16
  * decode q/k/v GEMV ........................... qkv_70, kernels_dsl.py:1384-1480
      out[o] = srq(scale[o] * (sum_i q[o][i] * a[i] - 8 * sum_a), out_q), 4-bit rows,
      q rows then k rows then v rows in one scale vector (:1436-1437, :1458-1459, :1476-1480)
  * prefill projection .......................... prefill_gpu.py:327-342:
      srqh_b (kernels_dsl.py:233-242: a -> f16(srq(a, s))), dq_f16, gemm_tiled
      (:34-136: f32 accumulation, f16(alpha * acc) output), srq_b (:246-255:
      srq(f32(c), s) for the q path)
  * srq ......................................... gemma4_150/reference.py:30-31

Pinning (tests/test_oracle_projection.py): known-answer words whose unpacked
values are written out by hand, a float64 reconstruction of dq_f16 (the
reference's own exactness check, tests/test_kernels_dsl_parity.py:785-829), a
pure-Python restatement of qkv_70's lo/hi-nibble vec4 loop, the zero-point
closed form (all values at the zero point give 0 whatever the input), and
GEMM rows against the GEMV.
"""
from __future__ import annotations

import numpy as np

from .attention import srq


def unpack_values(words, n_in, bits):
    """Unsigned values [n_out][n_in] of packed rows (dq_f16's order, kernels_dsl.py:2127-2138)."""
    assert bits in (2, 4, 8)
    words = np.ascontiguousarray(words, dtype=np.uint32)
    per_byte = 8 // bits
    row_bytes = n_in // per_byte
    by = words.view(np.uint8).reshape(-1, row_bytes)  # little-endian bytes of each row
    shifts = (bits * np.arange(per_byte)).astype(np.uint8)
    vals = (by[:, :, None] >> shifts[None, None, :]) & np.uint8((1 << bits) - 1)
    return vals.reshape(by.shape[0], n_in).astype(np.int32)


def pack_values(vals, bits):
    """Inverse of unpack_values: [n_out][n_in] unsigned values -> uint32 words."""
    vals = np.asarray(vals, np.uint32)
    n_out, n_in = vals.shape
    per_byte = 8 // bits
    v = vals.reshape(n_out, n_in // per_byte, per_byte)
    by = np.zeros(v.shape[:2], np.uint32)
    for j in range(per_byte):
        by |= v[:, :, j] << np.uint32(bits * j)
    return np.ascontiguousarray(by.astype(np.uint8)).view(np.uint32).reshape(n_out, -1)


def dequant_f16(words, scale, n_in, n_out, bits):
    """f16(scale[o] * (q - zp)) computed in f32, as dq_f16 does (kernels_dsl.py:2127-2138)."""
    q = unpack_values(words, n_in, bits)[:n_out].astype(np.float32)
    zp = np.float32(1 << (bits - 1))
    s = np.asarray(scale, np.float32)[:n_out, None]
    return (s * (q - zp)).astype(np.float16)


def qkv_gemv(a, sum_a, q_bits, k_bits, v_bits, scales, q_dim, kv_dim, q_out=0.0, k_out=0.0,
             v_out=0.0):
    """qkv_70 (kernels_dsl.py:1384-1480): three 4-bit GEMVs sharing the input a.

    Sums in float64; the srq grid step is applied to the f32 value. kv_dim 0 computes q only
    (the KV-sharing layers' dispatch, runner.py:416-419). Returns (q, k, v) f32 (k, v None
    when kv_dim is 0)."""
    a = np.asarray(a, np.float64)
    n_in = a.shape[0]
    sa = float(np.float32(sum_a))
    scales = np.asarray(scales, np.float32)

    def one(bits_, sc, n, s_out):
        qv = unpack_values(bits_, n_in, 4)[:n].astype(np.float64)
        raw = sc[:n].astype(np.float64) * (qv @ a - 8.0 * sa)
        return srq(raw.astype(np.float32), s_out)

    q = one(q_bits, scales, q_dim, q_out)
    if kv_dim == 0:
        return q, None, None
    k = one(k_bits, scales[q_dim:], kv_dim, k_out)
    v = one(v_bits, scales[q_dim + kv_dim:], kv_dim, v_out)
    return q, k, v


def proj_gemm(a, w_f16, a_in_q=0.0, out_f32=False, out_q=0.0):
    """srqh_b -> gemm_tiled (tr = 1) -> optional srq_b (prefill_gpu.py:327-342).

    a f32 [M][K]; w_f16 f16 [N][K] (dq_f16's output). The product of the f16 operands is
    accumulated in float64 and rounded to f16 (gemm_tiled's f16(alpha * acc), alpha 1);
    out_f32 applies srq(f32(c), out_q) as srq_b does."""
    ah = srq(np.asarray(a, np.float32), a_in_q).astype(np.float16)
    c = (ah.astype(np.float64) @ np.asarray(w_f16, np.float16).astype(np.float64).T).astype(np.float16)
    if not out_f32:
        return c
    return srq(c.astype(np.float32), out_q)
