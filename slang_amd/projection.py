"""Host-side q/k/v producer over libg4attn: QAT-weight projections on torch tensors.

Two layers, as in attention.py:
  * ``dequant`` / ``qkv_gemv`` / ``srqh`` / ``gemm16`` / ``proj`` / ``prefill_qkv`` -- the library operations
    with explicit keyword arguments;
  * ``dq_f16`` / ``qkv_70`` -- drop-ins for the reference dispatches of the same names,
    with their binding slots in order (gemma4_150/kernels_dsl.py:1384-1480 and
    :2101-2138; bound at runner.py:408-423 and prefill_gpu.py:186-200).

Packed weights are int32 (or uint32) tensors holding the reference's uint32 words. Every
call is asynchronous on torch's current stream; nothing is computed on the host.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from ._lib import check
from .attention import _need, _ptr, _stream

__all__ = ["dequant", "dq_f16", "qkv_gemv", "qkv_70", "proj", "srqh", "gemm16", "GemmWorkspace", "gemm16_ws_bytes",
           "gemm16_geglu",
           "prefill_qkv", "packed_bits"]

_WORDS = (torch.int32, torch.uint32)


def packed_bits(words: torch.Tensor, n_in: int, n_out: int) -> int:
    """Bit width of a packed [n_out][n_in] matrix, read off the buffer size as
    PrefillGPU._dq does (prefill_gpu.py:195-196): 2, 4 or 8."""
    nbits = words.numel() * 32 // (n_in * n_out)
    if nbits not in (2, 4, 8) or nbits * n_in * n_out != words.numel() * 32:
        raise ValueError(f"odd width for a [{n_out}x{n_in}] matrix in {words.numel()} words")
    return nbits


def dequant(words, scale, n_in: int, n_out: int, out=None, bits: int | None = None):
    """f16 [n_out][n_in] = f16(scale[o] * (q - 2^(bits-1))) (dq_f16)."""
    _need(words, "words", _WORDS)
    _need(scale, "scale", torch.float32)
    bits = packed_bits(words, n_in, n_out) if bits is None else bits
    if scale.numel() < n_out:
        raise ValueError("scale needs n_out entries")
    if out is None:
        out = torch.empty(n_out, n_in, device=words.device, dtype=torch.float16)
    _need(out, "out", torch.float16)
    if out.numel() != n_out * n_in:
        raise ValueError("out must hold n_out*n_in values")
    check(_lib.load().g4a_dequant(bits, n_in, n_out, _ptr(words), _ptr(scale), _ptr(out), _stream()))
    return out


def dq_f16(bits, scale, out, p, scale_offset: int = 0):
    """Drop-in for the dq_f16 dispatch: slots [bits, scale(+offset bytes), dst, (n_in, n_out)]
    (PrefillGPU._dq, prefill_gpu.py:186-200)."""
    n_in, n_out = int(p[0]), int(p[1])
    if scale_offset % 4:
        raise ValueError("scale offset must be a multiple of 4 bytes")
    sc = scale.view(-1)[scale_offset // 4:]
    return dequant(bits, sc, n_in, n_out, out=out)


def qkv_gemv(a, sum_a, q_bits, scales, q_dim: int, kv_dim: int = 0, k_bits=None, v_bits=None,
             q_out: float = 0.0, k_out: float = 0.0, v_out: float = 0.0,
             out_q=None, out_k=None, out_v=None, pro=None, hidden: int | None = None):
    """Decode q/k/v of one token from 4-bit rows (qkv_70). kv_dim 0: q only (KV-sharing
    layers). Returns (q, k, v); k and v are None when kv_dim is 0.

    pro: a decoder.norm_in(...) prologue (w2 given, f16 off) that makes the input in the kernel
    from the previous layer's tail (g4a_qkv_gemv_norm); a and sum_a are then None or the
    buffers that receive the made input and its sum, and hidden gives the width."""
    if pro is None:
        hidden = a.numel()
        _need(a, "a", torch.float32)
        _need(sum_a, "sum_a", torch.float32)
    elif hidden is None:
        raise ValueError("qkv_gemv with a prologue needs hidden")
    _need(scales, "scales", torch.float32)
    for t, nm, rows in ((q_bits, "q_bits", q_dim), (k_bits, "k_bits", kv_dim), (v_bits, "v_bits", kv_dim)):
        if rows:
            _need(t, nm, _WORDS)
            if t.numel() * 8 != rows * hidden:
                raise ValueError(f"{nm} must hold {rows} 4-bit rows of {hidden} values")
    if scales.numel() < q_dim + 2 * kv_dim:
        raise ValueError("scales needs q_dim + 2*kv_dim entries")
    dev = scales.device
    out_q = torch.empty(q_dim, device=dev, dtype=torch.float32) if out_q is None else out_q
    if kv_dim:
        out_k = torch.empty(kv_dim, device=dev, dtype=torch.float32) if out_k is None else out_k
        out_v = torch.empty(kv_dim, device=dev, dtype=torch.float32) if out_v is None else out_v
    for t, nm, n in ((out_q, "out_q", q_dim), (out_k, "out_k", kv_dim), (out_v, "out_v", kv_dim)):
        if n:
            _need(t, nm, torch.float32)
            if t.numel() < n:
                raise ValueError(f"{nm} needs {n} entries")
    lib = _lib.load()
    kb, vb = _ptr(k_bits if kv_dim else None), _ptr(v_bits if kv_dim else None)
    ok, ov = _ptr(out_k if kv_dim else None), _ptr(out_v if kv_dim else None)
    if pro is None:
        check(lib.g4a_qkv_gemv(hidden, q_dim, kv_dim, _ptr(a), _ptr(sum_a), _ptr(q_bits), kb, vb,
                               _ptr(scales), q_out, k_out, v_out, _ptr(out_q), ok, ov, _stream()))
    else:
        pro = _lib.G4ANormIn.from_buffer_copy(pro)  # the caller's struct stays as it was
        if a is not None:
            _need(a, "a", torch.float32)
            pro.z_out = _ptr(a)
        if sum_a is not None:
            _need(sum_a, "sum_a", torch.float32)
        check(lib.g4a_qkv_gemv_norm(hidden, q_dim, kv_dim, ctypes.byref(pro), _ptr(sum_a), _ptr(q_bits), kb, vb,
                                    _ptr(scales), q_out, k_out, v_out, _ptr(out_q), ok, ov, _stream()))
    return (out_q, out_k, out_v) if kv_dim else (out_q, None, None)


def qkv_70(a, q_bits, k_bits, v_bits, scales, sum_a, out_q, out_k, out_v, params, shared=False):
    """Drop-in for the qkv_70 dispatch with its slots in order (runner.py:416-423):
    [a, q_bits, k_bits, v_bits, scales, sum_a, out_q, out_k, out_v, (q_out, k_out, v_out, _)].
    ``shared`` is the KV-sharing layer's q-only dispatch (runner.py:416-419)."""
    q_dim = out_q.numel()
    kv_dim = 0 if shared else out_k.numel()
    qo, ko, vo = (float(x) for x in list(params)[:3])
    qkv_gemv(a, sum_a, q_bits, scales, q_dim, kv_dim, k_bits=k_bits, v_bits=v_bits,
             q_out=qo, k_out=ko, v_out=vo, out_q=out_q, out_k=out_k, out_v=out_v)


def proj(a, w_f16, a_in_q: float = 0.0, out_f32: bool = False, out_q: float = 0.0, out=None):
    """out = A . W^T for M tokens: f16(srq(a, a_in_q)) operands, f32 accumulation, f16
    result (srqh_b -> gemm_tiled), or f32 srq(result, out_q) with out_f32 (-> srq_b).

    a f32 [M][K]; w_f16 f16 [N][K]."""
    _need(a, "a", torch.float32)
    _need(w_f16, "w_f16", torch.float16)
    M, K = a.shape
    N = w_f16.shape[0]
    if w_f16.shape[1] != K:
        raise ValueError(f"w is [{N}][{w_f16.shape[1]}], a has K = {K}")
    dt = torch.float32 if out_f32 else torch.float16
    if out is None:
        out = torch.empty(M, N, device=a.device, dtype=dt)
    _need(out, "out", dt)
    gemm16(srqh(a, a_in_q), [(w_f16, out, out_q if out_f32 else None)])
    return out


def srqh(a, a_in_q: float = 0.0, out=None):
    """srqh_b (kernels_dsl.py:232-242): f16(srq(a, a_in_q)), 0 = convert only."""
    _need(a, "a", torch.float32)
    if out is None:
        out = torch.empty(a.shape, device=a.device, dtype=torch.float16)
    _need(out, "out", torch.float16)
    if out.numel() != a.numel():
        raise ValueError("out must hold as many values as a")
    check(_lib.load().g4a_srqh(a.numel(), _ptr(a), a_in_q, _ptr(out), _stream()))
    return out


class GemmWorkspace:
    """Scratch of ``gemm16(..., workspace=)``: per-tile tickets (zero between calls; a new
    buffer is allocated zeroed, and every call leaves them zero) and the f32 partial tiles of
    the K split. Calls that may run concurrently need separate workspaces.

    Unreserved, it grows on demand; a superseded buffer is kept alive, never freed, so a HIP
    graph captured over earlier calls still owns what it points at. ``reserve(nbytes)``
    allocates once and pins the buffer: a later call that needs more raises instead of
    reallocating."""

    def __init__(self, device="cuda"):
        self.device = device
        self.buf = None
        self.reserved = False
        self._retired = []

    def reserve(self, nbytes: int) -> "GemmWorkspace":
        if self.reserved:
            raise RuntimeError("workspace already reserved")
        if self.buf is None or self.buf.numel() < nbytes:
            self._grow(int(nbytes))
        self.reserved = True
        return self

    def _grow(self, nbytes: int):
        if self.buf is not None:
            self._retired.append(self.buf)
        size = max(nbytes, _lib.GEMM_TICKET_BYTES, 2 * self.buf.numel() if self.buf is not None else 0)
        self.buf = torch.zeros(size, dtype=torch.uint8, device=self.device)

    def get(self, nbytes: int) -> torch.Tensor:
        if self.buf is None or self.buf.numel() < nbytes:
            if self.reserved:
                raise RuntimeError(f"gemm workspace reserved for {self.buf.numel()} bytes; this call needs {nbytes}")
            self._grow(nbytes)
        return self.buf


def gemm16_ws_bytes(M: int, K: int, ns) -> int:
    """g4a_gemm16_ws_bytes of a gemm16 call with A [M][K] and matrices of ns rows each."""
    tab = (_lib.G4AGemmMat * len(ns))()
    for i, n in enumerate(ns):
        tab[i] = _lib.G4AGemmMat(0, 0, int(n), 0, 0.0, 1.0)
    return int(_lib.load().g4a_gemm16_ws_bytes(int(M), int(K), len(ns), tab))


def _gemm_table(a16, mats):
    _need(a16, "a16", torch.float16)
    M, K = a16.shape
    if not 1 <= len(mats) <= 3:
        raise ValueError("gemm16 takes 1 to 3 matrices")
    tab = (_lib.G4AGemmMat * len(mats))()
    for i, m in enumerate(mats):
        w, out, oq = m[:3]
        alpha = float(m[3]) if len(m) > 3 else 1.0
        _need(w, "w_f16", torch.float16)
        _need(out, "out", (torch.float16, torch.float32))
        if w.dim() != 2 or w.shape[1] != K:
            raise ValueError(f"w is {tuple(w.shape)}, a16 has K = {K}")
        if out.numel() != M * w.shape[0]:
            raise ValueError("out must hold M*N values")
        tab[i] = _lib.G4AGemmMat(w.data_ptr(), out.data_ptr(), w.shape[0], int(out.dtype == torch.float32),
                                 float(oq or 0.0), alpha)
    return M, K, tab


def gemm16(a16, mats, workspace: GemmWorkspace | None = None):
    """Up to three products sharing the f16 activation a16 [M][K], one launch (g4a_gemm16).

    mats: sequence of (w_f16 [N][K], out, out_q or None[, alpha]); out f16 [M][N] gets the f16
    GEMM result f16(alpha * sum) (gemm_tiled), out f32 [M][N] gets srq(f32(that), out_q) (srq_b).
    With a workspace, launches with too few output tiles to fill the GPU split K
    (g4a_gemm16_ws); the partial sums are added in a fixed order, so results are deterministic."""
    M, K, tab = _gemm_table(a16, mats)
    lib = _lib.load()
    if workspace is None:
        check(lib.g4a_gemm16(M, K, _ptr(a16), len(mats), tab, _stream()))
        return
    need = lib.g4a_gemm16_ws_bytes(M, K, len(mats), tab)
    ws = workspace.get(need) if need else None
    check(lib.g4a_gemm16_ws(M, K, _ptr(a16), len(mats), tab, _ptr(ws), ws.numel() if ws is not None else 0,
                            _stream()))


def gemm16_geglu(a16, w_gate, w_up, gate_q: float, up_q: float, out_q: float, out=None, gelu_lut=None):
    """The MLP's gate and up GEMMs with geglu_b in one launch (g4a_gemm16_geglu;
    prefill_gpu.py:365-371): f16 code of gelu(srq(f16(a.Wg^T), gate_q)) * srq(f16(a.Wu^T), up_q)
    on out_q's grid, [M][n], the values gemm16 + geglu16 give. gelu_lut: the layer's GELU table
    of gate_q's grid (L{L}.gelu_gate), or None for gelu_tanh."""
    _need(a16, "a16", torch.float16)
    _need(w_gate, "w_gate", torch.float16)
    _need(w_up, "w_up", torch.float16)
    M, K = a16.shape
    n = w_gate.shape[0]
    if tuple(w_gate.shape) != (n, K) or tuple(w_up.shape) != (n, K):
        raise ValueError(f"w_gate {tuple(w_gate.shape)} and w_up {tuple(w_up.shape)} must both be [n][{K}]")
    if out is None:
        out = torch.empty(M, n, device=a16.device, dtype=torch.float16)
    _need(out, "out", torch.float16)
    if out.numel() != M * n:
        raise ValueError("out must hold M*n values")
    lut = None
    if gelu_lut is not None:
        _need(gelu_lut, "gelu_lut", torch.float32)
        if gelu_lut.numel() != 256:
            raise ValueError("a GELU table holds 256 values")
        lut = _ptr(gelu_lut)
    check(_lib.load().g4a_gemm16_geglu(M, K, _ptr(a16), _ptr(w_gate), _ptr(w_up), n, float(gate_q), float(up_q),
                                       float(out_q), _ptr(out), lut, _stream()))
    return out


def prefill_qkv(a, wq_f16, wk_f16=None, wv_f16=None, a_in_q: float = 0.0, q_out: float = 0.0,
                workspace: GemmWorkspace | None = None):
    """The q/k/v block of PrefillGPU._layer (prefill_gpu.py:327-342) over dequantised weights:
    q = srq_b(gemm(srqh_b(a), wq)) f32 [S][q_dim]; kraw, vraw = gemm(...) f16 [S][kv_dim]
    (None on KV-sharing layers), ready for kvnorm_b. srqh_b runs once for the three GEMMs,
    which run as one launch (split over K with a workspace, as gemm16)."""
    S = a.shape[0]
    a16 = srqh(a, a_in_q)
    q = torch.empty(S, wq_f16.shape[0], device=a.device, dtype=torch.float32)
    mats = [(wq_f16, q, q_out)]
    if wk_f16 is None:
        gemm16(a16, mats, workspace)
        return q, None, None
    k = torch.empty(S, wk_f16.shape[0], device=a.device, dtype=torch.float16)
    v = torch.empty(S, wv_f16.shape[0], device=a.device, dtype=torch.float16)
    gemm16(a16, mats + [(wk_f16, k, None), (wv_f16, v, None)], workspace)
    return q, k, v
