"""Host-side attention entry points over libg4attn (torch tensors in, device work out).

Two layers:
  * ``decode`` / ``prefill`` / ``kv_write`` -- the library's operations on torch
    tensors with explicit keyword arguments;
  * ``attn_101`` / ``kvnorm`` / ``kvnorm_b`` / ``attn_prefill`` / ``attn_gemm`` --
    drop-ins for the reference runners' dispatches of the same names, taking the
    same binding-slot arguments in the same order (gemma4_150/kernels_dsl.py
    signatures; runner.py:424-441, prefill_gpu.py:259-354), so a runner swaps a
    ``dispatch(...)`` line for one of these calls.

torch is used for device memory and the current stream only. Every call is
asynchronous on torch's current stream. Nothing here computes attention on the
host: when libg4attn.so is missing, the first call raises.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np
import torch

from . import _lib
from ._lib import G4ACfg, check

__all__ = [
    "AttnConfig", "DecodeWorkspace", "Workspace", "decode", "prefill", "prefill_ws_bytes", "qprep", "kv_write",
    "rope_tables", "attn_101", "kvnorm", "kvnorm_b", "attn_prefill", "attn_gemm", "qprep_b",
]


@dataclass(frozen=True)
class AttnConfig:
    """Per-layer attention constants (the reference bakes them into kernel consts)."""
    n_q_heads: int
    n_kv_heads: int
    head_dim: int
    window: int = 0          # 0 = global layer
    scale: float = 1.0       # Gemma 4: 1.0 (reference.py:162); Gemma 3: 1/sqrt(hd)
    eps: float = 1e-6
    out_q: float = 0.0       # SRQ step of the output (attn_101 OUT_Q), 0 = none

    def c(self, flags: int = 0) -> G4ACfg:
        return G4ACfg(self.n_q_heads, self.n_kv_heads, self.head_dim, self.window, flags,
                      self.scale, self.eps, self.out_q)


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _need(t, name, dtype=None, dev=True):
    if t is None:
        return
    if dev and not t.is_cuda:
        raise ValueError(f"{name} must be a device tensor")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if dtype is not None and t.dtype not in (dtype if isinstance(dtype, tuple) else (dtype,)):
        raise ValueError(f"{name} must be {dtype}, got {t.dtype}")


def rope_tables(positions, head_dim: int, theta: float, cutoff: int | None = None,
                device="cuda"):
    """cos/sin f32 [len(positions)][head_dim/2]; angles in f64 then cast, pairs >= cutoff identity.

    Same construction as the runners' tables (runner.py:283-289, prefill_wgpu.py:142-153).
    """
    half = head_dim // 2
    cutoff = half if cutoff is None else cutoff
    i = np.arange(half, dtype=np.float64)
    inv = np.where(i < cutoff, 1.0 / float(theta) ** (i / half), 0.0)
    ang = np.outer(np.asarray(positions, dtype=np.float64), inv)
    cos = torch.from_numpy(np.cos(ang).astype(np.float32))
    sin = torch.from_numpy(np.sin(ang).astype(np.float32))
    return cos.to(device), sin.to(device)


class DecodeWorkspace:
    """Device scratch of the attention calls, owned by the caller as the runners own theirs
    (runner.py:102-109, prefill_gpu.py:229-256): the split-KV partials of ``decode`` (the
    reference's `partials` buffer, runner.py:367-371) and, for ``prefill``, the f16 copies of
    f32 caches, hd-512 q and the key split's partials (the role of PrefillGPU's qf16 / kf16 /
    vf16 / scores buffers).

    Needs no initialisation. Calls that may run concurrently need separate workspaces.
    Unreserved, it grows on demand (an allocation when a call needs more than it holds).
    ``reserve(nbytes)`` allocates once, up front, and pins the buffer: from then on no call
    allocates, a call that needs more raises instead of reallocating, and the buffer's
    address never changes -- what a HIP graph captured over calls on it relies on.
    """

    def __init__(self, device="cuda"):
        self.device = device
        self.buf = None
        self.reserved = False
        self._retired = []  # superseded buffers, kept alive (see get)

    def reserve(self, nbytes: int) -> "DecodeWorkspace":
        if self.reserved:
            raise RuntimeError("workspace already reserved")
        if self.buf is None or self.buf.numel() < nbytes:
            self._grow(int(nbytes))
        self.reserved = True
        return self

    def _grow(self, nbytes: int):
        # a superseded buffer is never freed: a HIP graph captured over earlier calls still
        # points at it, and freed memory could be handed to other tensors by the caching
        # allocator. Growth at least doubles, so few are ever retired.
        if self.buf is not None:
            self._retired.append(self.buf)
        size = max(nbytes, 256, 2 * self.buf.numel() if self.buf is not None else 0)
        self.buf = torch.empty(size, dtype=torch.uint8, device=self.device)

    def get(self, nbytes: int) -> torch.Tensor:
        if self.buf is None or self.buf.numel() < nbytes:
            if self.reserved:
                raise RuntimeError(f"workspace reserved for {self.buf.numel()} bytes; this call needs {nbytes} "
                                   "(reserve the largest call's size up front)")
            self._grow(nbytes)
        return self.buf


Workspace = DecodeWorkspace


def decode(q, k_cache, v_cache, key_len, cfg: AttnConfig, *, q_gain=None, rope_cos=None,
           rope_sin=None, out=None, workspace: DecodeWorkspace | None = None,
           max_key_len: int | None = None, k_new=None, v_new=None, k_gain=None,
           k_in_q: float = 0.0, v_in_q: float = 0.0):
    """Decode attention for n_seq sequences (one query each).

    q [n_seq][nH][hd] (or [nH][hd]) f32; caches [n_seq][max_seq][kvH][hd] (or
    [max_seq][kvH][hd]) f16/f32; key_len int32 device tensor [n_seq] or python ints;
    rope_cos/sin [n_seq][hd/2] (or [hd/2]) rows for each query position.
    With k_new/v_new (f32 [n_seq][kvH][hd], or [kvH][hd]) the step's KV write is fused
    in (g4a_decode_kv): those raw rows are prepared as kv_write prepares them (srq with
    k_in_q/v_in_q, k RMSNorm*k_gain + RoPE with the query's rope row, v RMSNorm) and
    stored at row key_len-1 before being attended.
    Returns out f32 shaped like q.
    """
    single = q.dim() == 2
    q3 = q.unsqueeze(0) if single else q
    kc = k_cache.unsqueeze(0) if k_cache.dim() == 3 else k_cache
    vc = v_cache.unsqueeze(0) if v_cache.dim() == 3 else v_cache
    n_seq = q3.shape[0]
    if q3.shape[1:] != (cfg.n_q_heads, cfg.head_dim):
        raise ValueError(f"q shape {tuple(q.shape)} does not match {cfg}")
    if kc.shape[0] != n_seq or kc.shape[2:] != (cfg.n_kv_heads, cfg.head_dim) or vc.shape != kc.shape:
        raise ValueError(f"cache shape {tuple(k_cache.shape)} does not match q / {cfg}")
    if kc.dtype != vc.dtype or kc.dtype not in (torch.float16, torch.float32):
        raise ValueError("k/v caches must both be float16 or both float32")
    _need(q3, "q", torch.float32)
    _need(kc, "k_cache")
    _need(vc, "v_cache")
    _need(q_gain, "q_gain", torch.float32)
    _need(rope_cos, "rope_cos", torch.float32)
    _need(rope_sin, "rope_sin", torch.float32)
    if not torch.is_tensor(key_len):
        kl = np.atleast_1d(np.asarray(key_len, np.int32))
        if kl.size != n_seq:
            raise ValueError("key_len must have one entry per sequence")
        if kl.size and kl.min() == kl.max() and kl[0] > 0:
            # one host-known length (a batch-1 decode step): no device array, the kernel
            # takes the length from max_key_len and starts loading without a memory read
            if not int(kl[0]) <= kc.shape[1]:
                raise ValueError("key_len beyond the cache length")
            max_key_len = int(kl[0])
            key_len = None
        else:
            if max_key_len is None and kl.size:
                max_key_len = int(kl.max())   # exact bound
            key_len = torch.tensor(kl, device=q.device)
    if key_len is not None:
        _need(key_len, "key_len", torch.int32)
        if key_len.numel() != n_seq:
            raise ValueError("key_len must have one entry per sequence")
    if max_key_len is None:
        max_key_len = kc.shape[1]
    if not 0 < max_key_len <= kc.shape[1]:
        raise ValueError("max_key_len must be in [1, cache length]")
    flags = _lib.KV_F32 if kc.dtype == torch.float32 else 0
    c = cfg.c(flags)
    lib = _lib.load()
    ws_bytes = lib.g4a_decode_ws_bytes(ctypes.byref(c), n_seq, max_key_len)
    if ws_bytes == 0:
        check(-1)
    ws = (workspace or DecodeWorkspace(q.device)).get(ws_bytes)
    if out is None:
        out = torch.empty_like(q3)
    _need(out, "out", torch.float32)
    if (k_new is None) != (v_new is None):
        raise ValueError("k_new and v_new go together")
    if k_new is None:
        check(lib.g4a_decode(ctypes.byref(c), n_seq, max_key_len, _ptr(key_len), _ptr(q3), _ptr(q_gain),
                             _ptr(rope_cos), _ptr(rope_sin), _ptr(kc), _ptr(vc),
                             kc.stride(0), _ptr(out), _ptr(ws), ws.numel(), ctypes.c_void_p(_stream())))
    else:
        rows = (n_seq, cfg.n_kv_heads, cfg.head_dim)
        for name, x in (("k_new", k_new), ("v_new", v_new)):
            _need(x, name, torch.float32)
            if x.numel() != n_seq * cfg.n_kv_heads * cfg.head_dim:
                raise ValueError(f"{name} must hold {rows} f32 rows")
        _need(k_gain, "k_gain", torch.float32)
        check(lib.g4a_decode_kv(ctypes.byref(c), n_seq, max_key_len, _ptr(key_len), _ptr(q3), _ptr(q_gain),
                                _ptr(rope_cos), _ptr(rope_sin), _ptr(k_new), _ptr(v_new), float(k_in_q),
                                float(v_in_q), _ptr(k_gain), _ptr(kc), _ptr(vc), kc.stride(0), _ptr(out),
                                _ptr(ws), ws.numel(), ctypes.c_void_p(_stream())))
    return out[0] if single and out.dim() == 3 else out


def _prefill_flags(kv_f32: bool, out_f32: bool, q_hilo: bool) -> int:
    return (_lib.KV_F32 if kv_f32 else 0) | (_lib.OUT_F32 if out_f32 else 0) | (_lib.Q_HILO if q_hilo else 0)


def prefill_ws_bytes(S: int, start_pos: int, cfg: AttnConfig, *, kv_f32: bool = False,
                     q_hilo: bool = False) -> int:
    """Workspace bytes a ``prefill`` call of this shape and mode uses (g4a_prefill_ws_bytes):
    0 for hd 256 on f16 caches at S long enough to run unsplit. Reserve the largest call's."""
    c = cfg.c(_prefill_flags(kv_f32, False, q_hilo))
    return int(_lib.load().g4a_prefill_ws_bytes(ctypes.byref(c), int(S), int(start_pos)))


def prefill(q, k_cache, v_cache, start_pos: int, cfg: AttnConfig, *, workspace: DecodeWorkspace,
            q_gain=None, rope_cos=None, rope_sin=None, out=None, out_dtype=torch.float16,
            q_hilo: bool = False, split: bool = True):
    """Causal prefill attention for S tokens at positions start_pos..start_pos+S-1.

    q [S][nH][hd] f32 raw; caches [>= start_pos+S][kvH][hd] f16/f32; rope_cos/sin
    [S][hd/2] rows for those positions. Returns out [S][nH][hd] (f16 by default).
    q_hilo keeps the normalised, rotated q at f32 accuracy (two f16 MFMA operands)
    instead of rounding it to f16 as qprep_b does; on f32 caches it keeps K at f32
    accuracy too (attn_prefill's form), where q in f16 converts both caches to f16 as the
    GEMM form's srqh_b does. `workspace` is the caller's scratch (prefill_ws_bytes bytes):
    f32 caches and hd 512 need it, and short prompts split long causal rows over
    workgroups through it. split=False runs the call unsplit on f16 caches: hd 256 without
    the workspace (one kernel, the q prologue fused in), hd 512 with only the workspace's
    f16 q rows (the launch long prompts take).
    """
    S = q.shape[0]
    if q.shape[1:] != (cfg.n_q_heads, cfg.head_dim):
        raise ValueError(f"q shape {tuple(q.shape)} does not match {cfg}")
    if k_cache.shape[1:] != (cfg.n_kv_heads, cfg.head_dim) or v_cache.shape != k_cache.shape:
        raise ValueError(f"cache shape {tuple(k_cache.shape)} does not match {cfg}")
    if k_cache.shape[0] < start_pos + S:
        raise ValueError(f"caches hold {k_cache.shape[0]} rows, need {start_pos + S}")
    if k_cache.dtype != v_cache.dtype or k_cache.dtype not in (torch.float16, torch.float32):
        raise ValueError("k/v caches must both be float16 or both float32")
    for t, nm in ((q, "q"), (q_gain, "q_gain"), (rope_cos, "rope_cos"), (rope_sin, "rope_sin")):
        _need(t, nm, torch.float32)
    _need(k_cache, "k_cache")
    _need(v_cache, "v_cache")
    if rope_cos is not None and rope_cos.shape != (S, cfg.head_dim // 2):
        raise ValueError("rope_cos must be [S][head_dim/2]")
    if out is None:
        out = torch.empty(q.shape, dtype=out_dtype, device=q.device)
    _need(out, "out", (torch.float16, torch.float32))
    kv32 = k_cache.dtype == torch.float32
    c = cfg.c(_prefill_flags(kv32, out.dtype == torch.float32, q_hilo))
    lib = _lib.load()
    ws_bytes = lib.g4a_prefill_ws_bytes(ctypes.byref(c), S, int(start_pos))
    if not split:
        if kv32:
            raise ValueError("split=False runs on f16 caches")
        # a workspace below the split's size (g4a_prefill_ws_bytes) but holding the f16 q
        # rows hd 512 needs runs the call unsplit
        q16 = (S * cfg.n_q_heads * cfg.head_dim * 2 + 255) // 256 * 256
        ws_bytes = 0 if cfg.head_dim == 256 else q16 * (2 if q_hilo else 1)
    ws = workspace.get(ws_bytes) if ws_bytes else None
    check(lib.g4a_prefill(ctypes.byref(c), S, int(start_pos), _ptr(q), _ptr(q_gain), _ptr(rope_cos),
                          _ptr(rope_sin), _ptr(k_cache), _ptr(v_cache), _ptr(out), _ptr(ws),
                          0 if ws is None else ws.numel(), ctypes.c_void_p(_stream())))
    return out


def qprep(q, cfg: AttnConfig, *, q_gain=None, rope_cos=None, rope_sin=None, out=None):
    """qprep_b (kernels_dsl.py:1837-1873): f16 [S][nH][hd] = f16(RoPE(RMSNorm(q) * q_gain)).

    Bit-identical to the f16 q that ``prefill`` feeds its MFMAs (without q_hilo)."""
    S = q.shape[0]
    if q.shape[1:] != (cfg.n_q_heads, cfg.head_dim):
        raise ValueError(f"q shape {tuple(q.shape)} does not match {cfg}")
    for t, nm in ((q, "q"), (q_gain, "q_gain"), (rope_cos, "rope_cos"), (rope_sin, "rope_sin")):
        _need(t, nm, torch.float32)
    if out is None:
        out = torch.empty(q.shape, dtype=torch.float16, device=q.device)
    _need(out, "out", torch.float16)
    c = cfg.c(0)
    check(_lib.load().g4a_qprep(ctypes.byref(c), S, _ptr(q), _ptr(q_gain), _ptr(rope_cos),
                                _ptr(rope_sin), _ptr(out), ctypes.c_void_p(_stream())))
    return out


def kv_write(k, v, k_cache, v_cache, start_pos: int, cfg: AttnConfig, *, k_gain=None,
             rope_cos=None, rope_sin=None, k_in_q: float = 0.0, v_in_q: float = 0.0,
             v_norm: bool = True):
    """Write S new tokens' k/v ([S][kvH][hd], f32 or f16) into cache rows start_pos.."""
    S = k.shape[0]
    if k.shape[1:] != (cfg.n_kv_heads, cfg.head_dim) or v.shape != k.shape or k.dtype != v.dtype:
        raise ValueError(f"k/v shape {tuple(k.shape)} does not match {cfg}")
    if k_cache.shape[1:] != (cfg.n_kv_heads, cfg.head_dim) or k_cache.shape[0] < start_pos + S:
        raise ValueError("cache too small or wrong shape")
    if k_cache.dtype != v_cache.dtype:
        raise ValueError("k/v caches must share a dtype")
    for t, nm in ((k, "k"), (v, "v"), (k_cache, "k_cache"), (v_cache, "v_cache")):
        _need(t, nm, (torch.float16, torch.float32))
    for t, nm in ((k_gain, "k_gain"), (rope_cos, "rope_cos"), (rope_sin, "rope_sin")):
        _need(t, nm, torch.float32)
    flags = (_lib.KV_F32 if k_cache.dtype == torch.float32 else 0) | \
            (_lib.IN_F16 if k.dtype == torch.float16 else 0) | (0 if v_norm else _lib.NO_V_NORM)
    c = cfg.c(flags)
    lib = _lib.load()
    check(lib.g4a_kv_write(ctypes.byref(c), S, int(start_pos), _ptr(k), _ptr(v), float(k_in_q),
                           float(v_in_q), _ptr(k_gain), _ptr(rope_cos), _ptr(rope_sin),
                           _ptr(k_cache), _ptr(v_cache), ctypes.c_void_p(_stream())))


# ----------------------------------------------------------------------------
# drop-ins for the reference runners' dispatches (same slot order and meaning)
# ----------------------------------------------------------------------------
def attn_101(q, q_norm, rcos, rsin, kc, vc, partials, out, params, *, head_dim, out_q=0.0):
    """attn_101 (kernels_dsl.py:1537-1749; runner.py:430-441).

    Slots [q, q_norm, cos, sin, k, v, partials, out, params]: q f32 [nH*hd];
    q_norm f32 [hd]; cos/sin f32 [hd/2] pre-offset to pos; k/v caches
    [max_seq][kvH][hd]; partials a DecodeWorkspace; out f32 [nH*hd];
    params = (seqQ=1, keyLen=pos+1, qOffset=pos, qHeads, kvHeads, window|0, 0, 0).
    """
    seq_q, key_len, q_off, qh, kvh, win = (int(x) for x in list(params)[:6])
    if seq_q != 1 or key_len != q_off + 1:
        raise ValueError("attn_101 takes one query at position keyLen-1 (seqQ=1, keyLen=qOffset+1)")
    cfg = AttnConfig(qh, kvh, head_dim, win, 1.0, 1e-6, out_q)
    maxseq = kc.numel() // (kvh * head_dim)
    kc3 = kc.view(maxseq, kvh, head_dim)
    vc3 = vc.view(maxseq, kvh, head_dim)
    decode(q.view(qh, head_dim), kc3, vc3, [key_len], cfg, q_gain=q_norm, rope_cos=rcos.view(1, -1),
           rope_sin=rsin.view(1, -1), out=out.view(1, qh, head_dim), workspace=partials)
    return out


def kvnorm(outk, outv, k_norm, rcos, rsin, kc, vc, pkv, *, head_dim, n_kv_heads=1):
    """kvnorm (kernels_dsl.py:573-618; runner.py:424-429): slots [outk, outv, k_norm, cos, sin,
    kc, vc, pkv] with pkv = (pos*kvH*hd, ...) the element offset of the cache row."""
    off = int(list(pkv)[0])
    row = n_kv_heads * head_dim
    if off % row:
        raise ValueError("pkv[0] must be a row offset (pos * kvH * hd)")
    cfg = AttnConfig(n_kv_heads, n_kv_heads, head_dim)
    maxseq = kc.numel() // row
    kv_write(outk.view(1, n_kv_heads, head_dim), outv.view(1, n_kv_heads, head_dim),
             kc.view(maxseq, n_kv_heads, head_dim), vc.view(maxseq, n_kv_heads, head_dim), off // row,
             cfg, k_gain=k_norm, rope_cos=rcos.view(1, -1), rope_sin=rsin.view(1, -1))


def kvnorm_b(kraw, vraw, k_norm, cosT, sinT, kc, vc, p, *, S, head_dim, n_kv_heads=1):
    """kvnorm_b (kernels_dsl.py:1789-1834; prefill_gpu.py:335-342): slots [kraw, vraw, k_norm,
    cosT, sinT, kc, vc, p] with p = (startPos, kScale, vScale); cosT/sinT absolute-position
    tables [max_pos][hd/2]; kraw/vraw f16 [S][kvH*hd]."""
    start, ks, vs = int(p[0]), float(p[1]), float(p[2])
    cfg = AttnConfig(n_kv_heads, n_kv_heads, head_dim)
    half = head_dim // 2
    maxseq = kc.numel() // (n_kv_heads * head_dim)
    kv_write(kraw.view(S, n_kv_heads, head_dim), vraw.view(S, n_kv_heads, head_dim),
             kc.view(maxseq, n_kv_heads, head_dim), vc.view(maxseq, n_kv_heads, head_dim), start, cfg,
             k_gain=k_norm, rope_cos=cosT.view(-1, half)[start:start + S],
             rope_sin=sinT.view(-1, half)[start:start + S], k_in_q=ks, v_in_q=vs)


def attn_prefill(q, q_norm, cosT, sinT, kc, vc, out, params, *, head_dim, workspace, out_q=0.0, q_f16=False):
    """attn_prefill (kernels_dsl.py:1950-2098; prefill_gpu.py:347-354): slots [q, q_norm, cosT,
    sinT, k, v, out, params] with params = (startPos, qH, kvH, W, S); cosT/sinT absolute tables
    [max_pos][hd/2]. `out` may be f32 (attn_prefill's own output) or f16 (attnh).

    The fused kernel keeps the normalised, rotated q in f32 (kernels_dsl.py:2007-2014) and
    reads its caches as they are, so this uses the f32-accurate q mode, and on f32 caches
    scores at f32 accuracy; q_f16=True rounds q (and f32 caches) to f16 first, as qprep_b and
    srqh_b do for the GEMM form. `workspace` is the runner-owned scratch this drop-in needs
    beyond the reference's slots (as PrefillGPU owns its qf16 / kf16 / vf16 buffers,
    prefill_gpu.py:229-256): reserve prefill_ws_bytes of the largest call once and no call
    allocates."""
    start, qh, kvh, win, S = (int(x) for x in list(params)[:5])
    cfg = AttnConfig(qh, kvh, head_dim, win, 1.0, 1e-6, out_q)
    half = head_dim // 2
    maxseq = kc.numel() // (kvh * head_dim)
    prefill(q.view(S, qh, head_dim), kc.view(maxseq, kvh, head_dim), vc.view(maxseq, kvh, head_dim),
            start, cfg, workspace=workspace, q_gain=q_norm, rope_cos=cosT.view(-1, half)[start:start + S],
            rope_sin=sinT.view(-1, half)[start:start + S], out=out.view(S, qh, head_dim), q_hilo=not q_f16)
    return out


def qprep_b(q, q_norm, cosT, sinT, qf16, p, *, S, head_dim):
    """qprep_b (kernels_dsl.py:1837-1873; prefill_gpu.py:283-285): slots [q, q_norm, cosT, sinT,
    qf16, p] with p = (startPos, qHeads); cosT/sinT absolute-position tables [max_pos][hd/2]."""
    start, qh = int(p[0]), int(p[1])
    half = head_dim // 2
    cfg = AttnConfig(qh, qh, head_dim)
    qprep(q.view(S, qh, head_dim), cfg, q_gain=q_norm, rope_cos=cosT.view(-1, half)[start:start + S],
          rope_sin=sinT.view(-1, half)[start:start + S], out=qf16.view(S, qh, head_dim))
    return qf16


def attn_gemm(q, q_norm, cosT, sinT, kc, vc, attnh, *, S, start_pos, n_q_heads, n_kv_heads,
              head_dim, window, o_in, workspace):
    """PrefillGPU._attn_gemm (prefill_gpu.py:259-313): writes attnh f16 [S][nH*hd] =
    f16(srq(softmax(qf16 . kf16^T) . vf16, o_in)) in one fused kernel (f32 caches are
    converted to f16 first, as its srqh_b does). `workspace` as for attn_prefill."""
    return attn_prefill(q, q_norm, cosT, sinT, kc, vc, attnh,
                        (start_pos, n_q_heads, n_kv_heads, window, S), head_dim=head_dim, out_q=o_in,
                        q_f16=True, workspace=workspace)
