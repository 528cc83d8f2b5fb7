"""ctypes binding of libg4attn.so (the C ABI declared in include/g4attn.h).

The library must have been built (``__graft_entry__.build()`` or
``python -m slang_amd.build``); loading fails loudly otherwise -- there is no
fallback implementation.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libg4attn.so")

# the allocation-free decode's device array (G4A_DECODE_SCRATCH_BYTES, g4attn.h)
DECODE_SCRATCH_BYTES = 8 << 20

# flags (g4attn.h)
KV_F32 = 0x1
IN_F16 = 0x2
NO_V_NORM = 0x4
OUT_F32 = 0x8
Q_HILO = 0x10

# every function include/g4attn.h declares
EXPORTS = (
    "g4a_strerror", "g4a_last_error", "g4a_version",
    "g4a_decode_ws_bytes", "g4a_decode", "g4a_decode_kv", "g4a_decode_noalloc",
    "g4a_prefill_ws_bytes", "g4a_prefill", "g4a_qprep",
    "g4a_kv_write",
    "g4a_dequant", "g4a_qkv_gemv", "g4a_qkv_gemv_norm", "g4a_srqh", "g4a_gemm16",
    "g4a_gemm16_ws_bytes", "g4a_gemm16_ws", "g4a_gemm16_geglu",
    "g4a_qgemv", "g4a_qgemv_geglu", "g4a_qgemv_gelu_mul", "g4a_gemv_f16", "g4a_rms_norm", "g4a_geglu",
    "g4a_embed", "g4a_embed_rows", "g4a_softcap_argmax_ws_bytes", "g4a_softcap_argmax",
    "g4a_rows_tail", "g4a_geglu16", "g4a_plegate16",
    "g4a_probe_sink_bytes", "g4a_probe_read", "g4a_probe_mfma",
)

# g4a_gemm16_ws: the workspace's leading ticket words (g4attn.h)
GEMM_TICKET_BYTES = 2048

# g4a_rows_tail modes (g4attn.h)
TAIL_NONE, TAIL_SRQ, TAIL_NORM, TAIL_NORM16 = 0, 1, 2, 3


class G4ACfg(ctypes.Structure):
    _fields_ = [
        ("n_q_heads", ctypes.c_uint32),
        ("n_kv_heads", ctypes.c_uint32),
        ("head_dim", ctypes.c_uint32),
        ("window", ctypes.c_uint32),
        ("flags", ctypes.c_uint32),
        ("scale", ctypes.c_float),
        ("eps", ctypes.c_float),
        ("out_q", ctypes.c_float),
    ]


class G4AGemmMat(ctypes.Structure):
    """struct g4a_gemm_mat: one product of g4a_gemm16."""
    _fields_ = [
        ("w_f16", ctypes.c_void_p),
        ("out", ctypes.c_void_p),
        ("n", ctypes.c_int),
        ("out_f32", ctypes.c_int),
        ("out_q", ctypes.c_float),
        ("alpha", ctypes.c_float),
    ]


class G4ANormIn(ctypes.Structure):
    """struct g4a_norm_in: the residual-add + norm prologue of the fused GEMVs."""
    _fields_ = [
        ("a", ctypes.c_void_p),
        ("res", ctypes.c_void_p),
        ("w1", ctypes.c_void_p),
        ("w2", ctypes.c_void_p),
        ("x_out", ctypes.c_void_p),
        ("z_out", ctypes.c_void_p),
        ("q2", ctypes.c_float),
        ("f16", ctypes.c_int),
        ("eps", ctypes.c_float),
        ("mult", ctypes.c_float),
    ]


class G4AError(RuntimeError):
    """A libg4attn call returned an error code."""

    def __init__(self, code: int, detail: str):
        super().__init__(f"g4attn error {code}: {detail}")
        self.code = code


_lib = None
P = ctypes.c_void_p


def load() -> ctypes.CDLL:
    """Load libg4attn.so once; raise if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is missing: build it with __graft_entry__.build() "
                           "(python -m slang_amd.build); there is no fallback path")
    lib = ctypes.CDLL(LIB_PATH)
    lib.g4a_strerror.restype = ctypes.c_char_p
    lib.g4a_strerror.argtypes = [ctypes.c_int]
    lib.g4a_last_error.restype = ctypes.c_char_p
    lib.g4a_last_error.argtypes = []
    lib.g4a_version.restype = ctypes.c_int
    lib.g4a_version.argtypes = []
    cfgp = ctypes.POINTER(G4ACfg)
    lib.g4a_decode_ws_bytes.restype = ctypes.c_size_t
    lib.g4a_decode_ws_bytes.argtypes = [cfgp, ctypes.c_int, ctypes.c_int]
    lib.g4a_decode.restype = ctypes.c_int
    lib.g4a_decode.argtypes = [cfgp, ctypes.c_int, ctypes.c_int, P, P, P, P, P, P, P,
                               ctypes.c_int64, P, P, ctypes.c_size_t, P]
    lib.g4a_decode_kv.restype = ctypes.c_int
    lib.g4a_decode_kv.argtypes = [cfgp, ctypes.c_int, ctypes.c_int, P, P, P, P, P, P, P, ctypes.c_float,
                                  ctypes.c_float, P, P, P, ctypes.c_int64, P, P, ctypes.c_size_t, P]
    lib.g4a_decode_noalloc.restype = ctypes.c_int
    lib.g4a_decode_noalloc.argtypes = [cfgp, ctypes.c_int, ctypes.c_int, P, P, P, P, P, P, P,
                                       ctypes.c_int64, P, P]
    lib.g4a_prefill_ws_bytes.restype = ctypes.c_size_t
    lib.g4a_prefill_ws_bytes.argtypes = [cfgp, ctypes.c_int, ctypes.c_int]
    lib.g4a_prefill.restype = ctypes.c_int
    lib.g4a_prefill.argtypes = [cfgp, ctypes.c_int, ctypes.c_int, P, P, P, P, P, P, P, P,
                                ctypes.c_size_t, P]
    lib.g4a_qprep.restype = ctypes.c_int
    lib.g4a_qprep.argtypes = [cfgp, ctypes.c_int, P, P, P, P, P, P]
    lib.g4a_kv_write.restype = ctypes.c_int
    lib.g4a_kv_write.argtypes = [cfgp, ctypes.c_int, ctypes.c_int, P, P, ctypes.c_float,
                                 ctypes.c_float, P, P, P, P, P, P]
    i, f = ctypes.c_int, ctypes.c_float
    lib.g4a_dequant.restype = ctypes.c_int
    lib.g4a_dequant.argtypes = [i, i, i, P, P, P, P]
    lib.g4a_qkv_gemv.restype = ctypes.c_int
    lib.g4a_qkv_gemv.argtypes = [i, i, i, P, P, P, P, P, P, f, f, f, P, P, P, P]
    lib.g4a_qkv_gemv_norm.restype = ctypes.c_int
    lib.g4a_qkv_gemv_norm.argtypes = [i, i, i, ctypes.POINTER(G4ANormIn), P, P, P, P, P, f, f, f, P, P, P, P]
    lib.g4a_srqh.restype = ctypes.c_int
    lib.g4a_srqh.argtypes = [i, P, f, P, P]
    lib.g4a_gemm16.restype = ctypes.c_int
    lib.g4a_gemm16.argtypes = [i, i, P, i, ctypes.POINTER(G4AGemmMat), P]
    lib.g4a_gemm16_ws_bytes.restype = ctypes.c_size_t
    lib.g4a_gemm16_ws_bytes.argtypes = [i, i, i, ctypes.POINTER(G4AGemmMat)]
    lib.g4a_gemm16_ws.restype = ctypes.c_int
    lib.g4a_gemm16_ws.argtypes = [i, i, P, i, ctypes.POINTER(G4AGemmMat), P, ctypes.c_size_t, P]
    lib.g4a_gemm16_geglu.restype = ctypes.c_int
    lib.g4a_gemm16_geglu.argtypes = [i, i, P, P, P, i, f, f, f, P, P, P]
    lib.g4a_qgemv.restype = ctypes.c_int
    lib.g4a_qgemv.argtypes = [i, i, i, P, f, P, P, f, P, P]
    lib.g4a_gemv_f16.restype = ctypes.c_int
    lib.g4a_gemv_f16.argtypes = [i, i, P, P, P, P]
    lib.g4a_rms_norm.restype = ctypes.c_int
    lib.g4a_qgemv_geglu.restype = ctypes.c_int
    npro = ctypes.POINTER(G4ANormIn)
    lib.g4a_qgemv_geglu.argtypes = [i, i, i, P, P, P, f, f, P, P, f, f, f, P, npro, P, P]
    lib.g4a_qgemv_gelu_mul.restype = ctypes.c_int
    lib.g4a_qgemv_gelu_mul.argtypes = [i, i, i, P, f, P, P, f, P, P, npro, P, P]
    lib.g4a_rms_norm.argtypes = [i, i, P, f, P, P, f, f, P, P, f, i, P, P, P]
    lib.g4a_geglu.restype = ctypes.c_int
    lib.g4a_geglu.argtypes = [i, P, P, f, P, P]
    lib.g4a_embed.restype = ctypes.c_int
    lib.g4a_embed.argtypes = [i, i, P, ctypes.c_int64, P, P, i, f, P, P]
    lib.g4a_embed_rows.restype = ctypes.c_int
    lib.g4a_embed_rows.argtypes = [i, i, P, ctypes.c_int64, P, i, P, i, f, P, P]
    lib.g4a_rows_tail.restype = ctypes.c_int
    lib.g4a_rows_tail.argtypes = [i, i, P, f, P, f, f, P, i, P, f, P, P]
    lib.g4a_geglu16.restype = ctypes.c_int
    lib.g4a_geglu16.argtypes = [i, P, P, f, f, f, P, P, P]
    lib.g4a_plegate16.restype = ctypes.c_int
    lib.g4a_plegate16.argtypes = [i, i, P, f, P, i, f, P, P, P]
    lib.g4a_softcap_argmax.restype = ctypes.c_int
    lib.g4a_softcap_argmax_ws_bytes.restype = ctypes.c_size_t
    lib.g4a_softcap_argmax_ws_bytes.argtypes = [i]
    lib.g4a_softcap_argmax.argtypes = [i, P, f, P, P, ctypes.c_size_t, P]
    lib.g4a_probe_sink_bytes.restype = ctypes.c_size_t
    lib.g4a_probe_sink_bytes.argtypes = []
    lib.g4a_probe_read.restype = ctypes.c_int
    lib.g4a_probe_read.argtypes = [P, ctypes.c_size_t, i, P, P]
    lib.g4a_probe_mfma.restype = ctypes.c_int
    lib.g4a_probe_mfma.argtypes = [i, i, P, P]
    _lib = lib
    return lib


def check(rc: int) -> None:
    if rc != 0:
        lib = load()
        raise G4AError(rc, f"{lib.g4a_strerror(rc).decode()}: {lib.g4a_last_error().decode()}")
