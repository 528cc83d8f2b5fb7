"""MI355X (gfx950) Gemma 4 E2B attention hot path: decode, batched causal prefill and the
KV-cache write, as hand-written HIP kernels in libg4attn.so behind a C ABI
(include/g4attn.h), with a thin torch/ctypes host layer mirroring the reference
runners' dispatch entry points (attn_101, kvnorm, kvnorm_b, attn_prefill)."""
from .attention import (AttnConfig, DecodeWorkspace, attn_101, attn_gemm, attn_prefill, decode,
                        kv_write, kvnorm, kvnorm_b, prefill, qprep, qprep_b, rope_tables)

__all__ = ["AttnConfig", "DecodeWorkspace", "decode", "prefill", "qprep", "kv_write", "rope_tables",
           "attn_101", "kvnorm", "kvnorm_b", "attn_prefill", "attn_gemm", "qprep_b"]
