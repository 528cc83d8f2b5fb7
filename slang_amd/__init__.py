"""MI355X (gfx950) Gemma 4 E2B attention hot path: decode, batched causal prefill, the
KV-cache write and the q/k/v projections that feed them, as hand-written HIP kernels in
libg4attn.so behind a C ABI (include/g4attn.h), with a thin torch/ctypes host layer
mirroring the reference runners' dispatch entry points (attn_101, kvnorm, kvnorm_b,
attn_prefill, qkv_70, dq_f16), and the exported model format (weights.bin +
manifest.json) whose per-layer schedule drives them."""
from .attention import (AttnConfig, DecodeWorkspace, Workspace, attn_101, attn_gemm, attn_prefill, decode,
                        kv_write, kvnorm, kvnorm_b, prefill, prefill_ws_bytes, qprep, qprep_b, rope_tables)
from .manifest import AttentionStack, Manifest, ManifestError, load_manifest
from .projection import (GemmWorkspace, dequant, dq_f16, gemm16, gemm16_geglu, gemm16_ws_bytes, packed_bits,
                         prefill_qkv, proj, qkv_70, qkv_gemv, srqh)

__all__ = ["AttnConfig", "DecodeWorkspace", "Workspace", "decode", "prefill", "prefill_ws_bytes", "qprep", "kv_write",
           "rope_tables", "attn_101", "kvnorm", "kvnorm_b", "attn_prefill", "attn_gemm", "qprep_b",
           "dequant", "dq_f16", "qkv_gemv", "qkv_70", "proj", "srqh", "gemm16", "GemmWorkspace", "gemm16_ws_bytes",
           "gemm16_geglu", "prefill_qkv", "packed_bits",
           "AttentionStack", "Manifest", "ManifestError", "load_manifest"]
