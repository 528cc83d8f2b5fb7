"""The exported model format (weights.bin + manifest.json) and the attention block driven by
its per-layer schedule.

Reference: gemma4_150/export.py:99-181 writes the pair; gemma4_150/runner.py:55-59 reads
it, :275-291 builds the per-step RoPE rows and attention params from the layer entries,
:344-357 allocates one K/V cache per non-shared layer and :373-441 runs each layer's
attention block (qkv_70 -> kvnorm -> attn_101 with OUT_Q = o_in). The batched prefill
does the same per layer (prefill_gpu.py:327-354: dq_f16 + GEMM for q/k/v, kvnorm_b with
srq(k_out / v_out), attention).

Format (export.py:37-53, 161-181):
  * weights.bin: the tensors back to back, each padded to a multiple of 4 bytes;
  * manifest.json: {"config": {H, nL, nH, vocab, window, ...}, "layers": [{index,
    sliding, head_dim, q_dim, intermediate, shared, kv_source, rope_theta, rope_cutoff,
    scales: {qkv_in, q_out, o_in, k_out, v_out, ...}}], "tensors": {name: {off, len,
    dtype in u8/u32/f32/f16, shape}}, "bytes": total}.
  The attention block reads per layer L: L{L}.q_norm (f32 [hd]); L{L}.q_bits (u32, 4-bit
  rows [q_dim][H/8]); on a non-shared layer L{L}.k_norm, L{L}.k_bits, L{L}.v_bits and
  L{L}.qkv_scales (f32 [q_dim + 2 kv_dim]); on a KV-sharing layer L{L}.q_scale (f32
  [q_dim]) and the caches of layer kv_source.

Everything here is host-side bookkeeping: tensors are read from a read-only memory map,
validated, and uploaded once; every computation runs in libg4attn on the device.
"""
from __future__ import annotations

import json
import os
from dataclasses import dataclass, field

import numpy as np
import torch

from . import attention as A
from . import projection as P

__all__ = ["DTYPES", "LayerSpec", "Manifest", "ManifestError", "load_manifest", "AttentionStack"]

DTYPES = {"u8": np.uint8, "u32": np.uint32, "f32": np.float32, "f16": np.float16}


class ManifestError(ValueError):
    """The manifest and weights.bin do not describe a consistent model."""


@dataclass(frozen=True)
class LayerSpec:
    """One entry of manifest["layers"] (export.py:161-166)."""
    index: int
    sliding: bool
    head_dim: int
    q_dim: int
    intermediate: int
    shared: bool
    kv_source: int
    rope_theta: float
    rope_cutoff: int
    scales: dict = field(default_factory=dict)

    @property
    def n_q_heads(self) -> int:
        return self.q_dim // self.head_dim


class Manifest:
    """A parsed manifest.json over a read-only memory map of weights.bin."""

    def __init__(self, meta: dict, blob: np.ndarray, path: str = ""):
        self.path = path
        self.meta = meta
        self.blob = blob
        try:
            self.config = dict(meta["config"])
            self.tensors = dict(meta["tensors"])
            layers = meta["layers"]
        except (KeyError, TypeError) as e:
            raise ManifestError(f"manifest lacks {e}") from None
        self._check_tensors()
        self.layers = [self._layer(i, s) for i, s in enumerate(layers)]
        self._check_layers()

    # ---- validation
    def _check_tensors(self):
        size = self.blob.size
        if self.meta.get("bytes", size) != size:
            raise ManifestError(f"manifest says {self.meta['bytes']} bytes, weights.bin holds {size}")
        for name, t in self.tensors.items():
            try:
                off, n, dt, shape = int(t["off"]), int(t["len"]), t["dtype"], [int(x) for x in t["shape"]]
            except (KeyError, TypeError, ValueError):
                raise ManifestError(f"tensor {name}: malformed entry {t!r}") from None
            if dt not in DTYPES:
                raise ManifestError(f"tensor {name}: unknown dtype {dt!r}")
            if off < 0 or off % 4 or off + n > size:
                raise ManifestError(f"tensor {name}: [{off}, {off + n}) is not a 4-byte aligned range "
                                    f"of the {size}-byte file")
            if int(np.prod(shape, dtype=np.int64)) * np.dtype(DTYPES[dt]).itemsize != n:
                raise ManifestError(f"tensor {name}: {n} bytes do not hold {dt} {shape}")

    def _layer(self, i, s) -> LayerSpec:
        try:
            spec = LayerSpec(int(s["index"]), bool(s["sliding"]), int(s["head_dim"]), int(s["q_dim"]),
                             int(s["intermediate"]), bool(s["shared"]), int(s["kv_source"]),
                             float(s["rope_theta"]), int(s["rope_cutoff"]),
                             {k: float(v) for k, v in s.get("scales", {}).items()})
        except (KeyError, TypeError, ValueError) as e:
            raise ManifestError(f"layer {i}: malformed entry ({e})") from None
        if spec.index != i:
            raise ManifestError(f"layer {i} has index {spec.index}")
        return spec

    def _check_layers(self):
        nL = int(self.config.get("nL", len(self.layers)))
        if nL != len(self.layers):
            raise ManifestError(f"config.nL = {nL} but {len(self.layers)} layer entries")
        H = self.hidden
        for s in self.layers:
            if s.head_dim % 2 or s.q_dim % s.head_dim:
                raise ManifestError(f"layer {s.index}: q_dim {s.q_dim} is not a multiple of head_dim {s.head_dim}")
            if not 0 <= s.rope_cutoff <= s.head_dim // 2:
                raise ManifestError(f"layer {s.index}: rope_cutoff {s.rope_cutoff} outside [0, head_dim/2]")
            src = self.layers[s.kv_source] if 0 <= s.kv_source < len(self.layers) else None
            if s.shared:
                # a KV-sharing layer reads an earlier, non-shared layer's caches of the same
                # geometry (export.py:107: the last non-shared layer of the same kind)
                if src is None or src.shared or s.kv_source >= s.index or src.head_dim != s.head_dim:
                    raise ManifestError(f"layer {s.index}: kv_source {s.kv_source} is not an earlier "
                                        f"non-shared layer of head_dim {s.head_dim}")
                self._need(f"L{s.index}.q_scale", "f32", (s.q_dim,))
            else:
                if s.kv_source != s.index:
                    raise ManifestError(f"layer {s.index}: a non-shared layer must be its own kv_source")
                kv = self.kv_dim(s.index)
                if kv % s.head_dim:
                    raise ManifestError(f"layer {s.index}: kv_dim {kv} not a multiple of head_dim")
                self._need(f"L{s.index}.k_norm", "f32", (s.head_dim,))
                self._need(f"L{s.index}.qkv_scales", "f32", (s.q_dim + 2 * kv,))
                self._need(f"L{s.index}.v_bits", "u32", (kv * H // 8,))
            self._need(f"L{s.index}.q_norm", "f32", (s.head_dim,))
            self._need(f"L{s.index}.q_bits", "u32", (s.q_dim * H // 8,))

    def _need(self, name, dtype, n_elems):
        t = self.tensors.get(name)
        if t is None:
            raise ManifestError(f"missing tensor {name}")
        if t["dtype"] != dtype or int(np.prod(t["shape"], dtype=np.int64)) != int(np.prod(n_elems)):
            raise ManifestError(f"tensor {name}: {t['dtype']} {t['shape']}, expected {dtype} of "
                                f"{int(np.prod(n_elems))} elements")

    # ---- access
    @property
    def hidden(self) -> int:
        return int(self.config["H"])

    @property
    def window(self) -> int:
        return int(self.config.get("window", 0))

    def tensor(self, name: str) -> np.ndarray:
        """Read-only view of a tensor in its dtype and shape (no copy)."""
        t = self.tensors.get(name)
        if t is None:
            raise KeyError(name)
        raw = self.blob[int(t["off"]):int(t["off"]) + int(t["len"])]
        return raw.view(DTYPES[t["dtype"]]).reshape(t["shape"])

    def kv_dim(self, L: int) -> int:
        """Output rows of layer L's k (and v) projection: the source layer's k_bits hold
        kv_dim 4-bit rows of H values."""
        src = self.layers[L].kv_source
        t = self.tensors.get(f"L{src}.k_bits")
        if t is None:
            raise ManifestError(f"missing tensor L{src}.k_bits")
        words = int(np.prod(t["shape"], dtype=np.int64))
        if (words * 8) % self.hidden:
            raise ManifestError(f"L{src}.k_bits: {words} words are not whole 4-bit rows of {self.hidden}")
        return words * 8 // self.hidden

    def n_kv_heads(self, L: int) -> int:
        return self.kv_dim(L) // self.layers[L].head_dim

    def attn_config(self, L: int) -> A.AttnConfig:
        """The kernels' per-layer constants: heads from q_dim / kv rows, the sliding window of
        config.window on sliding layers (runner.py:290), scale 1.0 (reference.py:162) and
        the output srq step o_in (runner.py:434)."""
        s = self.layers[L]
        return A.AttnConfig(s.n_q_heads, self.n_kv_heads(L), s.head_dim,
                            self.window if s.sliding else 0, 1.0, 1e-6, s.scales.get("o_in", 0.0))

    def rope_key(self, L: int):
        """(head_dim, theta, cutoff): layers sharing it share RoPE tables (runner.py:280-282)."""
        s = self.layers[L]
        return (s.head_dim, s.rope_theta, s.rope_cutoff)


def load_manifest(model_dir) -> Manifest:
    """Read <model_dir>/manifest.json and memory-map <model_dir>/weights.bin (runner.py:55-59)."""
    model_dir = os.fspath(model_dir)
    try:
        with open(os.path.join(model_dir, "manifest.json")) as f:
            meta = json.load(f)
    except (OSError, ValueError) as e:
        raise ManifestError(f"cannot read manifest.json in {model_dir}: {e}") from None
    wpath = os.path.join(model_dir, "weights.bin")
    try:
        size = os.path.getsize(wpath)
    except OSError as e:
        raise ManifestError(f"cannot read weights.bin in {model_dir}: {e}") from None
    blob = np.memmap(wpath, np.uint8, "r") if size else np.zeros(0, np.uint8)
    return Manifest(meta, blob, model_dir)


class AttentionStack:
    """The attention block of every layer, driven by the manifest's schedule on one GPU.

    Owns one f16 K/V cache [max_seq][kvH][hd] per non-shared layer; a KV-sharing layer
    reads its kv_source's caches and writes none (runner.py:344-357, 378-380). Weights
    (norm gains, packed q/k/v rows and their scales) are uploaded once. RoPE rows come
    from one table per (head_dim, theta, cutoff), pairs at or past the cutoff identity
    (runner.py:283-289).
    """

    def __init__(self, man: Manifest, max_seq: int, device="cuda"):
        self.man = man
        self.max_seq = int(max_seq)
        self.device = device
        dev = lambda name: torch.from_numpy(np.array(man.tensor(name))).to(device)  # noqa: E731
        self.w = {}
        for s in man.layers:
            L = s.index
            w = {"q_norm": dev(f"L{L}.q_norm"),
                 "q_bits": dev(f"L{L}.q_bits").view(torch.int32).reshape(-1)}
            if s.shared:
                w["scales"] = dev(f"L{L}.q_scale")
            else:
                w.update(k_norm=dev(f"L{L}.k_norm"), scales=dev(f"L{L}.qkv_scales"),
                         k_bits=dev(f"L{L}.k_bits").view(torch.int32).reshape(-1),
                         v_bits=dev(f"L{L}.v_bits").view(torch.int32).reshape(-1))
            self.w[L] = w
        self.kc, self.vc = {}, {}
        for s in man.layers:
            if not s.shared:
                shape = (self.max_seq, man.n_kv_heads(s.index), s.head_dim)
                self.kc[s.index] = torch.zeros(shape, dtype=torch.float16, device=device)
                self.vc[s.index] = torch.zeros(shape, dtype=torch.float16, device=device)
        self.rope = {}
        for s in man.layers:
            key = man.rope_key(s.index)
            if key not in self.rope:
                hd, theta, cutoff = key
                self.rope[key] = A.rope_tables(np.arange(self.max_seq), hd, theta, cutoff, device=device)
        self.dq = {}  # dequantised f16 weights for prefill, made on first use per layer
        self.ws = A.DecodeWorkspace(device)
        self.gemm_ws = P.GemmWorkspace(device)  # the K split of the prefill GEMMs

    def caches(self, L: int):
        src = self.man.layers[L].kv_source
        return self.kc[src], self.vc[src]

    def _rows(self, L, lo, hi):
        cos, sin = self.rope[self.man.rope_key(L)]
        return cos[lo:hi], sin[lo:hi]

    def decode_layer(self, L: int, pos: int, a: torch.Tensor, sum_a: torch.Tensor, out=None, pro=None):
        """Layer L's attention for one token at position pos from its normed, srq'd input a
        f32 [H] (and sum_a f32 [1]): qkv_70 -> kvnorm (non-shared layers) -> attn_101.
        Returns the srq'd attention output f32 [nH][hd] (runner.py:408-441). The KV write of
        a non-shared layer runs inside the decode call (g4a_decode_kv). pro: a norm prologue
        (decoder.norm_in) that makes a and sum_a inside the q/k/v GEMV from the previous
        layer's tail instead (a, sum_a then receive them)."""
        s, man, w = self.man.layers[L], self.man, self.w[L]
        if not 0 <= pos < self.max_seq:
            raise ValueError(f"position {pos} outside the {self.max_seq}-row caches")
        cfg = man.attn_config(L)
        kv_dim = 0 if s.shared else man.kv_dim(L)
        sc = s.scales
        q, k, v = P.qkv_gemv(a, sum_a, w["q_bits"], w["scales"], s.q_dim, kv_dim,
                             k_bits=w.get("k_bits"), v_bits=w.get("v_bits"), q_out=sc.get("q_out", 0.0),
                             k_out=sc.get("k_out", 0.0), v_out=sc.get("v_out", 0.0), pro=pro,
                             hidden=man.hidden)
        kc, vc = self.caches(L)
        cos, sin = self._rows(L, pos, pos + 1)
        kv = {} if s.shared else dict(k_new=k, v_new=v, k_gain=w["k_norm"])
        return A.decode(q.view(cfg.n_q_heads, s.head_dim), kc, vc, [pos + 1], cfg, q_gain=w["q_norm"],
                        rope_cos=cos, rope_sin=sin, out=out, workspace=self.ws, max_key_len=pos + 1, **kv)

    def _dequant(self, L):
        if L not in self.dq:
            s, man, w = self.man.layers[L], self.man, self.w[L]
            H = man.hidden
            wq = P.dequant(w["q_bits"], w["scales"], H, s.q_dim, bits=4)
            if s.shared:
                self.dq[L] = (wq, None, None)
            else:
                kv = man.kv_dim(L)
                wk = P.dequant(w["k_bits"], w["scales"][s.q_dim:], H, kv, bits=4)
                wv = P.dequant(w["v_bits"], w["scales"][s.q_dim + kv:], H, kv, bits=4)
                self.dq[L] = (wq, wk, wv)
        return self.dq[L]

    def prefill_layer(self, L: int, start_pos: int, a: torch.Tensor, out=None, trace: dict | None = None):
        """Layer L's attention for S tokens at positions start_pos.. from their normed inputs
        a f32 [S][H] (or already the GEMM operand f16(srq(a, qkv_in)) [S][H]): dequantised
        q/k/v GEMMs (q srq'd with q_out, k/v f16), kvnorm_b with srq(k_out / v_out) on
        non-shared layers, then causal prefill attention. Returns the attention output f16
        [S][nH][hd] (prefill_gpu.py:327-354). trace: gets q, kraw and vraw."""
        s, man = self.man.layers[L], self.man
        S = a.shape[0]
        if start_pos < 0 or start_pos + S > self.max_seq:
            raise ValueError(f"positions [{start_pos}, {start_pos + S}) outside the {self.max_seq}-row caches")
        cfg = man.attn_config(L)
        sc = s.scales
        wq, wk, wv = self._dequant(L)
        if a.dtype == torch.float16:  # the operand is made: the three GEMMs straight from it
            q = torch.empty(S, wq.shape[0], device=a.device, dtype=torch.float32)
            mats = [(wq, q, sc.get("q_out", 0.0))]
            kraw = vraw = None
            if wk is not None:
                kraw = torch.empty(S, wk.shape[0], device=a.device, dtype=torch.float16)
                vraw = torch.empty(S, wv.shape[0], device=a.device, dtype=torch.float16)
                mats += [(wk, kraw, None), (wv, vraw, None)]
            P.gemm16(a, mats, self.gemm_ws)
        else:
            q, kraw, vraw = P.prefill_qkv(a, wq, wk, wv, a_in_q=sc.get("qkv_in", 0.0), q_out=sc.get("q_out", 0.0),
                                          workspace=self.gemm_ws)
        if trace is not None:
            trace.update(q=q.clone(), kraw=None if kraw is None else kraw.clone(),
                         vraw=None if vraw is None else vraw.clone())
        kc, vc = self.caches(L)
        cos, sin = self._rows(L, start_pos, start_pos + S)
        if not s.shared:
            A.kv_write(kraw.view(S, cfg.n_kv_heads, s.head_dim), vraw.view(S, cfg.n_kv_heads, s.head_dim), kc, vc,
                       start_pos, A.AttnConfig(cfg.n_kv_heads, cfg.n_kv_heads, s.head_dim),
                       k_gain=self.w[L]["k_norm"], rope_cos=cos, rope_sin=sin,
                       k_in_q=sc.get("k_out", 0.0), v_in_q=sc.get("v_out", 0.0))
        return A.prefill(q.view(S, cfg.n_q_heads, s.head_dim), kc, vc, start_pos, cfg, q_gain=self.w[L]["q_norm"],
                         rope_cos=cos, rope_sin=sin, out=out, workspace=self.ws)
