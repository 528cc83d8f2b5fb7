"""A synthetic model in the exported format (weights.bin + manifest.json), for the manifest
reader and the layer-schedule tests. Written the way gemma4_150/export.py:37-53 lays the
file out (tensors back to back, each padded to 4 bytes, offsets/lengths/dtype/shape in the
manifest) and with the per-layer entries of :161-181, over random weights: there is no
checkpoint to export from. Only the attention block's tensors are written.
"""
from __future__ import annotations

import json
import os

import numpy as np

from oracle.projection import pack_values

# (sliding, head_dim, rope_cutoff, shared, kv_source): two own-cache layers (a sliding
# hd-256 one and a global hd-512 one with partial RoPE), then one KV-sharing layer of each
SCHEDULE = [(True, 256, 128, False, 0), (False, 512, 64, False, 1),
            (True, 256, 128, True, 0), (False, 512, 64, True, 1)]


class _Writer:
    def __init__(self, path):
        self.f = open(path, "wb")
        self.pos = 0
        self.tensors = {}

    def put(self, name, arr, dtype):
        b = np.ascontiguousarray(arr).tobytes()
        self.f.write(b)
        self.tensors[name] = {"off": self.pos, "len": len(b), "dtype": dtype, "shape": list(arr.shape)}
        self.pos += len(b)
        pad = (-len(b)) % 4
        if pad:
            self.f.write(b"\0" * pad)
            self.pos += pad

    def close(self):
        self.f.close()


def write_model(out_dir, H=256, n_heads=4, kv_heads=1, window=64, schedule=SCHEDULE, seed=0,
                extra_odd_tensor=True):
    """Write the model; returns (manifest dict, {tensor name: array}) for the checks."""
    rng = np.random.default_rng(seed)
    os.makedirs(out_dir, exist_ok=True)
    w = _Writer(os.path.join(out_dir, "weights.bin"))
    arrays = {}

    def put(name, arr, dtype):
        arrays[name] = arr
        w.put(name, arr, dtype)

    if extra_odd_tensor:  # a u8 tensor of odd length first, so later offsets need the padding
        put("embed_q", rng.integers(0, 256, size=(3, 7), dtype=np.uint8), "u8")
    layers = []
    for L, (sliding, hd, cutoff, shared, src) in enumerate(schedule):
        q_dim, kv_dim = n_heads * hd, kv_heads * hd
        put(f"L{L}.in_norm", (1 + 0.1 * rng.standard_normal(H)).astype(np.float32), "f32")
        put(f"L{L}.q_norm", (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32), "f32")
        if not shared:
            put(f"L{L}.k_norm", (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32), "f32")
        rows = q_dim if shared else q_dim + 2 * kv_dim
        scales = (0.01 * (1 + 0.2 * rng.random(rows))).astype(np.float32)
        put(f"L{L}.q_bits", pack_values(rng.integers(0, 16, size=(q_dim, H)), 4), "u32")
        if shared:
            put(f"L{L}.q_scale", scales, "f32")
        else:
            put(f"L{L}.k_bits", pack_values(rng.integers(0, 16, size=(kv_dim, H)), 4), "u32")
            put(f"L{L}.v_bits", pack_values(rng.integers(0, 16, size=(kv_dim, H)), 4), "u32")
            put(f"L{L}.qkv_scales", scales, "f32")
        sc = {"qkv_in": 0.05, "q_out": 0.02, "o_in": 0.01, "o_out": 0.05}
        if not shared:
            sc.update(k_out=0.02, v_out=0.02)
        layers.append({"index": L, "sliding": sliding, "head_dim": hd, "q_dim": q_dim,
                       "intermediate": 4 * H, "shared": shared, "kv_source": src,
                       "rope_theta": 1e4 if sliding else 1e6, "rope_cutoff": cutoff, "scales": sc})
    w.close()
    man = {"config": {"H": H, "nL": len(schedule), "nH": n_heads, "vocab": 16, "window": window,
                      "softcap": 30.0, "ple_d": 8, "embed_scale": float(np.sqrt(H)),
                      "ple_scale": float(np.sqrt(8)), "bos": 2, "eos": 1},
           "layers": layers, "tensors": w.tensors, "bytes": w.pos}
    with open(os.path.join(out_dir, "manifest.json"), "w") as f:
        json.dump(man, f)
    return man, arrays
