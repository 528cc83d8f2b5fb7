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

from oracle.decoder import gelu_lut
from oracle.projection import pack_values

# (sliding, head_dim, rope_cutoff, shared, kv_source): two own-cache layers (a sliding
# hd-256 one and a global hd-512 one with partial RoPE), then one KV-sharing layer of each
SCHEDULE = [(True, 256, 128, False, 0), (False, 512, 64, False, 1),
            (True, 256, 128, True, 0), (False, 512, 64, True, 1)]


class _Writer:
    """Lays tensors out as export.py's Writer does; the bytes go to the file at close(), so a
    tensor's contents may still be set after later tensors were put (its size may not)."""

    def __init__(self, path):
        self.path = path
        self.pos = 0
        self.tensors = {}
        self.arrays = []

    def put(self, name, arr, dtype):
        a = np.ascontiguousarray(arr)
        self.tensors[name] = {"off": self.pos, "len": a.nbytes, "dtype": dtype, "shape": list(a.shape)}
        self.arrays.append((self.pos, a))
        self.pos += a.nbytes + (-a.nbytes) % 4

    def close(self):
        with open(self.path, "wb") as f:
            for off, a in self.arrays:
                f.seek(off)
                f.write(a.tobytes())
            f.truncate(self.pos)


def write_model(out_dir, H=256, n_heads=4, kv_heads=1, window=64, schedule=SCHEDULE, seed=0,
                extra_odd_tensor=True, full=False, vocab=512, ple_d=32, mlp_bits=(4, 2, 4, 2), gelu_tables=True):
    """Write the model; returns (manifest dict, {tensor name: array}) for the checks.
    full: also the tensors of the rest of the decoder (export.py:86-98, 113-161): the
    embedding and per-layer-embedding tables, lm_head blocks, o_proj, the MLP (layer L's
    gate/up/down rows mlp_bits[L]-bit), the int8 per-layer-embedding linears, the norms and
    (gelu_tables) the per-layer GELU tables of the gate grids."""
    rng = np.random.default_rng(seed)
    os.makedirs(out_dir, exist_ok=True)
    w = _Writer(os.path.join(out_dir, "weights.bin"))
    arrays = {}

    def put(name, arr, dtype):
        arrays[name] = arr
        w.put(name, arr, dtype)

    nL = len(schedule)
    if full:
        gains = lambda n: (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)  # noqa: E731
        put("embed_q", rng.integers(0, 256, size=(vocab, H // 4), dtype=np.uint8), "u8")
        put("embed_scale", (0.02 * (1 + rng.random(vocab))).astype(np.float32), "f32")
        put("ple_q", rng.integers(0, 256, size=(vocab, nL * ple_d // 2), dtype=np.uint8), "u8")
        put("ple_scale", (0.05 * (1 + rng.random(vocab * nL))).astype(np.float32), "f32")
        rows = pack_values(rng.integers(0, 4, size=(vocab, H)), 2)  # [vocab][H/16] words
        put("lmhead_blk", np.ascontiguousarray(rows.reshape(vocab, H // 64, 4).transpose(1, 0, 2)), "u32")
        put("lmhead_scale", (0.02 * (1 + rng.random(vocab))).astype(np.float32), "f32")
        put("pl_model_proj", (0.05 * rng.standard_normal((nL * ple_d, H))).astype(np.float16), "f16")
        put("final_norm", gains(H), "f32")
        put("pl_proj_norm", gains(ple_d), "f32")
    elif extra_odd_tensor:  # a u8 tensor of odd length first, so later offsets need the padding
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
        if full:
            inter, mb = 4 * H, mlp_bits[L % len(mlp_bits)]
            qrows = lambda n_out, n_in, b: pack_values(rng.integers(0, 1 << b, size=(n_out, n_in)), b)  # noqa: E731
            rsc = lambda n, s: (s * (1 + 0.2 * rng.random(n))).astype(np.float32)  # noqa: E731
            put(f"L{L}.o_bits", qrows(H, q_dim, 4), "u32")
            put(f"L{L}.o_scale", rsc(H, 0.01), "f32")
            put(f"L{L}.o_w12", np.concatenate([gains(H), gains(H)]), "f32")
            put(f"L{L}.down_nw", gains(H), "f32")
            put(f"L{L}.pleproj_w12s", np.concatenate([gains(H), gains(H), [np.float32(0.5 + rng.random())]]
                                                     ).astype(np.float32), "f32")
            step = 0.01 * (1 << (4 - mb))  # coarser rows for fewer bits, similar output size
            for tag, n_out, n_in in (("gate", inter, H), ("up", inter, H), ("down", H, inter)):
                put(f"L{L}.{tag}_bits", qrows(n_out, n_in, mb), "u32")
                put(f"L{L}.{tag}_scale", rsc(n_out, step), "f32")
            for tag, n_out, n_in in (("plegate", ple_d, H), ("pleproj", H, ple_d)):
                put(f"L{L}.{tag}_codes", qrows(n_out, n_in, 8), "u32")
                put(f"L{L}.{tag}_rowscale", rsc(n_out, 0.002), "f32")
            sc.update(gate_in=0.05, gate_out=0.02, up_in=0.04, up_out=0.02, down_in=0.01, down_out=0.02,
                      plegate_in=0.05, plegate_out=0.03, pleproj_in=0.03, pleproj_out=0.01)
            if gelu_tables:  # export.py:150, :161: the GELU tables of the two gate grids
                put(f"L{L}.gelu_gate", gelu_lut(sc["gate_out"]), "f32")
                put(f"L{L}.gelu_plegate", gelu_lut(sc["plegate_out"]), "f32")
        layers.append({"index": L, "sliding": sliding, "head_dim": hd, "q_dim": q_dim,
                       "intermediate": 4 * H, "shared": shared, "kv_source": src,
                       "rope_theta": 1e4 if sliding else 1e6, "rope_cutoff": cutoff, "scales": sc})
    if full:  # export.py:110, 119-122: the middle third of pleproj_w12s is the next layer's
        for L in range(nL):  # input norm, the final norm after the last layer
            nxt = arrays[f"L{L + 1}.in_norm"] if L + 1 < nL else arrays["final_norm"]
            arrays[f"L{L}.pleproj_w12s"][H:2 * H] = nxt
    w.close()
    man = {"config": {"H": H, "nL": nL, "nH": n_heads, "vocab": vocab if full else 16, "window": window,
                      "softcap": 30.0, "ple_d": ple_d if full else 8, "embed_scale": float(np.sqrt(H)),
                      "ple_scale": float(np.sqrt(ple_d if full else 8)), "bos": 2, "eos": 1},
           "layers": layers, "tensors": w.tensors, "bytes": w.pos}
    with open(os.path.join(out_dir, "manifest.json"), "w") as f:
        json.dump(man, f)
    return man, arrays
