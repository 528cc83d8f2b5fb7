"""The weights.bin + manifest.json reader (gemma4_150/export.py:37-53, 161-181;
runner.py:55-59) on a synthetic model: tensor views, the 4-byte padding, the per-layer
schedule mapped to kernel constants (heads, window on sliding layers only, o_in as the
output srq step, RoPE table keys with the partial cutoff, KV sharing), and the errors a
malformed export must raise. CPU only."""
import json
import os

import numpy as np
import pytest

from manifest_fixture import SCHEDULE, write_model
from slang_amd.manifest import Manifest, ManifestError, load_manifest


@pytest.fixture
def model(tmp_path):
    man, arrays = write_model(tmp_path)
    return tmp_path, man, arrays


def rewrite(path, man):
    with open(os.path.join(path, "manifest.json"), "w") as f:
        json.dump(man, f)


def test_tensor_views_round_trip(model):
    path, man, arrays = model
    m = load_manifest(path)
    assert set(m.tensors) == set(arrays)
    for name, arr in arrays.items():
        got = m.tensor(name)
        assert got.dtype == arr.dtype and got.shape == arr.shape, name
        np.testing.assert_array_equal(got, arr)
        assert m.tensors[name]["off"] % 4 == 0
    assert not m.tensor("L0.q_norm").flags.writeable  # a read-only map, never a copy to mutate


def test_layer_schedule_to_kernel_constants(model):
    path, man, _ = model
    m = load_manifest(path)
    assert len(m.layers) == len(SCHEDULE)
    for L, (sliding, hd, cutoff, shared, src) in enumerate(SCHEDULE):
        c = m.attn_config(L)
        assert (c.n_q_heads, c.n_kv_heads, c.head_dim) == (4, 1, hd)
        assert c.window == (64 if sliding else 0)        # runner.py:290: window only when sliding
        assert c.scale == 1.0 and c.eps == 1e-6           # reference.py:162, :38-39
        assert c.out_q == man["layers"][L]["scales"]["o_in"]
        assert m.kv_dim(L) == hd and m.layers[L].kv_source == src
        assert m.rope_key(L) == (hd, 1e4 if sliding else 1e6, cutoff)
    # the KV-sharing layers read their source's caches: same rope tables and geometry
    assert m.rope_key(2) == m.rope_key(0) and m.rope_key(3) == m.rope_key(1)


def test_missing_files(tmp_path):
    with pytest.raises(ManifestError, match="manifest.json"):
        load_manifest(tmp_path)
    write_model(tmp_path)
    os.remove(os.path.join(tmp_path, "weights.bin"))
    with pytest.raises(ManifestError, match="weights.bin"):
        load_manifest(tmp_path)


@pytest.mark.parametrize("edit, match", [
    (lambda m: m["tensors"]["L0.q_norm"].update(off=m["tensors"]["L0.q_norm"]["off"] + 2), "aligned"),
    (lambda m: m["tensors"]["L0.q_norm"].update(off=m["bytes"] - 4), "aligned range"),
    (lambda m: m["tensors"]["L0.q_norm"].update(shape=[255]), "do not hold"),
    (lambda m: m["tensors"]["L0.q_norm"].update(dtype="bf16"), "unknown dtype"),
    (lambda m: m["tensors"].pop("L1.k_norm"), "missing tensor L1.k_norm"),
    (lambda m: m["tensors"].pop("L3.q_scale"), "missing tensor L3.q_scale"),
    (lambda m: m.update(bytes=m["bytes"] + 4), "bytes"),
    (lambda m: m["config"].update(nL=3), "nL"),
    (lambda m: m["layers"][2].update(kv_source=3), "kv_source"),      # a later layer
    (lambda m: m["layers"][3].update(kv_source=2), "kv_source"),      # a shared layer
    (lambda m: m["layers"][2].update(kv_source=1), "kv_source"),      # another head_dim
    (lambda m: m["layers"][1].update(kv_source=0), "own kv_source"),  # non-shared, not its own
    (lambda m: m["layers"][1].update(rope_cutoff=300), "rope_cutoff"),
    (lambda m: m["layers"][0].update(q_dim=1000), "q_dim"),
    (lambda m: m["layers"][0].update(index=5), "index"),
    (lambda m: m["layers"][0].pop("head_dim"), "malformed"),
])
def test_malformed_exports_raise(model, edit, match):
    path, man, _ = model
    edit(man)
    rewrite(path, man)
    with pytest.raises(ManifestError, match=match):
        load_manifest(path)


def test_manifest_from_parts_matches_loader(model):
    """Manifest() over an in-memory blob (what load_manifest maps) gives the same views."""
    path, man, arrays = model
    blob = np.fromfile(os.path.join(path, "weights.bin"), np.uint8)
    m = Manifest(man, blob)
    np.testing.assert_array_equal(m.tensor("L1.v_bits"), arrays["L1.v_bits"])
    assert m.n_kv_heads(3) == 1
