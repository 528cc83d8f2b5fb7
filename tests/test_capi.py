"""CPU checks of the C ABI: the library loads, exports exactly what include/g4attn.h
declares, and rejects bad arguments before launching anything (no GPU needed)."""
import ctypes
import os
import re

import pytest

from slang_amd import _lib
from slang_amd._lib import G4ACfg

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "g4attn.h")


def declared_functions():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(g4a_[a-z_0-9]+)\s*\(", src)))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(_lib.LIB_PATH):
        pytest.fail("libg4attn.so is not built: run __graft_entry__.build() first")
    return _lib.load()


def test_exports_match_header(lib):
    decl = declared_functions()
    assert decl == sorted(_lib.EXPORTS), f"header declares {decl}, binding lists {sorted(_lib.EXPORTS)}"
    for name in decl:
        assert hasattr(lib, name), f"{name} not exported by libg4attn.so"


def test_cfg_struct_layout_matches_header():
    assert ctypes.sizeof(G4ACfg) == 8 * 4
    assert [f[0] for f in G4ACfg._fields_] == ["n_q_heads", "n_kv_heads", "head_dim", "window",
                                                "flags", "scale", "eps", "out_q"]


def test_strerror_and_version(lib):
    assert lib.g4a_version() == 2  # G4A_VERSION of include/g4attn.h
    for code in (0, -1, -2, -3, -4):
        assert lib.g4a_strerror(code)


def cfg(**kw):
    base = dict(n_q_heads=8, n_kv_heads=2, head_dim=256, window=0, flags=0, scale=1.0, eps=1e-6, out_q=0.0)
    base.update(kw)
    return G4ACfg(**base)


FAKE = ctypes.c_void_p(0x10000)  # never dereferenced: every case fails validation first


def decode(lib, c, **kw):
    a = dict(n_seq=1, max_key_len=64, key_len=FAKE, q=FAKE, gain=None, cos=None, sin=None, k=FAKE,
             v=FAKE, stride=0, out=FAKE, ws=FAKE, ws_bytes=1 << 30)
    a.update(kw)
    return lib.g4a_decode(ctypes.byref(c) if c is not None else None, a["n_seq"], a["max_key_len"],
                          a["key_len"], a["q"], a["gain"], a["cos"], a["sin"], a["k"], a["v"],
                          a["stride"], a["out"], a["ws"], a["ws_bytes"], None)


def test_decode_argument_errors(lib):
    assert decode(lib, None) == -1
    assert decode(lib, cfg(n_q_heads=6, n_kv_heads=4)) == -1          # not a multiple
    assert decode(lib, cfg(n_q_heads=12, n_kv_heads=1)) == -1         # group 12 > 8
    assert decode(lib, cfg(head_dim=128)) == -2                       # not instantiated
    assert decode(lib, cfg(), n_seq=0) == -1
    assert decode(lib, cfg(), q=None) == -1
    assert decode(lib, cfg(), cos=FAKE) == -1                         # sin missing
    assert decode(lib, cfg(), ws_bytes=16) == -3                      # workspace too small
    assert decode(lib, cfg(), ws=None) == -3
    assert b"workspace" in lib.g4a_last_error()


def test_decode_kv_argument_errors(lib):
    """g4a_decode_kv checks its own arguments, then those of g4a_decode."""
    D = lib.g4a_decode_kv

    def call(c=None, k_new=FAKE, v_new=FAKE, k_in_q=0.0, v_in_q=0.0, **kw):
        a = dict(n_seq=1, max_key_len=64, key_len=FAKE, q=FAKE, k=FAKE, v=FAKE, ws=FAKE, ws_bytes=1 << 30)
        a.update(kw)
        return D(ctypes.byref(c or cfg()), a["n_seq"], a["max_key_len"], a["key_len"], a["q"], None, None, None,
                 k_new, v_new, k_in_q, v_in_q, None, a["k"], a["v"], 0, FAKE, a["ws"], a["ws_bytes"], None)

    assert call(k_new=None) == -1
    assert call(v_new=None) == -1
    assert call(k_in_q=-1.0) == -1
    assert call(c=cfg(flags=0x2)) == -2                                # f16 raw rows not taken
    assert call(k_new=ctypes.c_void_p(0x10002)) == -1                   # misaligned
    assert call(n_seq=0) == -1                                          # g4a_decode's checks
    assert call(ws_bytes=16) == -3


def test_decode_ws_bytes(lib):
    c = cfg()
    small = lib.g4a_decode_ws_bytes(ctypes.byref(c), 1, 64)
    big = lib.g4a_decode_ws_bytes(ctypes.byref(c), 16, 32768)
    assert 0 < small < big
    assert lib.g4a_decode_ws_bytes(ctypes.byref(c), 0, 64) == 0


def test_prefill_and_kv_write_argument_errors(lib):
    c = cfg()
    P = lib.g4a_prefill
    assert P(ctypes.byref(c), 0, 0, FAKE, None, None, None, FAKE, FAKE, FAKE, None, 0, None) == -1
    assert P(ctypes.byref(c), 4, -1, FAKE, None, None, None, FAKE, FAKE, FAKE, None, 0, None) == -1
    assert P(ctypes.byref(cfg(head_dim=64)), 4, 0, FAKE, None, None, None, FAKE, FAKE, FAKE, None, 0, None) == -2
    assert P(ctypes.byref(c), 4, 0, ctypes.c_void_p(0x10004), None, None, None, FAKE, FAKE, FAKE,
             None, 0, None) == -1                                     # misaligned q
    K = lib.g4a_kv_write
    assert K(ctypes.byref(c), 1, 0, None, FAKE, 0.0, 0.0, None, None, None, FAKE, FAKE, None) == -1
    assert K(ctypes.byref(c), 1, 0, FAKE, FAKE, -1.0, 0.0, None, None, None, FAKE, FAKE, None) == -1
    assert K(ctypes.byref(cfg(head_dim=100)), 1, 0, FAKE, FAKE, 0.0, 0.0, None, None, None, FAKE,
             FAKE, None) == -2


def test_host_mirror_raises_without_library(monkeypatch, tmp_path):
    """The product path has no fallback: a missing library is an error, not a CPU path."""
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "LIB_PATH", str(tmp_path / "missing.so"))
    with pytest.raises(RuntimeError, match="no fallback"):
        _lib.load()


def test_projection_argument_errors(lib):
    f = FAKE
    # g4a_dequant(bits, n_in, n_out, w_bits, w_scale, out, stream)
    assert lib.g4a_dequant(3, 256, 4, f, f, f, None) == -2            # width not supported
    assert lib.g4a_dequant(4, 200, 4, f, f, f, None) == -1            # n_in not a multiple of 32
    assert lib.g4a_dequant(4, 256, 4, None, f, f, None) == -1
    assert lib.g4a_dequant(4, 256, 4, ctypes.c_void_p(0x10004), f, f, None) == -1  # misaligned
    # g4a_qkv_gemv(hidden, q_dim, kv_dim, a, sum_a, qb, kb, vb, scales, qo, ko, vo, oq, ok, ov, stream)
    g = lambda hidden=1536, qd=2048, kvd=512, kb=f, qo=0.0, **k: lib.g4a_qkv_gemv(
        hidden, qd, kvd, f, f, f, kb, f, f, qo, 0.0, 0.0, f, f, f, None)
    assert g(hidden=1530) == -1
    assert g(hidden=8192) == -1
    assert g(qd=2044) == -1
    assert g(kvd=-8) == -1
    assert g(kb=None) == -1                                           # k rows missing
    assert g(qo=-1.0) == -1
    # g4a_srqh(n, a, a_in_q, out, stream)
    assert lib.g4a_srqh(12, f, 0.0, f, None) == -1                     # n % 8
    assert lib.g4a_srqh(16, None, 0.0, f, None) == -1
    assert lib.g4a_srqh(16, f, -1.0, f, None) == -1
    # g4a_gemm16(M, K, a16, n_mats, mats, stream)
    mat = lambda n=128, w=f, out=f, oq=0.0: _lib.G4AGemmMat(w.value if w else None, out.value, n, 0, oq)  # noqa: E731
    tab = lambda *ms: (_lib.G4AGemmMat * len(ms))(*ms)  # noqa: E731
    assert lib.g4a_gemm16(16, 96, f, 1, tab(mat()), None) == -1        # K % 64
    assert lib.g4a_gemm16(0, 128, f, 1, tab(mat()), None) == -1
    assert lib.g4a_gemm16(16, 128, f, 0, tab(mat()), None) == -1       # no matrix
    assert lib.g4a_gemm16(16, 128, f, 4, tab(mat(), mat(), mat(), mat()), None) == -1
    assert lib.g4a_gemm16(16, 128, None, 1, tab(mat()), None) == -1
    assert lib.g4a_gemm16(16, 128, f, 2, tab(mat(), mat(n=100)), None) == -1   # n % 128
    assert lib.g4a_gemm16(16, 128, f, 1, tab(mat(w=None)), None) == -1
    assert lib.g4a_gemm16(16, 128, f, 1, tab(mat(oq=-1.0)), None) == -1
    assert b"matrix 0" in lib.g4a_last_error()


def test_gemm16_split_plan(lib):
    """g4a_gemm16_ws_bytes, the host side of the K split: launches with fewer 128 x 64 tiles
    than CUs split K so about 768 workgroups run (each range at least 4 k-steps), the rest do
    not split (0 bytes); the size is the ticket words plus one f32 partial tile (128 x 64) per
    (tile, split)."""
    f = FAKE
    mat = lambda n: _lib.G4AGemmMat(f.value, f.value, n, 0, 0.0, 1.0)  # noqa: E731
    tab = lambda *ns: (_lib.G4AGemmMat * len(ns))(*[mat(n) for n in ns])  # noqa: E731
    ws = lambda M, K, *ns: lib.g4a_gemm16_ws_bytes(M, K, len(ns), tab(*ns))  # noqa: E731
    part = 128 * 64 * 4
    assert ws(1024, 6144, 1536) == _lib.GEMM_TICKET_BYTES + 192 * 4 * part   # down: 192 tiles, 4 splits
    assert ws(1024, 2048, 1536) == _lib.GEMM_TICKET_BYTES + 192 * 4 * part   # o_proj
    assert ws(1024, 1536, 256) == _lib.GEMM_TICKET_BYTES + 32 * 6 * part     # PLE gate: 24 k-steps, 6 ranges
    assert ws(77, 4096, 128, 384) == _lib.GEMM_TICKET_BYTES + 8 * 16 * part  # one m-tile: 16 ranges of 4
    assert ws(1024, 256, 1536) == 0                                          # 4 k-steps: nothing to split
    assert ws(1024, 1536, 2048, 256, 256) == 0                               # 320 tiles: enough
    assert ws(1024, 1536, 6144, 6144) == 0                                   # 128-wide tiles
    assert ws(1024, 100, 1536) == 0 and ws(0, 1536, 1536) == 0 and ws(64, 1536, 100) == 0  # invalid: 0
    # a short workspace is refused before anything runs
    need = ws(1024, 2048, 1536)
    assert lib.g4a_gemm16_ws(1024, 2048, f, 1, tab(1536), f, need - 16, None) == -3
    assert lib.g4a_gemm16_ws(1024, 2048, f, 1, tab(1536), ctypes.c_void_p(0x10010), need, None) == -1  # alignment
    # g4a_gemm16_geglu(M, K, a, w_gate, w_up, n, gate_q, up_q, out_q, out, gelu_lut, stream)
    assert lib.g4a_gemm16_geglu(16, 96, f, f, f, 128, 0.1, 0.1, 0.1, f, None, None) == -1  # K % 64
    assert lib.g4a_gemm16_geglu(16, 128, f, f, f, 96, 0.1, 0.1, 0.1, f, None, None) == -1  # n % 64
    assert lib.g4a_gemm16_geglu(16, 128, f, None, f, 128, 0.1, 0.1, 0.1, f, None, None) == -1
    assert lib.g4a_gemm16_geglu(16, 128, f, f, f, 128, 0.1, -0.1, 0.1, f, None, None) == -1


def test_gemm_mat_struct_layout():
    """struct g4a_gemm_mat: two pointers, two ints, two floats (8-byte aligned, 32 bytes)."""
    assert [f[0] for f in _lib.G4AGemmMat._fields_] == ["w_f16", "out", "n", "out_f32", "out_q", "alpha"]
    assert _lib.G4AGemmMat.n.offset == 16 and _lib.G4AGemmMat.out_q.offset == 24
    assert _lib.G4AGemmMat.alpha.offset == 28
    assert ctypes.sizeof(_lib.G4AGemmMat) == 32


def test_decoder_argument_errors(lib):
    E, U = -1, -2
    f = ctypes.c_float
    # qgemv: bits, row shape, NULLs, alignment, negative steps
    assert lib.g4a_qgemv(3, 64, 4, FAKE, f(0), FAKE, FAKE, f(0), FAKE, None) == U
    assert lib.g4a_qgemv(16, 64, 4, FAKE, f(0), FAKE, FAKE, f(0), FAKE, None) == U
    assert lib.g4a_qgemv(4, 48, 4, FAKE, f(0), FAKE, FAKE, f(0), FAKE, None) == E      # 48 % 32
    assert lib.g4a_qgemv(2, 32, 4, FAKE, f(0), FAKE, FAKE, f(0), FAKE, None) == E      # 32 % 64
    assert lib.g4a_qgemv(4, 64, 0, FAKE, f(0), FAKE, FAKE, f(0), FAKE, None) == E
    assert lib.g4a_qgemv(4, 64, 4, FAKE, f(0), FAKE, None, f(0), FAKE, None) == E      # no scale
    assert lib.g4a_qgemv(4, 64, 4, ctypes.c_void_p(0x10004), f(0), FAKE, FAKE, f(0), FAKE, None) == E
    assert lib.g4a_qgemv(4, 64, 4, FAKE, f(-1), FAKE, FAKE, f(0), FAKE, None) == E
    assert lib.g4a_qgemv(4, 1 << 16, 1 << 16, FAKE, f(0), FAKE, FAKE, f(0), FAKE, None) == E  # 2 GiB rows
    assert lib.g4a_gemv_f16(12, 4, FAKE, FAKE, FAKE, None) == E                          # 12 % 8
    assert b"multiple" in lib.g4a_last_error()
    # rms_norm: rows, NULLs, sum2 without out2, negative eps
    args = lambda **k: [k.get(n, d) for n, d in (("rows", 1), ("n", 64), ("x", FAKE), ("pre", f(1)), ("w", None),  # noqa: E731
                        ("res", None), ("mult", f(1)), ("eps", f(1e-6)), ("out", FAKE), ("w2", None), ("q2", f(0)), ("f16", 0),
                        ("out2", None), ("sum2", None), ("s", None))]
    assert lib.g4a_rms_norm(*args(rows=0)) == E
    assert lib.g4a_rms_norm(*args(x=None)) == E
    assert lib.g4a_rms_norm(*args(sum2=FAKE)) == E
    assert lib.g4a_rms_norm(*args(w2=FAKE)) == E                                        # w2 without out2
    assert lib.g4a_rms_norm(*args(eps=f(-1))) == E
    assert lib.g4a_geglu(0, FAKE, FAKE, f(0), FAKE, None) == E
    assert lib.g4a_geglu(8, FAKE, FAKE, f(-0.5), FAKE, None) == E
    # embed: bits, n vs group, NULL token
    assert lib.g4a_embed(3, 64, FAKE, 8, FAKE, FAKE, 64, f(1), FAKE, None) == U
    assert lib.g4a_embed(2, 64, FAKE, 8, FAKE, FAKE, 48, f(1), FAKE, None) == E
    assert lib.g4a_embed(2, 64, FAKE, 8, None, FAKE, 64, f(1), FAKE, None) == E
    assert lib.g4a_softcap_argmax(0, FAKE, f(30), FAKE, FAKE, 64, None) == E
    assert lib.g4a_softcap_argmax(8, FAKE, f(-1), FAKE, FAKE, 64, None) == E
    assert lib.g4a_softcap_argmax_ws_bytes(262144) == 64 * 8 and lib.g4a_softcap_argmax_ws_bytes(0) == 0
    assert lib.g4a_softcap_argmax(262144, FAKE, f(30), FAKE, FAKE, 511, None) == -3        # workspace
    # fused GEMV variants: the same checks, and their own operands (..., pro, gelu_lut, stream)
    assert lib.g4a_qgemv_geglu(4, 48, 4, FAKE, FAKE, FAKE, f(0), f(0), FAKE, FAKE, f(0), f(0), f(0), FAKE, None, None,
                               None) == E
    assert lib.g4a_qgemv_geglu(4, 64, 4, FAKE, FAKE, FAKE, f(0), f(0), FAKE, None, f(0), f(0), f(0), FAKE, None, None,
                               None) == E
    assert lib.g4a_qgemv_geglu(4, 64, 4, FAKE, FAKE, FAKE, f(0), f(0), FAKE, FAKE, f(0), f(0), f(-1), FAKE, None,
                               None, None) == E
    assert lib.g4a_qgemv_gelu_mul(4, 64, 4, FAKE, f(0), FAKE, FAKE, f(0), None, FAKE, None, None, None) == E
    assert lib.g4a_qgemv_gelu_mul(16, 64, 4, FAKE, f(0), FAKE, FAKE, f(0), FAKE, FAKE, None, None, None) == U
    pro = _lib.G4ANormIn(FAKE.value, FAKE.value, None, None, FAKE.value, None, 0.0, 0, 1e-6)  # no w1
    assert lib.g4a_qgemv_gelu_mul(4, 64, 4, None, f(0), FAKE, FAKE, f(0), FAKE, FAKE, ctypes.byref(pro), None,
                                  None) == E
    pro.w1 = FAKE.value
    assert lib.g4a_qgemv_gelu_mul(4, 4096, 4, None, f(0), FAKE, FAKE, f(0), FAKE, FAKE, ctypes.byref(pro), None,
                                  None) == E


def test_decode_noalloc_limit(lib):
    """The allocation-free decode states its array size in the header and rejects calls whose
    partials exceed it before touching the device."""
    src = open(HEADER).read()
    m = re.search(r"#define G4A_DECODE_SCRATCH_BYTES \((\d+)u << (\d+)\)", src)
    assert m and int(m.group(1)) << int(m.group(2)) == _lib.DECODE_SCRATCH_BYTES
    c = cfg(n_q_heads=64, n_kv_heads=8, head_dim=512)  # 256 splits x 64 heads x 512 dims of partials
    need = lib.g4a_decode_ws_bytes(ctypes.byref(c), 1, 1 << 20)
    assert need > _lib.DECODE_SCRATCH_BYTES
    rc = lib.g4a_decode_noalloc(ctypes.byref(c), 1, 1 << 20, FAKE, FAKE, None, None, None, FAKE, FAKE,
                                0, FAKE, None)
    assert rc == -3 and b"at most" in lib.g4a_last_error()
