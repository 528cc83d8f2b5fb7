"""The decode step of the whole decoder on one GPU: embedding rows, every layer (attention
block, o_proj, MLP, per-layer-embedding block) and the greedy lm_head, over libg4attn.

Reference: gemma4_150/reference.py:114-207 (ReferenceSRQ.embed / ple_input / layer /
forward) is the arithmetic; gemma4_150/runner.py:373-505 (G4Runner.layer / forward) is
the resident form this mirrors: weights uploaded once, the hidden state and the next
token stay on the device, and the argmax's token feeds the next step's embedding rows
without a host round trip.

Two layers, as in attention.py:
  * ``qgemv`` / ``gemv_f16`` / ``rms_norm`` / ``geglu`` / ``embed`` / ``softcap_argmax``
    -- the library operations on torch tensors;
  * ``DecoderStack`` -- the model: an ``AttentionStack`` for the attention blocks plus the
    rest of each layer, driven by the manifest (export.py:86-181).

Every call is asynchronous on torch's current stream; nothing is computed on the host.
"""
from __future__ import annotations

import ctypes

import numpy as np
import torch

from . import _lib
from ._lib import check
from .attention import _need, _ptr, _stream
from .manifest import AttentionStack, Manifest, ManifestError
from .projection import GemmWorkspace, dequant, gemm16, gemm16_geglu, gemm16_ws_bytes, packed_bits, srqh

__all__ = ["qgemv", "norm_in", "qgemv_geglu", "qgemv_gelu_mul", "gemv_f16", "rms_norm", "geglu", "embed", "softcap_argmax",
           "embed_rows", "rows_tail", "geglu16", "plegate16", "DecoderStack", "EPS"]

EPS = 1e-6  # reference.py:27
_WORDS = (torch.int32, torch.uint32)


def qgemv(x, words, scale, n_in: int, n_out: int, *, in_q: float = 0.0, out_q: float = 0.0,
          bits: int | None = None, out=None):
    """out[o] = srq(scale[o] * sum_i (q[o][i] - zp) srq(x[i], in_q), out_q) (reference.py:96-111)."""
    _need(x, "x", torch.float32)
    _need(words, "words", _WORDS)
    _need(scale, "scale", torch.float32)
    bits = bits or packed_bits(words, n_in, n_out)
    if out is None:
        out = torch.empty(n_out, dtype=torch.float32, device=x.device)
    check(_lib.load().g4a_qgemv(bits, n_in, n_out, _ptr(x), float(in_q), _ptr(words), _ptr(scale), float(out_q),
                                _ptr(out), _stream()))
    return out


def norm_in(a, res, w1, x_out, *, w2=None, z_out=None, q2: float = 0.0, f16: bool = False, eps: float = EPS,
            mult: float = 1.0):
    """The residual-add + norm prologue of the fused GEMVs (struct g4a_norm_in): their input
    becomes srq(rms(x) * w2, q2) (f16-rounded around the srq with f16), with
    x = (res + rms(a) * w1) * mult stored to x_out (which must not alias a, res or w1).
    The struct holds raw device pointers: the tensors must stay alive until the call that
    takes it has been issued."""
    for t, n in ((a, "a"), (res, "res"), (w1, "w1"), (x_out, "x_out")):
        _need(t, n, torch.float32)
    return _lib.G4ANormIn(_ptr(a), _ptr(res), _ptr(w1), _ptr(w2) if w2 is not None else None, _ptr(x_out),
                          _ptr(z_out) if z_out is not None else None, float(q2), int(f16), float(eps), float(mult))


def _lut(t):
    """A layer's GELU table (f32 [256]) for the C ABI, or None."""
    if t is None:
        return None
    _need(t, "gelu_lut", torch.float32)
    if t.numel() != 256:
        raise ValueError("a GELU table holds 256 values")
    return _ptr(t)


def qgemv_geglu(x, gate, up, n_in: int, n_out: int, *, out_q: float, bits: int | None = None, out=None,
                pro=None, gelu_lut=None):
    """out = srq(gelu(qgemv(x, *gate)) * qgemv(x, *up), out_q) in one pass (gateup_74/95,
    reference.py:176-181); gate and up are (words, scale, in_q, out_q). pro: a norm_in(...)
    prologue that makes x (then x may be None). gelu_lut: the layer's GELU table of the gate's
    out_q grid (L{L}.gelu_gate, export.py:30-33), looked up as the runners do; None computes
    gelu_tanh."""
    (gw, gs, gi, go), (uw, us, ui, uo) = gate, up
    if pro is None:
        _need(x, "x", torch.float32)
    for t, n in ((gw, "gate words"), (uw, "up words")):
        _need(t, n, _WORDS)
    bits = bits or packed_bits(gw, n_in, n_out)
    if out is None:
        out = torch.empty(n_out, dtype=torch.float32, device=gw.device)
    check(_lib.load().g4a_qgemv_geglu(bits, n_in, n_out, _ptr(x) if x is not None else None, _ptr(gw), _ptr(gs),
                                      float(gi), float(go), _ptr(uw), _ptr(us), float(ui), float(uo), float(out_q),
                                      _ptr(out), ctypes.byref(pro) if pro is not None else None, _lut(gelu_lut),
                                      _stream()))
    return out


def qgemv_gelu_mul(x, words, scale, mul, n_in: int, n_out: int, *, in_q: float = 0.0, out_q: float = 0.0,
                   bits: int | None = None, out=None, pro=None, gelu_lut=None):
    """out = gelu(qgemv(x)) * mul (plegate_76; reference.py:186-187); pro and gelu_lut (here the
    table of out_q's grid, L{L}.gelu_plegate) as for qgemv_geglu."""
    if pro is None:
        _need(x, "x", torch.float32)
    _need(words, "words", _WORDS)
    _need(mul, "mul", torch.float32)
    bits = bits or packed_bits(words, n_in, n_out)
    if out is None:
        out = torch.empty(n_out, dtype=torch.float32, device=words.device)
    check(_lib.load().g4a_qgemv_gelu_mul(bits, n_in, n_out, _ptr(x) if x is not None else None, float(in_q),
                                         _ptr(words), _ptr(scale), float(out_q), _ptr(mul), _ptr(out),
                                         ctypes.byref(pro) if pro is not None else None, _lut(gelu_lut),
                                         _stream()))
    return out


def gemv_f16(x, w_f16, out=None):
    """out = w @ x, w f16 [n_out][n_in], f32 accumulation (reference.py:136)."""
    _need(x, "x", torch.float32)
    _need(w_f16, "w", torch.float16)
    n_out, n_in = w_f16.shape
    if out is None:
        out = torch.empty(n_out, dtype=torch.float32, device=x.device)
    check(_lib.load().g4a_gemv_f16(n_in, n_out, _ptr(x), _ptr(w_f16), _ptr(out), _stream()))
    return out


def rms_norm(x, w=None, *, res=None, pre: float = 1.0, mult: float = 1.0, eps: float = EPS, out=None,
             w2=None, q2: float | None = None, f16_2: bool = False, out2=None, sum2=None):
    """Rows of x [.., n]: out = (res + rms(x * pre) * w) * mult; optional out2 = srq(z, q2)
    (f16_2: f16(srq(f16(z), q2))) with z = out or, given w2, z = rms(out) * w2, and sum2 =
    sum of out2 per row (reference.py:38-43)."""
    _need(x, "x", torch.float32)
    n = x.shape[-1]
    rows = x.numel() // n
    if out is None:
        out = torch.empty_like(x)
    if (q2 is not None or w2 is not None) and out2 is None:
        out2 = torch.empty_like(x)
    lib = _lib.load()
    check(lib.g4a_rms_norm(rows, n, _ptr(x), float(pre), _ptr(w) if w is not None else None,
                           _ptr(res) if res is not None else None, float(mult), float(eps), _ptr(out),
                           _ptr(w2) if w2 is not None else None, float(q2 or 0.0), int(f16_2), _ptr(out2) if out2 is not None else None,
                           _ptr(sum2) if sum2 is not None else None, _stream()))
    return (out, out2) if out2 is not None else out


def geglu(a, b, out_q: float = 0.0, out=None):
    """out = srq(gelu_tanh(a) * b, out_q) (reference.py:34-35, :181, :188)."""
    _need(a, "a", torch.float32)
    _need(b, "b", torch.float32)
    if out is None:
        out = torch.empty_like(a)
    check(_lib.load().g4a_geglu(a.numel(), _ptr(a), _ptr(b), float(out_q), _ptr(out), _stream()))
    return out


def embed(table_u8, tok, row_scale, n: int, bits: int, group: int, mult: float, out=None):
    """Row tok[0] (device int32) of a packed table: mult * scale * (code - zp) (reference.py:114-131)."""
    _need(table_u8, "table", torch.uint8)
    _need(tok, "tok", torch.int32)
    _need(row_scale, "row_scale", torch.float32)
    if out is None:
        out = torch.empty(n, dtype=torch.float32, device=table_u8.device)
    check(_lib.load().g4a_embed(bits, n, _ptr(table_u8), table_u8.shape[0], _ptr(tok), _ptr(row_scale), group,
                                float(mult), _ptr(out), _stream()))
    return out


def embed_rows(table_u8, tok, row_scale, n: int, bits: int, group: int, mult: float, out=None):
    """embed for every id of tok (device int32 [S]): out [S][n] (embed_00 / plegather_01 over S
    tokens, kernels_dsl.py:433-479)."""
    _need(table_u8, "table", torch.uint8)
    _need(tok, "tok", torch.int32)
    _need(row_scale, "row_scale", torch.float32)
    S = tok.numel()
    if out is None:
        out = torch.empty(S, n, dtype=torch.float32, device=table_u8.device)
    _need(out, "out", torch.float32)
    check(_lib.load().g4a_embed_rows(bits, n, _ptr(table_u8), table_u8.shape[0], _ptr(tok), S, _ptr(row_scale),
                                     group, float(mult), _ptr(out), _stream()))
    return out


def rows_tail(hidden, x16=None, *, x_q: float = 0.0, w1=None, mult: float = 1.0, mode: int = _lib.TAIL_NONE,
              w2=None, q2: float = 0.0, y16=None, eps: float = EPS):
    """Per row of hidden f32 [S][n]: with x16 (f16 [S][n], a GEMM output) the residual add
    hidden = (hidden + rms(srq(x16, x_q)) * w1) * mult (rmsadd_b), then the next GEMM operand
    y16 f16 by mode: TAIL_SRQ f16(srq(hidden, q2)) (srqh_b), TAIL_NORM f16(srq(rms(hidden) * w2,
    q2)) (rmssrq_69), TAIL_NORM16 f16(srq(f32(f16(rms(hidden) * w2)), q2)) (rmssrqh_b)
    (kernels_dsl.py:158-206, 233-242, 622-710). Returns y16."""
    _need(hidden, "hidden", torch.float32)
    _need(x16, "x16", torch.float16)
    S, n = hidden.shape
    if mode != _lib.TAIL_NONE and y16 is None:
        y16 = torch.empty(S, n, dtype=torch.float16, device=hidden.device)
    _need(y16, "y16", torch.float16)
    check(_lib.load().g4a_rows_tail(S, n, _ptr(x16), float(x_q), _ptr(w1), float(mult), float(eps), _ptr(hidden),
                                    int(mode), _ptr(w2), float(q2), _ptr(y16), _stream()))
    return y16


def geglu16(gate16, up16, gate_q: float, up_q: float, out_q: float, out=None, gelu_lut=None):
    """geglu_b (kernels_dsl.py:259-290): f16 code round(gelu(srq(g, gate_q)) * srq(u, up_q) / out_q);
    gelu_lut the layer's table of gate_q's grid (qgemv_geglu)."""
    _need(gate16, "gate", torch.float16)
    _need(up16, "up", torch.float16)
    if out is None:
        out = torch.empty_like(gate16)
    check(_lib.load().g4a_geglu16(gate16.numel(), _ptr(gate16), _ptr(up16), float(gate_q), float(up_q),
                                  float(out_q), _ptr(out), _lut(gelu_lut), _stream()))
    return out


def plegate16(lin16, lin_q: float, ple, ple_stride: int, out_q: float, out=None, gelu_lut=None):
    """plegate_b then srqh_b (kernels_dsl.py:1767-1786, 233-242): f16(srq(gelu(srq(lin, lin_q)) *
    ple, out_q)) over lin16 f16 [S][d]; ple points at the layer's slice of [S][nL][d] (row stride
    ple_stride values); gelu_lut the layer's table of lin_q's grid (qgemv_geglu)."""
    _need(lin16, "lin", torch.float16)
    S, d = lin16.shape
    if out is None:
        out = torch.empty_like(lin16)
    check(_lib.load().g4a_plegate16(S, d, _ptr(lin16), float(lin_q), _ptr(ple), int(ple_stride), float(out_q),
                                    _ptr(out), _lut(gelu_lut), _stream()))
    return out


def softcap_argmax(logits, cap: float, tok=None, ws=None):
    """logits <- cap * tanh(logits / cap) in place; tok[0] = first argmax (reference.py:207).
    ws: a byte tensor of at least g4a_softcap_argmax_ws_bytes(n) (allocated when absent)."""
    _need(logits, "logits", torch.float32)
    lib = _lib.load()
    if tok is None:
        tok = torch.empty(1, dtype=torch.int32, device=logits.device)
    if ws is None:
        ws = torch.empty(lib.g4a_softcap_argmax_ws_bytes(logits.numel()), dtype=torch.uint8, device=logits.device)
    check(lib.g4a_softcap_argmax(logits.numel(), _ptr(logits), float(cap), _ptr(tok), _ptr(ws), ws.numel(),
                                 _stream()))
    return tok


def lmhead_rows(blk: np.ndarray) -> np.ndarray:
    """export.py:91-93 writes the lm_head as [H/64][vocab][4] words (one 16-byte block of
    every row after another); the GEMV reads whole rows, [vocab][H/16] words."""
    nb, vocab, four = blk.shape
    return np.ascontiguousarray(blk.transpose(1, 0, 2)).reshape(vocab, nb * four)


class DecoderStack:
    """Every layer of the exported model for one token per step (reference.py:141-207).

    Holds an AttentionStack (caches, q/k/v weights) and uploads the rest once: embedding
    and per-layer-embedding tables, lm_head rows, o_proj, MLP and per-layer-embedding
    linears and the norms. ``step(pos)`` runs the token in ``self.tok`` (device int32 [1])
    at position pos and leaves the argmax in ``self.tok`` and the soft-capped logits in
    ``self.logits``, so consecutive steps never touch the host.
    """

    def __init__(self, man: Manifest, max_seq: int, device="cuda"):
        self.man = man
        self.device = device
        need = ["embed_q", "embed_scale", "ple_q", "ple_scale", "lmhead_blk", "lmhead_scale", "pl_model_proj",
                "final_norm", "pl_proj_norm"]
        for L in range(len(man.layers)):
            need += [f"L{L}.{n}" for n in ("in_norm", "o_bits", "o_scale", "o_w12", "down_nw", "pleproj_w12s",
                                           "gate_bits", "gate_scale", "up_bits", "up_scale", "down_bits",
                                           "down_scale", "plegate_codes", "plegate_rowscale", "pleproj_codes",
                                           "pleproj_rowscale")]
        missing = [n for n in need if n not in man.tensors]
        if missing:
            raise ManifestError(f"the decoder needs tensors the manifest lacks: {missing[:4]}...")
        c = man.config
        self.H, self.nL, self.d = man.hidden, int(c["nL"]), int(c["ple_d"])
        self.vocab, self.softcap = int(c["vocab"]), float(c.get("softcap", 0.0))
        self.embed_scale, self.ple_scale = float(c["embed_scale"]), float(c["ple_scale"])
        self.attn = AttentionStack(man, max_seq, device)
        dev = lambda a: torch.from_numpy(np.array(a)).to(device)  # noqa: E731  (a copy: the map is read-only)
        words = lambda name: dev(man.tensor(name)).view(torch.int32).reshape(-1)  # noqa: E731
        self.embed_q, self.embed_sc = dev(man.tensor("embed_q")), dev(man.tensor("embed_scale"))
        self.ple_q, self.ple_sc = dev(man.tensor("ple_q")), dev(man.tensor("ple_scale"))
        self.lm_rows = dev(lmhead_rows(man.tensor("lmhead_blk"))).view(torch.int32).reshape(-1)
        self.lm_sc = dev(man.tensor("lmhead_scale"))
        self.pl_proj = dev(man.tensor("pl_model_proj"))
        self.final_norm, self.pl_norm = dev(man.tensor("final_norm")), dev(man.tensor("pl_proj_norm"))
        H = self.H
        self.w = []
        for s in man.layers:
            L = s.index
            t = lambda n: dev(man.tensor(f"L{L}.{n}"))  # noqa: E731
            w = {n: t(n) for n in ("in_norm", "o_scale", "o_w12", "down_nw", "gate_scale", "up_scale",
                                   "down_scale", "plegate_rowscale", "pleproj_rowscale")}
            for n in ("o_bits", "gate_bits", "up_bits", "down_bits", "plegate_codes", "pleproj_codes"):
                w[n] = words(f"L{L}.{n}")
            pl = man.tensor(f"L{L}.pleproj_w12s")
            w["post_ple"] = dev(pl[:H])
            w["layer_scalar"] = float(pl[2 * H])
            w["o_w1"], w["o_w2"] = w["o_w12"][:H], w["o_w12"][H:]
            w["gate_bits_n"] = packed_bits(w["gate_bits"], H, s.intermediate)
            w["down_bits_n"] = packed_bits(w["down_bits"], s.intermediate, H)
            w["o_bits_n"] = packed_bits(w["o_bits"], s.q_dim, H)
            # the exporter's GELU tables of the gate and per-layer-embedding gate grids
            # (export.py:30-33, :150, :161), used as the runners use them; absent: gelu_tanh
            for n in ("gelu_gate", "gelu_plegate"):
                w[n] = t(n) if f"L{L}.{n}" in man.tensors else None
            self.w.append(w)
        f32 = lambda *shape: torch.zeros(*shape, dtype=torch.float32, device=device)  # noqa: E731
        inter = max(s.intermediate for s in man.layers)
        self.x, self.h, self.a, self.sum_a = f32(H), f32(H), f32(H), f32(1)
        self.o, self.y2, self.hf, self.xb = f32(H), f32(H), f32(H), f32(H)
        self.gg = f32(inter)
        self.down = f32(H)
        self.ple_tab, self.ple_proj, self.ple_in = f32(self.nL, self.d), f32(self.nL * self.d), f32(self.nL, self.d)
        self.pleg, self.pleproj = f32(self.d), f32(H)
        self.logits = f32(self.vocab)
        self.arg_ws = torch.empty(_lib.load().g4a_softcap_argmax_ws_bytes(self.vocab), dtype=torch.uint8,
                                  device=device)
        self.tok = torch.zeros(1, dtype=torch.int32, device=device)
        self.dq16, self._pb = {}, None  # batched prefill: f16 weights and activation buffers
        self._pb_retired, self._pb_pinned = [], False

    def embed_token(self):
        """x = embed(tok), ple_in = ple_input(tok, x), and layer 0's srq'd input norm
        (reference.py:114-139, 145-147)."""
        H, nL, d = self.H, self.nL, self.d
        embed(self.embed_q, self.tok, self.embed_sc, H, 2, H, self.embed_scale, out=self.x)
        embed(self.ple_q, self.tok, self.ple_sc, nL * d, 4, d, self.ple_scale, out=self.ple_tab.view(-1))
        gemv_f16(self.x, self.pl_proj, out=self.ple_proj)
        rms_norm(self.ple_proj.view(nL, d), self.pl_norm, res=self.ple_tab, pre=H ** -0.5, mult=2.0 ** -0.5,
                 out=self.ple_in)
        rms_norm(self.x, self.w[0]["in_norm"], out=self.h, q2=self.man.layers[0].scales["qkv_in"], out2=self.a,
                 sum2=self.sum_a)

    def layer(self, L: int, pos: int, trace: dict | None = None, prev: dict | None = None):
        """Layer L on the residual from its input norm (reference.py:141-191). Layer 0 starts
        from x and its srq'd input norm in self.a / self.sum_a (embed_token); every later layer
        first finishes the previous layer's tail inside its q/k/v GEMV: x3 = (x2 + rms(pleproj)
        * post_ple) * layer_scalar and a = srq(rms(x3) * in_norm, qkv_in), as pleproj_77 ends
        with rmssrq_69. The norms ride on the kernels after the adds as the runner fuses them
        (oproj_73 ends with the pre-FFN norm). The residual alternates between self.x and
        self.xb, since a workgroup that stores the new residual must not overwrite the one the
        others still read: layer L's input is in self.x for even L, self.xb for odd L, and the
        last layer's tail and the final norm run as one g4a_rms_norm in place (residual()).
        trace gets this layer's stages, prev (the previous layer's trace) its x3 and a_next."""
        s, w, H = self.man.layers[L], self.w[L], self.H
        sc, inter = s.scales, s.intermediate
        xin, xalt = (self.x, self.xb) if L % 2 == 0 else (self.xb, self.x)
        snap = (lambda k, t: trace.__setitem__(k, t.clone())) if trace is not None else (lambda k, t: None)
        if L == 0:
            attn = self.attn.decode_layer(L, pos, self.a, self.sum_a).view(-1)
        else:
            pw = self.w[L - 1]
            pro = norm_in(self.pleproj, xalt, pw["post_ple"], xin, w2=w["in_norm"], q2=sc["qkv_in"],
                          mult=pw["layer_scalar"])
            attn = self.attn.decode_layer(L, pos, self.a, self.sum_a, pro=pro).view(-1)
            if prev is not None:
                prev["x3"] = xin.clone()
                prev["a_next"] = self.a.clone()
        snap("x0", xin)
        snap("a", self.a)
        snap("attn", attn)
        # the attention output is already on o_in's grid and the GeGLU output on down_in's; the
        # GEMVs are told the grid all the same (srq(srq(v, s), s) = srq(v, s) exactly), so they
        # take the integer dot products: x staged as its int8 grid index
        qgemv(attn, w["o_bits"], w["o_scale"], s.q_dim, H, in_q=sc["o_in"], out_q=sc["o_out"], bits=w["o_bits_n"],
              out=self.o)
        snap("o", self.o)
        # x1 = x + rms(o) * w1 and the MLP input y2 = f16(srq(f16(rms(x1) * w2), gate_in)) are
        # made by the gate/up kernel's prologue (x1 into the other residual buffer)
        gg = self.gg[:inter]
        qgemv_geglu(None, (w["gate_bits"], w["gate_scale"], sc["gate_in"], sc["gate_out"]),
                    (w["up_bits"], w["up_scale"], sc["up_in"], sc["up_out"]), H, inter, out_q=sc["down_in"],
                    bits=w["gate_bits_n"], out=gg,
                    pro=norm_in(self.o, xin, w["o_w1"], xalt, w2=w["o_w2"], z_out=self.y2, q2=sc["gate_in"],
                                f16=True), gelu_lut=w["gelu_gate"])
        snap("x1", xalt)
        snap("y2", self.y2)
        snap("geglu", gg)
        qgemv(gg, w["down_bits"], w["down_scale"], inter, H, in_q=sc["down_in"], out_q=sc["down_out"],
              bits=w["down_bits_n"], out=self.down)
        snap("down", self.down)
        # x2 = x1 + rms(down) * w: the per-layer-embedding gate kernel's prologue, back into xin
        qgemv_gelu_mul(None, w["plegate_codes"], w["plegate_rowscale"], self.ple_in[L], H, self.d,
                       in_q=sc["plegate_in"], out_q=sc["plegate_out"], bits=8, out=self.pleg,
                       pro=norm_in(self.down, xalt, w["down_nw"], xin), gelu_lut=w["gelu_plegate"])
        snap("x2", xin)
        snap("pleg", self.pleg)
        qgemv(self.pleg, w["pleproj_codes"], w["pleproj_rowscale"], self.d, H, in_q=sc["pleproj_in"],
              out_q=sc["pleproj_out"], bits=8, out=self.pleproj)
        snap("pleproj", self.pleproj)
        if L + 1 == self.nL:
            # the last layer's tail and the final norm (no q/k/v GEMV follows to carry them)
            rms_norm(self.pleproj, w["post_ple"], res=xin, mult=w["layer_scalar"], out=xin,
                     w2=self.final_norm, out2=self.hf)
            snap("x3", xin)
            snap("hf", self.hf)

    def residual(self) -> torch.Tensor:
        """The residual stream after the last layer (x3 of layer nL - 1)."""
        return self.x if (self.nL - 1) % 2 == 0 else self.xb

    # ---------------------------------------------------------------- batched prefill
    def _prefill_weights(self, L: int) -> dict:
        """Layer L's o_proj, MLP and per-layer-embedding linears dequantised to f16 once and kept
        resident (PrefillGPU._dq dequantises them into scratch on every prefill,
        prefill_gpu.py:186-200; one GPU's HBM holds every layer's f16 copy many times over)."""
        if L not in self.dq16:
            s, w, H, d = self.man.layers[L], self.w[L], self.H, self.d
            it = s.intermediate
            self.dq16[L] = {
                "o": dequant(w["o_bits"], w["o_scale"], s.q_dim, H, bits=w["o_bits_n"]),
                "gate": dequant(w["gate_bits"], w["gate_scale"], H, it, bits=w["gate_bits_n"]),
                "up": dequant(w["up_bits"], w["up_scale"], H, it, bits=w["gate_bits_n"]),
                "down": dequant(w["down_bits"], w["down_scale"], it, H, bits=w["down_bits_n"]),
                "plegate": dequant(w["plegate_codes"], w["plegate_rowscale"], H, d, bits=8),
                "pleproj": dequant(w["pleproj_codes"], w["pleproj_rowscale"], d, H, bits=8)}
        return self.dq16[L]

    def reserve(self, max_S: int, start_pos: int = 0) -> "DecoderStack":
        """Size every buffer that prefill() of up to max_S tokens at start_pos, step() and
        generate() use -- the prefill activations, the attention workspace (decode up to the
        caches' length, prefill at every S <= max_S) and the GEMM workspace -- and pin them.
        After it no such call allocates a workspace or activation buffer, and one that would
        need more raises instead of reallocating, so the buffers a HIP graph captured over
        these calls points at stay its own. Call it before the first capture."""
        if not 0 < max_S <= self.attn.max_seq - start_pos:
            raise ValueError(f"max_S {max_S} at start_pos {start_pos} exceeds the {self.attn.max_seq}-row caches")
        man, lib, H, d = self.man, _lib.load(), self.H, self.d
        self._prefill_buffers(max_S)
        self._pb_pinned = True
        need = 0
        for cfg in {man.attn_config(L) for L in range(self.nL)}:
            c = cfg.c(0)
            need = max(need, lib.g4a_decode_ws_bytes(ctypes.byref(c), 1, self.attn.max_seq))
            for S in range(1, max_S + 1):
                need = max(need, lib.g4a_prefill_ws_bytes(ctypes.byref(c), S, start_pos))
        self.attn.ws.reserve(need)
        # the K split's scratch of every gemm16 a prefill issues: per-layer embedding
        # projection, q/k/v, o_proj, down (and gate/up on their own when traced)
        shapes = {(H, (self.nL * d,))}
        for s in man.layers:
            shapes |= {(H, (s.q_dim,) if s.shared else (s.q_dim, man.kv_dim(s.index), man.kv_dim(s.index))),
                       (s.q_dim, (H,)), (s.intermediate, (H,)), (H, (s.intermediate, s.intermediate))}
        gneed = max(gemm16_ws_bytes(M, K, ns) for M in range(1, max_S + 1) for K, ns in shapes)
        self.attn.gemm_ws.reserve(gneed)
        return self

    def _prefill_buffers(self, S: int):
        """Activations of an S-token prefill (flat, kept for later prompts of at most S tokens);
        returns take(name, *shape), a contiguous view of the first prod(shape) values. Buffers
        outgrown by a longer prompt are retired, not freed: a HIP graph captured over an
        earlier prefill still owns what it points at."""
        if self._pb is None or self._pb["S"] < S:
            if self._pb_pinned:
                raise RuntimeError(f"prefill buffers reserved for {self._pb['S']} tokens; this prompt has {S}")
            if self._pb is not None:
                self._pb_retired.append(self._pb)
            H, nL, d = self.H, self.nL, self.d
            it = max(s.intermediate for s in self.man.layers)
            qd = max(s.q_dim for s in self.man.layers)
            f32 = lambda n: torch.empty(S * n, dtype=torch.float32, device=self.device)  # noqa: E731
            f16 = lambda n: torch.empty(S * n, dtype=torch.float16, device=self.device)  # noqa: E731
            self._pb = {"S": S, "hidden": f32(H), "ctx": f32(nL * d), "plegath": f32(nL * d), "ple": f32(nL * d),
                        "a16": f16(H), "attn": f16(qd), "o16": f16(H), "y2": f16(H), "g16": f16(it),
                        "u16": f16(it), "gg16": f16(it), "d16": f16(H), "hh": f16(H), "plin": f16(d),
                        "gph": f16(d), "pp16": f16(H), "ids": torch.empty(S, dtype=torch.int32, device=self.device)}
        pb = self._pb
        return lambda name, *shape: pb[name][:int(np.prod(shape))].view(*shape)

    def prefill(self, toks, start_pos: int = 0, trace: list | None = None) -> int:
        """Run S prompt tokens through every layer at positions start_pos.., layers outer and
        tokens inner, leaving the K/V caches filled (PrefillGPU.prefill, prefill_gpu.py:398-436;
        the layer is _layer, :316-395). Each linear is one f16 GEMM over all S rows (weights
        dequantised once, activations f16(srq(..)) as srqh_b makes them, products f16 as
        gemm_tiled rounds them), the attention one batched causal prefill. Like the reference
        it makes no logits: decoding continues from the next token. toks: host ints or a device
        int32 tensor [S]. Returns start_pos + S. trace: gets one dict per layer of its stages."""
        ids = toks if torch.is_tensor(toks) else torch.tensor(list(toks), dtype=torch.int32)
        S = int(ids.numel())
        if S <= 0:
            return start_pos
        if start_pos < 0 or start_pos + S > self.attn.max_seq:
            raise ValueError(f"positions [{start_pos}, {start_pos + S}) outside the {self.attn.max_seq}-row caches")
        take = self._prefill_buffers(S)
        H, nL, d = self.H, self.nL, self.d
        tid = take("ids", S)
        tid.copy_(ids.to(device=self.device, dtype=torch.int32), non_blocking=True)
        hid, ple, ctx, plegath = take("hidden", S, H), take("ple", S, nL, d), take("ctx", S, nL * d), \
            take("plegath", S, nL * d)
        snap = (lambda t, k, v: t.__setitem__(k, v.clone())) if trace is not None else (lambda t, k, v: None)
        # token embeddings and the per-layer inputs (prefill_gpu.py:412-429)
        embed_rows(self.embed_q, tid, self.embed_sc, H, 2, H, self.embed_scale, out=hid)
        a16 = take("a16", S, H)
        srqh(hid, 0.0, out=a16)
        gws = self.attn.gemm_ws
        gemm16(a16, [(self.pl_proj, ctx, 0.0)], gws)  # f32(f16(h . P^T)): srq_b with step 0
        embed_rows(self.ple_q, tid, self.ple_sc, nL * d, 4, d, self.ple_scale, out=plegath)
        rms_norm(ctx.view(S * nL, d), self.pl_norm, res=plegath.view(S * nL, d), pre=H ** -0.5,
                 mult=2.0 ** -0.5, out=ple.view(S * nL, d))    # combine_b
        if trace is not None:
            trace.append({"hidden": hid.clone(), "ctx": ctx.clone(), "plegath": plegath.clone(), "ple": ple.clone()})
        rows_tail(hid, mode=_lib.TAIL_NORM, w2=self.w[0]["in_norm"], q2=self.man.layers[0].scales["qkv_in"], y16=a16)
        for L in range(nL):
            s, w, wd = self.man.layers[L], self.w[L], self._prefill_weights(L)
            sc, it = s.scales, s.intermediate
            t = {} if trace is not None else None
            snap(t, "a16", a16)
            snap(t, "x0", hid)
            attn = self.attn.prefill_layer(L, start_pos, a16, out=take("attn", S, s.q_dim // s.head_dim, s.head_dim),
                                           trace=t).view(S, s.q_dim)
            snap(t, "attn", attn)
            o16, y2 = take("o16", S, H), take("y2", S, H)
            gemm16(attn, [(wd["o"], o16, None)], gws)
            rows_tail(hid, o16, x_q=sc["o_out"], w1=w["o_w1"], mode=_lib.TAIL_NORM16, w2=w["o_w2"],
                      q2=sc["gate_in"], y16=y2)
            snap(t, "o16", o16)
            snap(t, "x1", hid)
            snap(t, "y2", y2)
            gg = take("gg16", S, it)
            gemm16_geglu(y2, wd["gate"], wd["up"], sc["gate_out"], sc["up_out"], sc["down_in"], out=gg,
                         gelu_lut=w["gelu_gate"])
            if t is not None:  # the two products on their own, for the stage checks
                g16, u16 = take("g16", S, it), take("u16", S, it)
                gemm16(y2, [(wd["gate"], g16, None), (wd["up"], u16, None)], gws)
                snap(t, "g16", g16)
                snap(t, "u16", u16)
            snap(t, "gg16", gg)
            d16, hh = take("d16", S, H), take("hh", S, H)
            gemm16(gg, [(wd["down"], d16, None, sc["down_in"])], gws)
            rows_tail(hid, d16, x_q=sc["down_out"], w1=w["down_nw"], mode=_lib.TAIL_SRQ, q2=sc["plegate_in"], y16=hh)
            snap(t, "d16", d16)
            snap(t, "x2", hid)
            snap(t, "hh", hh)
            plin, gph, pp = take("plin", S, d), take("gph", S, d), take("pp16", S, H)
            gemm16(hh, [(wd["plegate"], plin, None)], gws)
            plegate16(plin, sc["plegate_out"], ple[:, L], nL * d, sc["pleproj_in"], out=gph,
                      gelu_lut=w["gelu_plegate"])
            gemm16(gph, [(wd["pleproj"], pp, None)], gws)
            snap(t, "plin", plin)
            snap(t, "gph", gph)
            snap(t, "pp16", pp)
            if L + 1 < nL:  # the next layer's srq'd input norm as its GEMM operand (rmssrq_69 + srqh_b)
                rows_tail(hid, pp, x_q=sc["pleproj_out"], w1=w["post_ple"], mult=w["layer_scalar"],
                          mode=_lib.TAIL_NORM, w2=self.w[L + 1]["in_norm"],
                          q2=self.man.layers[L + 1].scales["qkv_in"], y16=a16)
            else:
                rows_tail(hid, pp, x_q=sc["pleproj_out"], w1=w["post_ple"], mult=w["layer_scalar"])
            snap(t, "x3", hid)
            if trace is not None:
                trace.append(t)
        return start_pos + S

    def generate(self, ids, n_new: int, start_pos: int = 0) -> torch.Tensor:
        """Greedy generation kept on the GPU (G4Runner.generate_resident, runner.py:542-569):
        prefill every prompt token but the last, then n_new decode steps from the last one, each
        step's argmax feeding the next step's embedding on the device. Returns the n_new tokens
        (device int32); the caller reads them back when it wants them. ids: host ints, or a device
        int32 tensor (then nothing goes through the host, so the call can be captured in a graph)."""
        dev_ids = torch.is_tensor(ids) and ids.device.type != "cpu"
        if not dev_ids:
            ids = list(ids)
        n = int(ids.numel()) if dev_ids else len(ids)
        if n == 0 or n_new <= 0:
            return torch.empty(0, dtype=torch.int32, device=self.device)
        pos = self.prefill(ids[:-1], start_pos) if n > 1 else start_pos
        if pos + n_new > self.attn.max_seq:
            raise ValueError(f"{pos + n_new} positions exceed the {self.attn.max_seq}-row caches")
        if dev_ids:
            self.tok.copy_(ids[-1:].to(torch.int32))
        else:
            self.tok.fill_(int(ids[-1]))
        out = torch.empty(n_new, dtype=torch.int32, device=self.device)
        for i in range(n_new):
            self.step(pos + i)
            out[i:i + 1].copy_(self.tok)
        return out

    def head(self):
        """2-bit lm_head over the final norm, softcap and argmax into self.tok (reference.py:200-207)."""
        qgemv(self.hf, self.lm_rows, self.lm_sc, self.H, self.vocab, bits=2, out=self.logits)
        softcap_argmax(self.logits, self.softcap, tok=self.tok, ws=self.arg_ws)

    def step(self, pos: int, trace: list | None = None):
        """One token at position pos: self.tok in, the next token in self.tok out."""
        self.embed_token()
        if trace is not None:
            trace.append({"x": self.x.clone(), "ple_in": self.ple_in.clone()})
        prev = None
        for L in range(self.nL):
            t = {} if trace is not None else None
            self.layer(L, pos, t, prev)
            if trace is not None:
                trace.append(t)
            prev = t
        self.head()
        return self.tok
