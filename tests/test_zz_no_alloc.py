"""g4a_decode_noalloc (decode with its split partials in the library's own device array, for
callers that cannot allocate) against g4a_decode with a caller workspace, through the C ABI.

Two calls in a row, the second smaller than the first: the array keeps the first call's
partials, which the second must neither need cleared nor read. Outputs are compared bit for
bit with g4a_decode (the same kernels and split plan), and the first call also against the
CPU oracle at the contract tolerance.
"""
import ctypes

import numpy as np
import pytest
import torch

import oracle.attention as O
import slang_amd as sa
from helpers import contract_close
from slang_amd import _lib

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _p(t):
    return ctypes.c_void_p(0 if t is None else t.data_ptr())


def both(cfg, n_seq, max_len, key_len, q, qg, cos, sin, kc, vc):
    """(g4a_decode output, g4a_decode_noalloc output) for the same inputs."""
    lib = _lib.load()
    c = cfg.c(0)
    need = lib.g4a_decode_ws_bytes(ctypes.byref(c), n_seq, max_len)
    assert 0 < need <= _lib.DECODE_SCRATCH_BYTES
    ws = torch.empty(need, dtype=torch.uint8, device=DEV)
    ref = torch.full_like(q, float("nan"))
    got = torch.full_like(q, float("nan"))
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = lib.g4a_decode(ctypes.byref(c), n_seq, max_len, _p(key_len), _p(q), _p(qg), _p(cos), _p(sin), _p(kc),
                        _p(vc), kc.stride(0), _p(ref), _p(ws), ws.numel(), st)
    assert rc == 0, lib.g4a_last_error()
    rc = lib.g4a_decode_noalloc(ctypes.byref(c), n_seq, max_len, _p(key_len), _p(q), _p(qg), _p(cos), _p(sin),
                                _p(kc), _p(vc), kc.stride(0), _p(got), st)
    assert rc == 0, lib.g4a_last_error()
    torch.cuda.synchronize()
    return ref, got


def inputs(seed, n_seq, T, nH=8, kvH=2, hd=256, theta=1e6):
    g = torch.Generator(device=DEV).manual_seed(seed)
    q = torch.randn(n_seq, nH, hd, device=DEV, generator=g)
    qg = 1 + 0.1 * torch.randn(hd, device=DEV, generator=g)
    kc = torch.randn(n_seq, T, kvH, hd, device=DEV, generator=g).half()
    vc = torch.randn(n_seq, T, kvH, hd, device=DEV, generator=g).half()
    return q, qg, kc, vc


def test_noalloc_matches_decode_twice_second_smaller():
    nH, kvH, hd = 8, 2, 256
    # first call: a batch of 4 sequences up to 8192 keys (the work-list plan, the largest partials)
    lens = np.array([8192, 3001, 6500, 1024], np.int32)
    q, qg, kc, vc = inputs(1, 4, 8192)
    cos, sin = (x.to(DEV) for x in sa.rope_tables(lens - 1, hd, 1e6))
    kl = torch.from_numpy(lens).to(DEV)
    cfg = sa.AttnConfig(nH, kvH, hd)
    ref, got = both(cfg, 4, 8192, kl, q, qg, cos, sin, kc, vc)
    assert torch.equal(ref, got), "first call: noalloc differs from g4a_decode"
    qn, kn, vn = q.cpu().numpy(), kc.float().cpu().numpy(), vc.float().cpu().numpy()
    for b, L in enumerate(lens):
        exp = O.decode_attention(qn[b], kn[b], vn[b], int(L), kvH, q_gain=qg.cpu().numpy(),
                                 cos=cos[b].cpu().numpy(), sin=sin[b].cpu().numpy())
        contract_close(got[b].cpu().numpy(), exp, f"noalloc seq {b} T {L}")
    # second call: one sequence of 1000 keys with a sliding window (fewer, smaller partials)
    q2, qg2, kc2, vc2 = inputs(2, 1, 1000)
    c2, s2 = (x.to(DEV) for x in sa.rope_tables([999], hd, 1e4))
    kl2 = torch.tensor([1000], dtype=torch.int32, device=DEV)
    cfg2 = sa.AttnConfig(nH, kvH, hd, 512)
    ref2, got2 = both(cfg2, 1, 1000, kl2, q2, qg2, c2, s2, kc2, vc2)
    assert torch.equal(ref2, got2), "second (smaller) call: noalloc differs from g4a_decode"
    assert torch.isfinite(got2).all()
