"""GPU parity of g4a_rows_tail, the row tail between the decoder prefill's GEMMs (rmsadd_b,
srqh_b, rmssrq_69, rmssrqh_b; kernels_dsl.py:158-206, 233-242, 622-710), against
oracle/decoder.py's rmsadd and tail_operand, through the C ABI.

Rows of n % 8 == 0 values run on the wave-per-row kernel, others on the workgroup-per-row
kernel; both are covered, with every mode, with and without the residual add, at the E2B
width (1536) and at the ends of the range (8, 4096). The updated residual is held to
2e-3 + 1e-2|ref| (the two kernels sum the squares in different f32 orders), the f16
operand to the oracle's f16(srq(., q2)) or one grid step beside it for a few values that sit
on a rounding midpoint.
"""
import ctypes

import numpy as np
import pytest
import torch

import oracle.decoder as OD
from helpers import contract_close
from slang_amd import _lib
from slang_amd.decoder import rows_tail

pytestmark = pytest.mark.gpu
DEV = "cuda"
MODES = {"none": _lib.TAIL_NONE, "srq": _lib.TAIL_SRQ, "norm": _lib.TAIL_NORM, "norm16": _lib.TAIL_NORM16}


def t(x):
    return torch.from_numpy(np.ascontiguousarray(x)).to(DEV)


def srq16_close(got16, ref16, step, what, frac=0.05):
    got = np.asarray(got16, np.float16).astype(np.float64)
    ref = np.asarray(ref16, np.float16).astype(np.float64)
    d = np.abs(got - ref)
    ulp = np.spacing(np.abs(ref.astype(np.float16))).astype(np.float64)
    assert (d <= step * 1.001 + ulp).all(), f"{what}: a value {d.max() / max(step, 1e-30):.2f} grid steps off"
    assert (d > ulp).mean() <= frac, f"{what}: {(d > ulp).mean():.2%} of the values one step off"


@pytest.mark.parametrize("rows,n", [(1024, 1536), (37, 4096), (5, 8), (9, 1000), (6, 1001)])
@pytest.mark.parametrize("mode", ["none", "srq", "norm", "norm16"])
@pytest.mark.parametrize("add", [True, False])
def test_rows_tail_matches_oracle(rows, n, mode, add):
    print(f"rows_tail rows {rows} n {n} mode {mode} add {add}", flush=True)
    if mode == "none" and not add:
        # no residual add and no operand: nothing to do, which the C ABI refuses before launching
        h = t(np.zeros((rows, n), np.float32))
        rc = _lib.load().g4a_rows_tail(rows, n, None, 0.0, None, 1.0, 1e-6, ctypes.c_void_p(h.data_ptr()),
                                       MODES["none"], None, 0.0, None, None)
        assert rc == -1, f"rc {rc}, expected G4A_EINVAL"
        assert "x16 or a mode" in _lib.load().g4a_last_error().decode()
        with pytest.raises(Exception, match="x16 or a mode"):
            rows_tail(h)
        return
    rng = np.random.default_rng(rows * 7 + n + len(mode) + add)
    hid = rng.standard_normal((rows, n)).astype(np.float32)
    x16 = (rng.standard_normal((rows, n)) * 3).astype(np.float16) if add else None
    w1 = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
    w2 = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
    x_q, q2, mult = 0.0625, 0.03125, 0.75
    h_d = t(hid)
    y = rows_tail(h_d, t(x16) if add else None, x_q=x_q, w1=t(w1), mult=mult, mode=MODES[mode], w2=t(w2), q2=q2)
    torch.cuda.synchronize()
    ref_h = OD.rmsadd(hid, x16, x_q, w1, mult) if add else hid
    got_h = h_d.cpu().numpy()
    if add:
        contract_close(got_h, ref_h, "residual")
    else:
        np.testing.assert_array_equal(got_h, hid)
    if mode != "none":
        # the operand from the GPU's own residual: the norm's f32 order is the kernel's only freedom
        ref_y = OD.tail_operand(got_h, mode, w2, q2)
        srq16_close(y.cpu().numpy(), ref_y, q2, f"operand ({mode})")
