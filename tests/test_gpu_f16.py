"""GPU: the binary16 small-B path (sc_spmm_f16: the plan's binary16 values,
binary16 B and C, N = 1, 2, 4, fp32 accumulation, C rounded once) against the
fp64 product of the same binary16 operands.

The reference's fp16 small-B kernels (PatternWith{pop}NNZByRowPanelFullHALF,
example_cuda/spmm_small_b_col_demo_gpu_utils.h:2987-5017) accumulate in
binary16 and are never run by a reference driver, so there is no reference
output to match bit for bit; the bar here is the rounding bound of one
binary16 rounding of an fp32-accumulated sum: |C - exact| <= 2^-11 |exact| +
1e-6 (|A||B|) + 2^-25 (half the binary16 subnormal spacing)."""
import numpy as np
import pytest

import sc_amd
from cases import synth_case

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def f16_reference(A, B16):
    """fp64 product of the binary16-rounded values of A and B16, and |A||B|."""
    ip, ix, dx = A.arrays()
    a16 = dx.astype(np.float32).astype(np.float16).astype(np.float64)
    m = A.shape[0]
    n = B16.shape[1]
    b = B16.astype(np.float64)
    c = np.zeros((m, n))
    cab = np.zeros((m, n))
    rows = np.repeat(np.arange(m), np.diff(ip))
    np.add.at(c, rows, a16[:, None] * b[ix])
    np.add.at(cab, rows, np.abs(a16[:, None]) * np.abs(b[ix]))
    return c, cab


def within_f16_bound(C16, c, cab):
    err = np.abs(C16.astype(np.float64) - c)
    bound = 2.0 ** -11 * np.abs(c) + 1e-6 * cab + 2.0 ** -25
    return bool(np.all(err <= bound)), float(np.max(err - bound))


# 0: the default plan (its one-row layout at these sizes); PLAN_PATTERNS: the
# km-row pattern layout alone
LAYOUTS = [0, sc_amd.PLAN_PATTERNS]


@pytest.mark.parametrize("layout", LAYOUTS)
@pytest.mark.parametrize("n", [1, 2, 4])
@pytest.mark.parametrize("km,kn", [(1, 1), (2, 3), (4, 1), (4, 2), (6, 8)])
def test_spmm_f16_matches_rounded_product(km, kn, n, layout):
    A, B = synth_case(515, 700, 0.15, n, seed=0x5EED0000 + 9950 + km * 10 + kn + n, sigma=0.5)
    B16 = B.astype(np.float16)
    plan = sc_amd.Plan(sc_amd.Cfmtx.build(A, km, kn), sc_amd.PLAN_F16_VALUES | layout)
    C16 = plan.spmm_f16(torch.from_numpy(B16).to(DEV)).cpu().numpy()
    c, cab = f16_reference(A, B16)
    ok, worst = within_f16_bound(C16, c, cab)
    assert ok, (km, kn, n, worst)
    # the fp32 path on the same plan is unaffected
    C32 = plan.spmm(torch.from_numpy(B).to(DEV)).cpu().numpy()
    assert C32.dtype == np.float32 and np.isfinite(C32).all()


@pytest.mark.parametrize("layout", LAYOUTS)
@pytest.mark.parametrize("waves", [1, 8])
def test_spmm_f16_accumulate(waves, layout):
    A, B = synth_case(256, 300, 0.2, 4, seed=0x5EED0000 + 9990 + waves, sigma=0.5)
    B16 = B.astype(np.float16)
    C0 = sc_amd.synth_dense(256 * 4, 23).reshape(256, 4).astype(np.float16)
    plan = sc_amd.Plan(sc_amd.Cfmtx.build(A, 4, 1), sc_amd.PLAN_F16_VALUES | layout)
    Ct = torch.from_numpy(C0.copy()).to(DEV)
    plan.spmm_f16(torch.from_numpy(B16).to(DEV), Ct, accumulate=True, waves=waves)
    c, cab = f16_reference(A, B16)
    ok, worst = within_f16_bound(Ct.cpu().numpy(), c + C0.astype(np.float64), cab + np.abs(C0))
    assert ok, worst


def test_spmm_f16_rejections():
    A, B = synth_case(64, 64, 0.2, 4, seed=0x5EED0000 + 9999)
    B16 = torch.from_numpy(B.astype(np.float16)).to(DEV)
    plain = sc_amd.Plan(sc_amd.Cfmtx.build(A, 4, 1))
    with pytest.raises(sc_amd.LibscError, match="SC_PLAN_F16_VALUES"):
        plain.spmm_f16(B16)
    plan = sc_amd.Plan(sc_amd.Cfmtx.build(A, 4, 1), sc_amd.PLAN_F16_VALUES)
    B3 = torch.zeros((64, 3), dtype=torch.float16, device=DEV)
    with pytest.raises(sc_amd.LibscError, match="N = 1, 2 or 4"):
        plan.spmm_f16(B3)
