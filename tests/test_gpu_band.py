"""GPU parity of the band kernel (SC_PLAN_BANDS, kernel_m 4, N a multiple of
64): B staged in LDS once per (band of panels, K range of up to 512 rows),
every slot on the matrix cores (four slots of one panel to an item, whatever
their patterns), split K over the ranges with the plan's workspace.  Against
the CPU oracle on the same inputs.

Floating point: max relative error <= 1e-5 normalised by (|A| |B|)_ij
against the fp64 product of the same fp32 operands (with accumulate, by
(|A| |B|)_ij + |C0_ij| against C0 + A*B); integer-valued inputs must come
out exact.
"""
import os

import numpy as np
import pytest

import oracle as O
import sc_amd
from cases import REL_TOL, csr_f32, oracle_check, oracle_check_acc, synth_case
from conftest import FIXTURE_STEM

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

DEV = "cuda:0"
BANDS = sc_amd.PLAN_BANDS


def run(plan, B, accumulate=None):
    Bt = torch.from_numpy(np.ascontiguousarray(B, np.float32)).to(DEV)
    if accumulate is not None:
        Ct = torch.from_numpy(accumulate.copy()).to(DEV)
        plan.spmm(Bt, Ct, accumulate=True)
    else:
        Ct = torch.full((plan.info()["m"], B.shape[1]), float("nan"), device=DEV)  # must be overwritten
        plan.spmm(Bt, Ct)
    torch.cuda.synchronize()
    return Ct.cpu().numpy()


@pytest.mark.parametrize("n", [64, 128, 256])
def test_band_structured_4096(n):
    # the headline matrix: 4x4 blocks (all-ones slots) and 1x8 vectors
    A, B = synth_case(4096, 4096, 0.10, n, seed=0x5EED0000 + 4000 + n, structured=True)
    plan = sc_amd.Plan(sc_amd.Cfmtx.build(A, 4, 1), BANDS)
    assert plan.describe(n).startswith("band_kernel"), plan.describe(n)
    C = run(plan, B)
    err, _ = oracle_check(A, B, C)
    assert err <= REL_TOL, (n, plan.describe(n), err)


@pytest.mark.parametrize("shape,density,n", [
    ((512, 512), 0.10, 64),      # 8 bands of 16 panels, one K range
    ((1000, 700), 0.20, 128),    # ragged last band and panel, two K ranges, the last short
    ((37, 53), 0.30, 64),        # one band, one panel row short, one K range
    ((2048, 512), 0.50, 128),    # FFN shapes
    ((512, 2048), 0.10, 192),    # three N chunks
    ((256, 4096), 0.02, 64),     # long K: eight K ranges
])
def test_band_uniform_shapes(shape, density, n):
    m, k = shape
    A, B = synth_case(m, k, density, n, seed=0x5EED0000 + 7000 + m + k + n)
    plan = sc_amd.Plan(sc_amd.Cfmtx.build(A, 4, 1), BANDS)
    assert plan.describe(n).startswith("band_kernel"), plan.describe(n)
    C = run(plan, B)
    err, _ = oracle_check(A, B, C)
    assert err <= REL_TOL, (shape, n, plan.describe(n), err)


@pytest.mark.parametrize("kn,drop", [(2, 0), (4, 0), (3, sc_amd.PLAN_DROP_PADDING), (0, 0)])
def test_band_column_packs(kn, drop):
    # the format's zero padding slots are skipped: even kn = 0 (packs of
    # 32 // pop) fits the band layout
    A, B = synth_case(600, 900, 0.15, 64, seed=0x5EED0000 + 7100 + kn)
    plan = sc_amd.Plan(sc_amd.Cfmtx.build(A, 4, kn), BANDS | drop)
    assert plan.describe(64).startswith("band_kernel"), plan.describe(64)
    C = run(plan, B)
    err, _ = oracle_check(A, B, C)
    assert err <= REL_TOL, (kn, drop, err)


def test_band_accumulate_and_determinism():
    A, B = synth_case(4096, 4096, 0.10, 128, seed=0x5EED0000 + 4128, structured=True)
    plan = sc_amd.Plan(sc_amd.Cfmtx.build(A, 4, 1), BANDS)
    C0 = sc_amd.synth_dense(4096 * 128, 4129).reshape(4096, 128)
    C = run(plan, B, accumulate=C0)
    assert oracle_check_acc(A, B, C, C0) <= REL_TOL
    # split-K partials are added in K-range order: launches agree bit for bit
    C1 = run(plan, B)
    C2 = run(plan, B)
    assert np.array_equal(C1, C2)


def test_band_integer_inputs_exact(reference_matrix_dir):
    # the reference's all-ones matrix times integer B: every sum is exact
    A = sc_amd.Csr.from_mtx(os.path.join(reference_matrix_dir, FIXTURE_STEM + ".mtx"))
    ip, ix, ax = csr_f32(A)
    rng = np.random.default_rng(5)
    for kn in (1, 2):
        plan = sc_amd.Plan(sc_amd.Cfmtx.build(A, 4, kn), BANDS)
        for n in (64, 128):
            B = rng.integers(-3, 4, size=(512, n)).astype(np.float32)
            assert np.array_equal(run(plan, B), O.spmm_csr_float(512, n, ip, ix, ax, B)), (kn, n)


def test_band_falls_back_off_its_shapes():
    # N not a multiple of 64 runs the other kernels of the same plan
    A, B = synth_case(512, 512, 0.10, 32, seed=0x5EED0000 + 7200)
    plan = sc_amd.Plan(sc_amd.Cfmtx.build(A, 4, 1), BANDS)
    assert not plan.describe(32).startswith("band_kernel")
    err, _ = oracle_check(A, B, run(plan, B))
    assert err <= REL_TOL


def test_band_falls_back_beyond_sixteen_k_ranges():
    # K = 20000 needs 40 K ranges of 512 rows: the plan builds no band layout
    # and runs its other kernels; K = 8000 (16 ranges, the last one short)
    # runs the band kernel with its split K over all sixteen
    rng = np.random.default_rng(9)
    for k, band in ((20000, False), (8000, True)):
        A, _ = synth_case(1024, k, 0.002, 1, seed=0x5EED0000 + 7400 + k)
        plan = sc_amd.Plan(sc_amd.Cfmtx.build(A, 4, 1), BANDS)
        assert plan.describe(64).startswith("band_kernel") == band, plan.describe(64)
        if band:
            assert "ks=16" in plan.describe(64), plan.describe(64)
        B = rng.uniform(-1, 1, size=(k, 64)).astype(np.float32)
        err, _ = oracle_check(A, B, run(plan, B))
        assert err <= REL_TOL, (k, err)


def test_band_wave_balance_shapes():
    # bands of 16 to 128 panels (1 to 8 a wave), panels with no slot in a K
    # range, a band whose last panel is short, and waves without panels
    rng = np.random.default_rng(11)
    for m, k, dens in ((4096, 8192, 0.01), (2052, 3000, 0.03), (64, 1100, 0.05), (8, 600, 0.2)):
        A, _ = synth_case(m, k, dens, 1, seed=0x5EED0000 + 7500 + m)
        plan = sc_amd.Plan(sc_amd.Cfmtx.build(A, 4, 1), BANDS)
        assert plan.describe(128).startswith("band_kernel"), plan.describe(128)
        B = rng.uniform(-1, 1, size=(k, 128)).astype(np.float32)
        err, _ = oracle_check(A, B, run(plan, B))
        assert err <= REL_TOL, (m, k, err)


def test_band_empty_matrix_overwrites_c():
    A = sc_amd.Csr.from_arrays(300, 200, np.zeros(301, np.int32), [], [])
    plan = sc_amd.Plan(sc_amd.Cfmtx.build(A, 4, 1), BANDS)
    B = sc_amd.synth_dense(200 * 64, 3).reshape(200, 64)
    assert np.all(run(plan, B) == 0)
