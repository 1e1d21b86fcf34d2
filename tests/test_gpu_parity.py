"""GPU parity: the pattern kernels (through libsc's C ABI) against the CPU
oracle on the same seeded inputs.

Floating point: max relative error <= 1e-5 normalised by (|A| |B|)_ij
against the fp64 product of the same fp32 operands.
Integer-valued inputs (the reference's all-ones fixture matrix times a
small-integer B): every partial sum is exact in fp32, so the GPU result must
equal the oracle's spmm_csr_float / spmv_csr_float restatement bit for bit.
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
# the km-row pattern layout only: these tests cover the pattern kernels (the
# one-row layout that default plans also hold is covered in test_gpu_rows.py)
PAT = sc_amd.PLAN_PATTERNS


def run_spmm(A, B, km, kn, flags=0, waves=0, accumulate=None):
    cf = sc_amd.Cfmtx.build(A, km, kn)
    plan = sc_amd.Plan(cf, flags | sc_amd.PLAN_PATTERNS)
    Bt = torch.from_numpy(np.ascontiguousarray(B, np.float32)).to(DEV)
    if accumulate is not None:
        Ct = torch.from_numpy(accumulate.copy()).to(DEV)
        plan.spmm(Bt, Ct, accumulate=True, waves=waves)
    else:
        Ct = torch.full((A.shape[0], B.shape[1]), float("nan"), device=DEV)  # must be overwritten
        plan.spmm(Bt, Ct, waves=waves)
    torch.cuda.synchronize()
    return Ct.cpu().numpy()


@pytest.mark.parametrize("n", [1, 2, 4, 32, 64, 128])
@pytest.mark.parametrize("km", [1, 2, 3, 4, 5, 6])
def test_spmm_512_uniform(km, n):
    A, B = synth_case(512, 512, 0.10, n, seed=0x5EED0000 + 2000 + km * 10 + n)
    C = run_spmm(A, B, km, 1)
    err, _ = oracle_check(A, B, C)
    assert err <= REL_TOL, (km, n, err)


@pytest.mark.parametrize("kn", [2, 3, 5, 8, 0])
def test_spmm_column_packs(kn):
    A, B = synth_case(512, 512, 0.20, 32, seed=0x5EED0000 + 1000 + kn)
    C = run_spmm(A, B, 4, kn)
    err, _ = oracle_check(A, B, C)
    assert err <= REL_TOL, (kn, err)


@pytest.mark.parametrize("n", [3, 5, 33, 100, 256, 300, 512])
def test_spmm_odd_and_wide_n(n):
    A, B = synth_case(96, 160, 0.15, n, seed=0x5EED0000 + 7000 + n)
    C = run_spmm(A, B, 4, 1)
    err, _ = oracle_check(A, B, C)
    assert err <= REL_TOL, (n, err)


@pytest.mark.parametrize("n", [33, 100, 128])
@pytest.mark.parametrize("waves", [0, 1, 5])
def test_spmm_n_chunks_split_over_workgroups(n, waves):
    # 128 long panels, fewer than the CUs: the lanes-over-slots kernel gives
    # each panel two workgroups, one per half of the N chunk (grid 128 x 2)
    A, B = synth_case(512, 2048, 0.30, n, seed=0x5EED0000 + 7300 + n)
    plan = sc_amd.Plan(sc_amd.Cfmtx.build(A, 4, 1), PAT)
    d = plan.describe(n)
    assert d.startswith("panel_kernel") and "grid=128x2" in d, d
    Bt = torch.from_numpy(np.ascontiguousarray(B, np.float32)).to(DEV)
    Ct = torch.full((512, n), float("nan"), device=DEV)
    plan.spmm(Bt, Ct, waves=waves)
    torch.cuda.synchronize()
    assert oracle_check(A, B, Ct.cpu().numpy())[0] <= REL_TOL
    C0 = np.random.default_rng(n).standard_normal((512, n)).astype(np.float32)
    Ct = torch.from_numpy(C0.copy()).to(DEV)
    plan.spmm(Bt, Ct, accumulate=True, waves=waves)
    torch.cuda.synchronize()
    assert oracle_check_acc(A, B, Ct.cpu().numpy(), C0) <= REL_TOL


@pytest.mark.parametrize("waves", [1, 2, 3, 8, 16])
def test_spmm_waves_per_panel(waves):
    A, B = synth_case(256, 384, 0.25, 64, seed=0x5EED0000 + 8000 + waves)
    C = run_spmm(A, B, 4, 2, waves=waves)
    err, _ = oracle_check(A, B, C)
    assert err <= REL_TOL, (waves, err)


def test_spmm_ragged_rows_and_empty_rows():
    # 37 rows (not a multiple of km), rows 5..12 and the last row empty
    rng = np.random.default_rng(5)
    dense = (rng.random((37, 53)) < 0.3) * rng.standard_normal((37, 53))
    dense[5:13] = 0
    dense[-1] = 0
    ip = np.concatenate([[0], np.cumsum((dense != 0).sum(1))]).astype(np.int32)
    ix = np.nonzero(dense)[1].astype(np.int32)
    dx = dense[dense != 0].astype(np.float32).astype(np.float64)
    A = sc_amd.Csr.from_arrays(37, 53, ip, ix, dx)
    B = sc_amd.synth_dense(53 * 8, 77).reshape(53, 8)
    for km in (1, 3, 4, 5, 6):
        C = run_spmm(A, B, km, 2)
        err, _ = oracle_check(A, B, C)
        assert err <= REL_TOL, (km, err)
        assert np.all(C[5:13] == 0) and np.all(C[-1] == 0)


def test_spmm_empty_matrix_overwrites_c():
    A = sc_amd.Csr.from_arrays(10, 12, np.zeros(11, np.int32), [], [])
    B = sc_amd.synth_dense(12 * 4, 3).reshape(12, 4)
    C = run_spmm(A, B, 4, 1)
    assert np.all(C == 0)


def test_spmm_accumulate_flag():
    A, B = synth_case(128, 128, 0.2, 32, seed=11)
    C0 = sc_amd.synth_dense(128 * 32, 12).reshape(128, 32)
    C = run_spmm(A, B, 4, 1, accumulate=C0)
    ip, ix, ax = csr_f32(A)
    c64, cab = O.spmm_f64(128, 32, ip, ix, ax, B)
    err = O.max_rel_err(C - C0.astype(np.float64), c64, cab + np.abs(C0))
    assert err <= REL_TOL


def test_spmm_drop_padding_plan():
    # Dropping the zero padding moves the slot split between waves, so the
    # fp32 summation order (not the exact sum) changes: both must pass the
    # tolerance, and the plan must hold fewer slots.
    A, B = synth_case(512, 512, 0.2, 64, seed=21)
    cf = sc_amd.Cfmtx.build(A, 4, 8)
    assert (sc_amd.Plan(cf, sc_amd.PLAN_DROP_PADDING | PAT).info()["nslots"]
            < sc_amd.Plan(cf, PAT).info()["nslots"])
    C1 = run_spmm(A, B, 4, 8)
    C2 = run_spmm(A, B, 4, 8, flags=sc_amd.PLAN_DROP_PADDING)
    assert oracle_check(A, B, C1)[0] <= REL_TOL
    assert oracle_check(A, B, C2)[0] <= REL_TOL


@pytest.mark.parametrize("flags", [0, sc_amd.PLAN_CHUNKED])
@pytest.mark.parametrize("n", [1, 32, 128])
def test_spmm_structured_4096(n, flags):
    A, B = synth_case(4096, 4096, 0.10, n, seed=0x5EED0000 + 4000 + n, structured=True)
    C = run_spmm(A, B, 4, 1, flags=flags)
    err, _ = oracle_check(A, B, C)
    assert err <= REL_TOL, (n, err)


@pytest.mark.parametrize("km,kn", [(4, 2), (4, 3), (2, 5), (6, 8), (1, 2), (3, 1)])
def test_fixture_matrix_bit_exact(km, kn, reference_matrix_dir):
    """The reference's own matrix (values 1, committed under tests/golden)
    times integer B: exact sums."""
    A = sc_amd.Csr.from_mtx(os.path.join(reference_matrix_dir, FIXTURE_STEM + ".mtx"))
    assert A.shape == (512, 512) and A.nnz == 104857
    rng = np.random.default_rng(km * 10 + kn)
    for n in (1, 4, 64):
        B = rng.integers(-3, 4, size=(512, n)).astype(np.float32)
        C = run_spmm(A, B, km, kn)
        ip, ix, ax = csr_f32(A)
        ref = O.spmm_csr_float(512, n, ip, ix, ax, B)
        assert np.array_equal(C, ref), (km, kn, n)


def test_reference_cfmtx_file_bit_exact(reference_matrix_dir):
    """The reference's own km 4 x kn 2 .cfmtx, read by the .cfmtx reader with
    its companion .mtx (loadCfmtxMatrices), on every layout: exact sums."""
    A, cf = sc_amd.load_cfmtx_matrices(os.path.join(reference_matrix_dir, FIXTURE_STEM + "-4-2.cfmtx"))
    ip, ix, ax = csr_f32(A)
    rng = np.random.default_rng(42)
    for n in (1, 4, 32, 128):
        B = rng.integers(-3, 4, size=(512, n)).astype(np.float32)
        ref = O.spmm_csr_float(512, n, ip, ix, ax, B)
        Bt = torch.from_numpy(B).to(DEV)
        for flags in (0, sc_amd.PLAN_PATTERNS, sc_amd.PLAN_ROWS):
            C = sc_amd.Plan(cf, flags).spmm(Bt)
            torch.cuda.synchronize()
            assert np.array_equal(C.cpu().numpy(), ref), (n, flags)


def test_spmv_matches_reference_cpu_path():
    A, B = synth_case(512, 512, 0.30, 1, seed=0x5EED0000 + 0)
    cf = sc_amd.Cfmtx.build(A, 1, 1)
    plan = sc_amd.Plan(cf, PAT)
    x = torch.from_numpy(B[:, 0].copy()).to(DEV)
    y = plan.spmv(x)
    torch.cuda.synchronize()
    y = y.cpu().numpy()
    err, _ = oracle_check(A, B, y.reshape(-1, 1))
    assert err <= REL_TOL
    ip, ix, ax = csr_f32(A)
    ycpu = O.spmv_csr_float(512, ip, ix, ax, B[:, 0])
    assert np.max(np.abs(y - ycpu)) <= 1e-5 * max(1.0, float(np.abs(ycpu).max()))


def test_plan_rejects_bad_device_buffer_shapes():
    A, B = synth_case(64, 64, 0.2, 4, seed=1)
    plan = sc_amd.Plan(sc_amd.Cfmtx.build(A, 4, 1), PAT)
    with pytest.raises(ValueError):
        plan.spmm(torch.zeros((63, 4), device=DEV))


@pytest.mark.parametrize("n", [96, 128])
def test_spmm_b_above_2_gib(n):
    # B of more than 2 GiB (n = 128: more than 4 GiB): byte offsets no longer
    # fit a buffer descriptor, so the lanes-over-slots kernel reads B through
    # 64-bit pointers (and the wide kernel hands N = 128 over to it); a skinny
    # A with a few thousand entries spread over all of K
    K = (2 ** 31 // (4 * n) + 4099) if n == 96 else (2 ** 32 // (4 * n) + 4099)
    A = sc_amd.Csr.synth_uniform(64, K, 3000 / (64 * K), 0.05, 0x5EED0000 + 9800 + n)
    gen = torch.Generator(device=DEV).manual_seed(n)
    Bt = torch.empty((K, n), dtype=torch.float32, device=DEV).uniform_(-1.0, 1.0, generator=gen)
    plan = sc_amd.Plan(sc_amd.Cfmtx.build(A, 4, 1), PAT)
    assert plan.describe(n).startswith("panel_kernel")
    C = plan.spmm(Bt)
    torch.cuda.synchronize()
    # the oracle on the B rows A touches only
    ip, ix, ax = csr_f32(A)
    used, local = np.unique(ix, return_inverse=True)
    Bs = Bt.index_select(0, torch.from_numpy(used.astype(np.int64)).to(DEV)).cpu().numpy()
    del Bt
    c64, cab = O.spmm_f64(64, n, ip, local.astype(np.int32), ax, Bs)
    assert O.max_rel_err(C.cpu().numpy(), c64, cab) <= REL_TOL


def test_spmm_wide_unstaged_dense_panels():
    # panels of km=6 rows over 4096 dense-ish columns hold more than 64 KiB of
    # stream, so the wide kernel reads columns/values from global memory
    A, B = synth_case(12, 4096, 0.9, 128, seed=31)
    C = run_spmm(A, B, 6, 1)
    err, _ = oracle_check(A, B, C)
    assert err <= REL_TOL, err


@pytest.mark.parametrize("n", [64, 128, 256])
@pytest.mark.parametrize("flags", [0, sc_amd.PLAN_TILED, sc_amd.PLAN_CHUNKED])
def test_spmm_split_k_ragged(n, flags):
    # 2050 x 3001: K not a multiple of the B tile, M not a multiple of the
    # row block; with PLAN_TILED enough reuse for the split-K LDS-tiled kernel
    A, B = synth_case(2050, 3001, 0.10, n, seed=0x5EED0000 + 9000 + n)
    C = run_spmm(A, B, 4, 1, flags=flags)
    err, _ = oracle_check(A, B, C)
    assert err <= REL_TOL, (n, err)
    C0 = sc_amd.synth_dense(2050 * n, 17).reshape(2050, n)
    Cacc = run_spmm(A, B, 4, 1, flags=flags, accumulate=C0)
    ip, ix, ax = csr_f32(A)
    c64, cab = O.spmm_f64(2050, n, ip, ix, ax, B)
    assert O.max_rel_err(Cacc - C0.astype(np.float64), c64, cab + np.abs(C0)) <= REL_TOL


@pytest.mark.parametrize("n", [64, 128, 256])
def test_tiled_split_k_back_to_back_inputs(n):
    # split-K units hand partial sums to the last unit of each row block
    # through the plan workspace; successive launches on one plan with
    # different B (and a different N in between) must each see only their
    # own partials, and every launch leaves the arrival counters at zero
    A, B1 = synth_case(1500, 2300, 0.12, n, seed=0x5EED0000 + 9100 + n)
    B2 = sc_amd.synth_dense(2300 * n, 0x5EED0000 + 9150 + n).reshape(2300, n)
    B3 = sc_amd.synth_dense(2300 * 64, 0x5EED0000 + 9170).reshape(2300, 64)
    plan = sc_amd.Plan(sc_amd.Cfmtx.build(A, 4, 1), sc_amd.PLAN_TILED)
    assert plan.describe(n).startswith("tiled_kernel")
    for Bx in (B1, B2, B3, B1):
        Ct = torch.full((1500, Bx.shape[1]), float("nan"), device=DEV)
        plan.spmm(torch.from_numpy(Bx).to(DEV), Ct)
        torch.cuda.synchronize()
        assert oracle_check(A, Bx, Ct.cpu().numpy())[0] <= REL_TOL


@pytest.mark.parametrize("flags", [0, sc_amd.PLAN_TILED, sc_amd.PLAN_CHUNKED])
def test_spmm_is_deterministic(flags):
    A, B = synth_case(4096, 4096, 0.10, 128, seed=77, structured=True)
    cf = sc_amd.Cfmtx.build(A, 4, 1)
    plan = sc_amd.Plan(cf, flags | sc_amd.PLAN_PATTERNS)
    Bt = torch.from_numpy(B).to(DEV)
    C1 = plan.spmm(Bt).cpu().numpy()
    C2 = plan.spmm(Bt).cpu().numpy()
    assert np.array_equal(C1, C2)
    assert oracle_check(A, B, C1)[0] <= REL_TOL


@pytest.mark.parametrize("n", [32, 64, 96, 128, 512])
@pytest.mark.parametrize("km,kn", [(1, 1), (2, 3), (3, 1), (4, 2), (5, 1), (6, 8)])
def test_chunk_kernel_coarsen_factors(km, kn, n):
    # B column chunks in LDS: every km, packs with padding slots, one K tile
    A, B = synth_case(300, 700, 0.12, n, seed=0x5EED0000 + 9500 + km * 10 + kn + n)
    cf = sc_amd.Cfmtx.build(A, km, kn)
    plan = sc_amd.Plan(cf, sc_amd.PLAN_CHUNKED)
    assert plan.describe(n).startswith("chunk_kernel")
    C = run_spmm(A, B, km, kn, flags=sc_amd.PLAN_CHUNKED)
    err, _ = oracle_check(A, B, C)
    assert err <= REL_TOL, (km, kn, n, err)


def test_chunk_kernel_tiles_and_ragged_k():
    # K = 2600: three LDS tiles, the last one partial; M ragged; accumulate
    A, B = synth_case(1030, 2600, 0.08, 64, seed=0x5EED0000 + 9600)
    C = run_spmm(A, B, 4, 1, flags=sc_amd.PLAN_CHUNKED)
    assert oracle_check(A, B, C)[0] <= REL_TOL
    C0 = sc_amd.synth_dense(1030 * 64, 18).reshape(1030, 64)
    Cacc = run_spmm(A, B, 4, 1, flags=sc_amd.PLAN_CHUNKED, accumulate=C0)
    ip, ix, ax = csr_f32(A)
    c64, cab = O.spmm_f64(1030, 64, ip, ix, ax, B)
    assert O.max_rel_err(Cacc - C0.astype(np.float64), c64, cab + np.abs(C0)) <= REL_TOL


def test_chunk_kernel_not_used_for_unsorted_segments(tmp_path):
    # a hand-written .cfmtx whose segment lists columns out of order: the plan
    # builds no column splits and the kernel falls back, still correct
    p = tmp_path / "u.cfmtx"
    p.write_text("4 8 4 1 1\n1111 0 \n0 2\n5 1\n"
                 "1.0 2.0 3.0 4.0 5.0 6.0 7.0 8.0\n")
    cf = sc_amd.Cfmtx.read(str(p))
    plan = sc_amd.Plan(cf, sc_amd.PLAN_CHUNKED)
    assert not plan.describe(32).startswith("chunk_kernel")
    B = sc_amd.synth_dense(8 * 32, 5).reshape(8, 32)
    C = plan.spmm(torch.from_numpy(B).to(DEV)).cpu().numpy()
    A = np.zeros((4, 8))
    A[:, 5] = [1, 2, 3, 4]
    A[:, 1] = [5, 6, 7, 8]
    assert np.allclose(C, A @ B.astype(np.float64), rtol=1e-6, atol=1e-6)


def test_chunk_kernel_generated_unit():
    # a unit from the reference-compatible generator CLI (km 3, kn 1) runs
    # through the chunk kernel on a chunked plan
    unit = sc_amd.GeneratedUnit(os.path.join(os.path.dirname(sc_amd.LIB_PATH), "units",
                                             "libsc_unit_spmm_km3_kn1.so"), "spmm_km3_kn1")
    A, B = synth_case(600, 1500, 0.1, 64, seed=0x5EED0000 + 9700)
    plan = sc_amd.Plan(sc_amd.Cfmtx.build(A, 3, 1), sc_amd.PLAN_CHUNKED)
    C = plan.spmm_generated(unit, torch.from_numpy(B).to(DEV))
    torch.cuda.synchronize()
    assert oracle_check(A, B, C.cpu().numpy())[0] <= REL_TOL


@pytest.mark.parametrize("n", [1, 2, 4])
@pytest.mark.parametrize("waves", [0, 1, 3, 8, 16])
def test_small_n_gather_kernel(n, waves):
    # N = 1, 2, 4: B rows of the panel gathered into LDS before the pattern
    # bodies run; ragged M, several waves per panel, accumulate
    A, B = synth_case(515, 700, 0.15, n, seed=0x5EED0000 + 9800 + n * 20 + waves)
    plan = sc_amd.Plan(sc_amd.Cfmtx.build(A, 4, 2), PAT)
    assert plan.describe(n).startswith("gather_kernel")
    C = run_spmm(A, B, 4, 2, waves=waves)
    assert oracle_check(A, B, C)[0] <= REL_TOL
    C0 = sc_amd.synth_dense(515 * n, 19).reshape(515, n)
    Cacc = run_spmm(A, B, 4, 2, waves=waves, accumulate=C0)
    ip, ix, ax = csr_f32(A)
    c64, cab = O.spmm_f64(515, n, ip, ix, ax, B)
    assert O.max_rel_err(Cacc - C0.astype(np.float64), c64, cab + np.abs(C0)) <= REL_TOL


@pytest.mark.parametrize("n", [2, 4])
def test_small_n_gather_kernel_generated_pack_unit(n):
    # a kn = 2 unit from the generator CLI: its bodies step two slots at a time
    unit = sc_amd.GeneratedUnit(os.path.join(os.path.dirname(sc_amd.LIB_PATH), "units",
                                             "libsc_unit_spmm_km4_kn2.so"), "spmm_km4_kn2")
    A, B = synth_case(256, 300, 0.2, n, seed=0x5EED0000 + 9900 + n)
    plan = sc_amd.Plan(sc_amd.Cfmtx.build(A, 4, 2), PAT)
    C = plan.spmm_generated(unit, torch.from_numpy(B).to(DEV))
    torch.cuda.synchronize()
    assert oracle_check(A, B, C.cpu().numpy())[0] <= REL_TOL


def test_tiled_first_launch_captured_in_a_graph():
    # a tiled plan owns its split-K workspace from creation: its very first
    # launch may sit inside a HIP graph capture (no allocation in the launch)
    A, B = synth_case(1000, 700, 0.2, 128, seed=0x5EED0000 + 7500)
    plan = sc_amd.Plan(sc_amd.Cfmtx.build(A, 4, 1), sc_amd.PLAN_TILED)
    assert plan.describe(128).startswith("tiled_kernel"), plan.describe(128)
    Bt = torch.from_numpy(B).to(DEV)
    Ct = torch.full((1000, 128), float("nan"), device=DEV)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        plan.spmm(Bt, Ct)
    ref = None
    for i in range(3):
        Ct.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        C = Ct.cpu().numpy()
        assert oracle_check(A, B, C)[0] <= REL_TOL, i
        ref = C if ref is None else ref
        assert np.array_equal(C, ref), i


@pytest.mark.parametrize("n", [32, 40, 128])
def test_launch_order_with_skewed_panels(n):
    # 1031 panels (four groups of CUs hold one more panel than the rest) whose
    # slot counts differ by 30x: the plan's launch order moves most panels
    # to another workgroup, and every panel must still be run exactly once
    rng = np.random.default_rng(0x5EED0000 + 9100 + n)
    m, k = 4 * 1031 - 2, 640
    dens = np.where(np.arange(m) % 97 < 9, 0.6, 0.02)
    mask = rng.random((m, k)) < dens[:, None]
    vals = rng.standard_normal(int(mask.sum())) * 0.05
    ip = np.concatenate([[0], np.cumsum(mask.sum(1))]).astype(np.int32)
    ix = np.nonzero(mask)[1].astype(np.int32)
    A = sc_amd.Csr.from_arrays(m, k, ip, ix, vals.astype(np.float32).astype(np.float64))
    B = sc_amd.synth_dense(k * n, 0x5EED0000 + 9200 + n).reshape(k, n)
    for km in (4, 3):
        C = run_spmm(A, B, km, 1)
        err, _ = oracle_check(A, B, C)
        assert err <= REL_TOL, (km, err)
    # the one-row layout of the same slots (4122 one-row panels)
    plan = sc_amd.Plan(sc_amd.Cfmtx.build(A, 4, 1), sc_amd.PLAN_ROWS)
    Bt = torch.from_numpy(np.ascontiguousarray(B, np.float32)).to(DEV)
    Ct = torch.full((m, n), float("nan"), device=DEV)
    plan.spmm(Bt, Ct)
    torch.cuda.synchronize()
    err, _ = oracle_check(A, B, Ct.cpu().numpy())
    assert err <= REL_TOL, ("rows", plan.describe(n), err)


def test_default_plan_launches_on_two_streams_at_once():
    # a default plan holds no launch state: launches of one plan on two
    # streams, interleaved with no ordering between them, both match the oracle
    A, B1 = synth_case(1024, 768, 0.1, 128, seed=0x5EED0000 + 9300)
    B2 = sc_amd.synth_dense(768 * 128, 0x5EED0000 + 9301).reshape(768, 128)
    plan = sc_amd.Plan(sc_amd.Cfmtx.build(A, 4, 1), 0)
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    Bt = [torch.from_numpy(B1).to(DEV), torch.from_numpy(B2).to(DEV)]
    Ct = [torch.full((1024, 128), float("nan"), device=DEV) for _ in range(2)]
    torch.cuda.synchronize()
    for _ in range(8):
        plan.spmm(Bt[0], Ct[0], stream=s1)
        plan.spmm(Bt[1], Ct[1], stream=s2)
    torch.cuda.synchronize()
    for B, Cg in ((B1, Ct[0]), (B2, Ct[1])):
        err, _ = oracle_check(A, B, Cg.cpu().numpy())
        assert err <= REL_TOL, err


@pytest.mark.parametrize("n", [32, 64, 128])
def test_large_b_every_coarsen_factor(n):
    # BASELINE config 2 as the sweep times it (same matrix seed and B): every
    # km 1..6 x kn 1..8 file, on the default plan and on the pattern layout
    A = sc_amd.Csr.synth_uniform(512, 512, 0.10, 0.05, 0x5EED0000 + 2000)
    B = sc_amd.synth_dense(512 * n, 0x5EED0000 + 500 + n).reshape(512, n)
    Bt = torch.from_numpy(B).to(DEV)
    for km in range(1, 7):
        for kn in range(1, 9):
            cf = sc_amd.Cfmtx.build(A, km, kn)
            for flags in (0, PAT):
                plan = sc_amd.Plan(cf, flags)
                Ct = torch.full((512, n), float("nan"), device=DEV)
                plan.spmm(Bt, Ct)
                torch.cuda.synchronize()
                err, _ = oracle_check(A, B, Ct.cpu().numpy())
                assert err <= REL_TOL, (km, kn, flags, plan.describe(n), err)
