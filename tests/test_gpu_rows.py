"""GPU parity of SC_PLAN_ROWS plans: a km > 1 .cfmtx re-laid on the device as
one-row panels (kernel_m 1), against the CPU oracle on the same inputs.

Floating point: max relative error <= 1e-5 normalised by (|A| |B|)_ij
against the fp64 product of the same fp32 operands; integer-valued inputs
must come out exact.
"""
import numpy as np
import pytest

import sc_amd
from cases import REL_TOL, oracle_check, oracle_check_acc, synth_case

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def run(A, B, km, kn, flags=sc_amd.PLAN_ROWS, accumulate=None):
    plan = sc_amd.Plan(sc_amd.Cfmtx.build(A, km, kn), flags)
    Bt = torch.from_numpy(np.ascontiguousarray(B, np.float32)).to(DEV)
    if accumulate is not None:
        Ct = torch.from_numpy(accumulate.copy()).to(DEV)
        plan.spmm(Bt, Ct, accumulate=True)
    else:
        Ct = torch.full((A.shape[0], B.shape[1]), float("nan"), device=DEV)  # must be overwritten
        plan.spmm(Bt, Ct)
    torch.cuda.synchronize()
    return plan, Ct.cpu().numpy()


@pytest.mark.parametrize("n", [1, 2, 4, 32, 128])
@pytest.mark.parametrize("km", [2, 3, 4, 5, 6])
def test_rows_plan_512(km, n):
    A, B = synth_case(512, 512, 0.20, n, seed=0x5EED0000 + 1000 + km * 10 + n)
    plan, C = run(A, B, km, 2)
    err, _ = oracle_check(A, B, C)
    assert err <= REL_TOL, (km, n, err)
    assert plan.info()["km"] == 1
    assert f"(rows of km={km})" in plan.describe(n)


@pytest.mark.parametrize("kn", [1, 3, 8, 0])
@pytest.mark.parametrize("drop", [0, sc_amd.PLAN_DROP_PADDING])
def test_rows_plan_column_packs(kn, drop):
    A, B = synth_case(256, 320, 0.15, 4, seed=0x5EED0000 + 9100 + kn)
    plan, C = run(A, B, 4, kn, sc_amd.PLAN_ROWS | drop)
    err, _ = oracle_check(A, B, C)
    assert err <= REL_TOL, (kn, drop, err)
    if drop:
        # every padding slot is gone: one slot per stored entry
        assert plan.info()["nslots"] == A.nnz


def test_rows_plan_ragged_and_empty_rows():
    # 37 rows (the last panel of km 4, 5, 6 is partial), rows 5..12 and the
    # last row empty
    rng = np.random.default_rng(11)
    dense = (rng.random((37, 53)) < 0.3) * rng.standard_normal((37, 53))
    dense[5:13] = 0
    dense[-1] = 0
    ip = np.concatenate([[0], np.cumsum((dense != 0).sum(1))]).astype(np.int32)
    ix = np.nonzero(dense)[1].astype(np.int32)
    dx = dense[dense != 0].astype(np.float32).astype(np.float64)
    A = sc_amd.Csr.from_arrays(37, 53, ip, ix, dx)
    B = sc_amd.synth_dense(53 * 8, 78).reshape(53, 8)
    for km in (3, 4, 5, 6):
        _, C = run(A, B, km, 2)
        err, _ = oracle_check(A, B, C)
        assert err <= REL_TOL, (km, err)
        assert np.all(C[5:13] == 0) and np.all(C[-1] == 0)


def test_rows_plan_integer_inputs_are_exact():
    # small-integer A and B: every partial sum is exact in fp32
    rng = np.random.default_rng(12)
    dense = (rng.random((200, 300)) < 0.2) * rng.integers(-3, 4, (200, 300))
    ip = np.concatenate([[0], np.cumsum((dense != 0).sum(1))]).astype(np.int32)
    ix = np.nonzero(dense)[1].astype(np.int32)
    dx = dense[dense != 0].astype(np.float64)
    A = sc_amd.Csr.from_arrays(200, 300, ip, ix, dx)
    B = rng.integers(-4, 5, (300, 32)).astype(np.float32)
    _, C = run(A, B, 4, 2)
    assert np.array_equal(C, (dense @ B.astype(np.float64)).astype(np.float32))


def test_rows_plan_accumulate_and_spmv():
    A, B = synth_case(512, 512, 0.20, 4, seed=0x5EED0000 + 9200)
    C0 = sc_amd.synth_dense(512 * 4, 9201).reshape(512, 4)
    _, C = run(A, B, 4, 2, accumulate=C0)
    err = oracle_check_acc(A, B, C, C0)
    assert err <= REL_TOL, err
    plan = sc_amd.Plan(sc_amd.Cfmtx.build(A, 4, 2), sc_amd.PLAN_ROWS)
    y = plan.spmv(torch.from_numpy(np.ascontiguousarray(B[:, 0])).to(DEV))
    torch.cuda.synchronize()
    err, _ = oracle_check(A, B[:, :1], y.cpu().numpy().reshape(-1, 1))
    assert err <= REL_TOL, err


def test_rows_plan_of_km1_file_is_the_plain_plan():
    A, B = synth_case(128, 128, 0.2, 32, seed=0x5EED0000 + 9300)
    plan, C = run(A, B, 1, 1)
    err, _ = oracle_check(A, B, C)
    assert err <= REL_TOL, err
    assert "rows of" not in plan.describe(32)


@pytest.mark.parametrize("n", [1, 4, 128])
def test_default_plan_runs_rows_while_gathers_are_small(n):
    # 512 x 512 at 80 % sparsity: 4 * 52429 * n bytes of B-row gathers in the
    # one-row layout, far under 128 MiB -> one-row layout, still exact
    A, B = synth_case(512, 512, 0.20, n, seed=0x5EED0000 + 9400 + n)
    plan = sc_amd.Plan(sc_amd.Cfmtx.build(A, 4, 2))
    assert plan.describe(n).endswith("(rows of km=4)")
    assert plan.info()["km"] == 4  # the plan still reports the file's layout
    Ct = plan.spmm(torch.from_numpy(B).to(DEV))
    torch.cuda.synchronize()
    err, _ = oracle_check(A, B, Ct.cpu().numpy())
    assert err <= REL_TOL, err


def test_default_plan_keeps_patterns_for_large_gathers():
    # 4096 x 4096 structured at 90 % sparsity, N = 128: 4 * 1.68 M * 128 bytes
    # of one-row gathers (859 MB) -> the km = 4 pattern layout; N = 1 -> rows
    A = sc_amd.Csr.synth_blocks(4096, 4096, 0.10, 0.05, 0x5EED0000 + 4128)
    plan = sc_amd.Plan(sc_amd.Cfmtx.build(A, 4, 1))
    assert plan.describe(128).startswith("panel_kernel km=4")
    assert plan.describe(1).endswith("(rows of km=4)")
    for flags in (sc_amd.PLAN_PATTERNS, sc_amd.PLAN_TILED):
        assert "rows of" not in sc_amd.Plan(sc_amd.Cfmtx.build(A, 4, 1), flags).describe(1)


def test_rows_and_patterns_flags_are_exclusive():
    A, _ = synth_case(64, 64, 0.2, 1, seed=0x5EED0000 + 9500)
    with pytest.raises(sc_amd.LibscError, match="exclusive"):
        sc_amd.Plan(sc_amd.Cfmtx.build(A, 4, 1), sc_amd.PLAN_ROWS | sc_amd.PLAN_PATTERNS)


@pytest.mark.parametrize("n", [3, 5, 33, 256, 300])
def test_rows_plan_odd_and_wide_n(n):
    A, B = synth_case(96, 160, 0.15, n, seed=0x5EED0000 + 9600 + n)
    _, C = run(A, B, 4, 1)
    err, _ = oracle_check(A, B, C)
    assert err <= REL_TOL, (n, err)


@pytest.mark.parametrize("n", [1, 4, 32, 128])
@pytest.mark.parametrize("shape", [(64, 8192, 0.25), (8, 65536, 0.2)])
def test_rows_plan_long_rows(shape, n):
    # ~2000 entries a row (staged in LDS as a long panel) and ~13000 a row
    # (over the 64 KiB staging limit: the unstaged path)
    m, k, d = shape
    A, B = synth_case(m, k, d, n, seed=0x5EED0000 + 9700 + m + n)
    _, C = run(A, B, 4, 2)
    err, _ = oracle_check(A, B, C)
    assert err <= REL_TOL, (shape, n, err)


@pytest.mark.parametrize("waves", [1, 2, 5, 16])
def test_rows_plan_waves_per_row(waves):
    A, B = synth_case(128, 2048, 0.3, 64, seed=0x5EED0000 + 9800 + waves)
    plan = sc_amd.Plan(sc_amd.Cfmtx.build(A, 4, 1), sc_amd.PLAN_ROWS)
    Ct = plan.spmm(torch.from_numpy(B).to(DEV), waves=waves)
    torch.cuda.synchronize()
    err, _ = oracle_check(A, B, Ct.cpu().numpy())
    assert err <= REL_TOL, (waves, err)


def test_default_plan_of_empty_matrix_overwrites_c():
    A = sc_amd.Csr.from_arrays(10, 12, np.zeros(11, np.int32), [], [])
    B = sc_amd.synth_dense(12 * 4, 3).reshape(12, 4)
    for flags in (0, sc_amd.PLAN_ROWS):
        _, C = run(A, B, 4, 1, flags)
        assert np.all(C == 0)


def test_rows_layout_of_dictionary_file_keeps_the_stored_subset():
    # A dictionary-mode file (format_generator.py --pattern_dictionary) stores
    # only the slots whose pattern is in the dictionary; every layout must
    # compute the product of exactly the entries the file stores.
    import os
    here = os.path.dirname(os.path.abspath(__file__))
    dic = os.path.join(here, "golden", "cfmtx", "dict4_sub.txt")
    m = k = 256
    A, B = synth_case(m, k, 0.2, 32, seed=0x5EED0000 + 9900)
    cf = sc_amd.Cfmtx.build(A, 4, 1, dictionary=dic)
    # the stored entries, decoded from the file's pattern blocks (the oracle's
    # decoding rule: slot j of panel q holds row q*4 + r of each '1' at r)
    kept = np.zeros((m, k))
    for p in cf.patterns():
        rows = [r for r, ch in enumerate(p["bits"]) if ch == "1"]
        for q in range(len(p["rpp"]) - 1):
            for j in range(p["rpp"][q], p["rpp"][q + 1]):
                for t, r in enumerate(rows):
                    if q * 4 + r < m:
                        kept[q * 4 + r, p["cb"][j]] += p["vals"][j * len(rows) + t]
    assert 0 < np.count_nonzero(kept) < A.nnz  # the dictionary dropped entries
    ref = kept @ B.astype(np.float64)
    bound = np.abs(kept) @ np.abs(B.astype(np.float64))
    Bt = torch.from_numpy(B).to(DEV)
    for flags in (0, sc_amd.PLAN_ROWS, sc_amd.PLAN_PATTERNS):
        C = sc_amd.Plan(cf, flags).spmm(Bt)
        torch.cuda.synchronize()
        err = np.max(np.abs(C.cpu().numpy() - ref) / np.maximum(bound, 1e-30))
        assert err <= REL_TOL, (flags, err)


@pytest.mark.parametrize("n", [1, 2, 4])
@pytest.mark.parametrize("kn,drop", [(1, 0), (3, 0), (3, sc_amd.PLAN_DROP_PADDING)])
@pytest.mark.parametrize("accumulate", [False, True])
def test_row_spmv_kernel_tails_empty_rows_padding(kn, drop, accumulate, n):
    # N = 1, 2, 4 on one-row panels runs row_spmv_kernel: rows of every length
    # mod 4 (0..9 entries and longer), empty rows, kn padding kept or dropped
    rng = np.random.default_rng(13 + kn)
    m, k = 203, 300
    lens = np.concatenate([np.arange(10), rng.integers(0, 120, m - 10)])
    dense = np.zeros((m, k))
    for i, ln in enumerate(lens):
        dense[i, rng.choice(k, size=int(ln), replace=False)] = rng.standard_normal(int(ln))
    ip = np.concatenate([[0], np.cumsum((dense != 0).sum(1))]).astype(np.int32)
    ix = np.nonzero(dense)[1].astype(np.int32)
    dx = dense[dense != 0].astype(np.float32).astype(np.float64)
    A = sc_amd.Csr.from_arrays(m, k, ip, ix, dx)
    B = sc_amd.synth_dense(k * n, 99).reshape(k, n)
    for km in (1, 4):
        plan = sc_amd.Plan(sc_amd.Cfmtx.build(A, km, kn), sc_amd.PLAN_ROWS | drop)
        assert plan.describe(n).startswith(f"row_spmv_kernel km=1 V={n}")
        C0 = sc_amd.synth_dense(m * n, 100).reshape(m, n)
        Ct = torch.from_numpy(C0.copy() if accumulate else np.full((m, n), np.nan, np.float32)).to(DEV)
        plan.spmm(torch.from_numpy(B).to(DEV), Ct, accumulate=accumulate)
        torch.cuda.synchronize()
        C = Ct.cpu().numpy()
        err = oracle_check_acc(A, B, C, C0) if accumulate else oracle_check(A, B, C)[0]
        assert err <= REL_TOL, (km, kn, drop, n, err)
        if not accumulate:
            assert np.all(C[lens == 0] == 0)
        else:
            assert np.array_equal(C[lens == 0], C0[lens == 0])


@pytest.mark.parametrize("n", [1, 2, 4])
def test_row_kernel_b_in_lds(n):
    # 4100 rows (a partial workgroup of 16 rows at the end, empty rows) over
    # K = 2048 at 5 % density: about 100 entries per B row, so the row kernel
    # copies B into LDS first; plain and accumulating
    rng = np.random.default_rng(21 + n)
    A, B = synth_case(4100, 2048, 0.05, n, seed=0x5EED0000 + 9700 + n)
    ip, ix, dx = A.arrays()
    keep = np.ones(A.nnz, bool)
    for r in (0, 17, 4099):
        keep[ip[r]:ip[r + 1]] = False  # rows 0, 17 and the last one empty
    rows = np.repeat(np.arange(4100), np.diff(ip))
    dense_rows, dense_cols, dense_vals = rows[keep], ix[keep], dx[keep]
    order = np.lexsort((dense_cols, dense_rows))
    ptr = np.zeros(4101, np.int32)
    np.add.at(ptr, dense_rows[order] + 1, 1)
    A = sc_amd.Csr.from_arrays(4100, 2048, np.cumsum(ptr).astype(np.int32), dense_cols[order], dense_vals[order])
    plan, C = run(A, B, 4, 1, 0)
    assert "B_in_lds=1" in plan.describe(n), plan.describe(n)
    err, _ = oracle_check(A, B, C)
    assert err <= REL_TOL, (n, err)
    assert np.all(C[[0, 17, 4099]] == 0)
    C0 = rng.uniform(-1, 1, size=(4100, n)).astype(np.float32)
    _, Ca = run(A, B, 4, 1, 0, accumulate=C0)
    assert oracle_check_acc(A, B, Ca, C0) <= REL_TOL


def test_row_kernel_b_in_lds_spmv_exact():
    # integer-valued A and x: the staged gathers give the exact sums
    rng = np.random.default_rng(23)
    m, k = 4096, 1024
    mask = rng.random((m, k)) < 0.08
    dense = np.where(mask, rng.integers(-3, 4, size=(m, k)), 0).astype(np.float64)
    r, c = np.nonzero(dense)
    ptr = np.zeros(m + 1, np.int32)
    np.add.at(ptr, r + 1, 1)
    A = sc_amd.Csr.from_arrays(m, k, np.cumsum(ptr).astype(np.int32), c.astype(np.int32), dense[r, c])
    x = rng.integers(-4, 5, size=k).astype(np.float32)
    plan = sc_amd.Plan(sc_amd.Cfmtx.build(A, 1, 1), 0)
    assert "B_in_lds=1" in plan.describe(1), plan.describe(1)
    y = plan.spmv(torch.from_numpy(x).to(DEV))
    torch.cuda.synchronize()
    assert np.array_equal(y.cpu().numpy(), (dense @ x.astype(np.float64)).astype(np.float32))
