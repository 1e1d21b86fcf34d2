"""sc_spmm_noalloc: the split-K kernels (band and tiled) with their partial
sums and counters in the library's static per-device scratch.  Each call is
checked against sc_spmm on the same plan (the K split is sized to fit both
workspaces, so the results must match bit for bit) and against the fp64
oracle (max relative error <= 1e-5 normalised by (|A| |B|)_ij): two calls in
a row, the second with a smaller input, and captured in a HIP graph."""
import numpy as np
import pytest

import sc_amd
from cases import REL_TOL, oracle_check, oracle_check_acc, synth_case

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def both(plan, B, C0=None):
    """(sc_spmm result, sc_spmm_noalloc result) on fresh outputs."""
    Bt = torch.from_numpy(np.ascontiguousarray(B, np.float32)).to(DEV)
    m = plan.info()["m"]
    out = []
    for noalloc in (False, True):
        if C0 is None:
            Ct = torch.full((m, B.shape[1]), float("nan"), device=DEV)
        else:
            Ct = torch.from_numpy(C0.copy()).to(DEV)
        if noalloc:
            plan.spmm_noalloc(Bt, Ct, accumulate=C0 is not None)
        else:
            plan.spmm(Bt, Ct, accumulate=C0 is not None)
        torch.cuda.synchronize()
        out.append(Ct.cpu().numpy())
    return out


@pytest.mark.parametrize("flags", [sc_amd.PLAN_BANDS, sc_amd.PLAN_TILED])
def test_noalloc_matches_spmm_two_calls(flags):
    # first call: the 4096^2 headline matrix, K split over several ranges
    A, B = synth_case(4096, 4096, 0.10, 128, seed=0x5EED0000 + 4128, structured=True)
    plan = sc_amd.Plan(sc_amd.Cfmtx.build(A, 4, 1), flags)
    kernel = plan.describe(128)
    assert kernel.startswith("band_kernel" if flags == sc_amd.PLAN_BANDS else "tiled_kernel"), kernel
    C1, C2 = both(plan, B)
    assert np.array_equal(C1, C2), kernel
    assert oracle_check(A, B, C2)[0] <= REL_TOL
    # second call, smaller: another plan, fewer rows and columns, accumulate
    A2, B2 = synth_case(520, 700, 0.12, 64, seed=0x5EED0000 + 7300)
    plan2 = sc_amd.Plan(sc_amd.Cfmtx.build(A2, 4, 1), flags)
    C0 = sc_amd.synth_dense(520 * 64, 7301).reshape(520, 64)
    D1, D2 = both(plan2, B2, C0)
    assert np.array_equal(D1, D2), plan2.describe(64)
    assert oracle_check_acc(A2, B2, D2, C0) <= REL_TOL


def test_noalloc_without_split_k_is_sc_spmm():
    # plans with no split-K kernel take the same launch as sc_spmm
    for flags, n in ((0, 128), (sc_amd.PLAN_PATTERNS, 4), (sc_amd.PLAN_BANDS, 32)):
        A, B = synth_case(512, 512, 0.10, n, seed=0x5EED0000 + 7400 + n)
        plan = sc_amd.Plan(sc_amd.Cfmtx.build(A, 4, 1), flags)
        C1, C2 = both(plan, B)
        assert np.array_equal(C1, C2), (flags, n)


def test_noalloc_in_a_graph():
    # captured with its counter clear; every replay equals the eager result
    A, B = synth_case(4096, 4096, 0.10, 128, seed=0x5EED0000 + 4128, structured=True)
    plan = sc_amd.Plan(sc_amd.Cfmtx.build(A, 4, 1), sc_amd.PLAN_BANDS)
    Bt = torch.from_numpy(B).to(DEV)
    ref = torch.empty(4096, 128, device=DEV)
    plan.spmm(Bt, ref)
    Ct = torch.full((4096, 128), float("nan"), device=DEV)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        plan.spmm_noalloc(Bt, Ct, stream=s)  # warm outside the capture
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        plan.spmm_noalloc(Bt, Ct)
    for i in range(3):
        Ct.fill_(float("nan"))
        plan.spmm(Bt, ref)  # eager work between the replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(Ct, ref), i
