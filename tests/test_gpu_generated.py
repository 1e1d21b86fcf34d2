"""GPU: kernel units emitted through the reference-compatible generator CLIs
(built by the libsc Makefile into lib/units) run through sc_spmm_generated,
which checks each unit against the plan before launching."""
import os

import numpy as np
import pytest

import sc_amd
from cases import REL_TOL, oracle_check, synth_case

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

DEV = "cuda:0"
UNITS = os.path.join(os.path.dirname(sc_amd.LIB_PATH), "units")
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "cfmtx")


def unit(name, so_name=None):
    """Unit `name` (its sc_gen_<name>_* symbols) from lib/units/libsc_unit_<so_name>.so."""
    return sc_amd.GeneratedUnit(os.path.join(UNITS, f"libsc_unit_{so_name or name}.so"), name)


def run(cf, u, B, flags=0):
    plan = sc_amd.Plan(cf, flags)
    Bt = torch.from_numpy(np.ascontiguousarray(B, np.float32)).to(DEV)
    C = plan.spmm_generated(u, Bt)
    torch.cuda.synchronize()
    return C.cpu().numpy()


@pytest.mark.parametrize("n", [1, 4, 32, 128])
def test_generated_unit_follows_the_layout_rule(n):
    # a default plan holds both layouts: sc_spmm_generated runs the unit's
    # one-row body where sc_spmm would run the one-row layout (all of these
    # sizes), the km-row bodies on a SC_PLAN_PATTERNS plan; both agree with
    # the oracle
    A, B = synth_case(512, 512, 0.10, n, seed=0x5EED0000 + 2000 + n)
    cf = sc_amd.Cfmtx.build(A, 4, 2)
    assert "(rows of km=4)" in sc_amd.Plan(cf).describe(n)
    u = unit("spmm_km4_kn2")
    for flags in (0, sc_amd.PLAN_PATTERNS):
        C = run(cf, u, B, flags)
        assert oracle_check(A, B, C)[0] <= REL_TOL, (n, flags)


# every unit on both layouts: its one-row body (default plans at these
# sizes) and its km-row bodies (SC_PLAN_PATTERNS)
LAYOUTS = [0, sc_amd.PLAN_PATTERNS]


@pytest.mark.parametrize("flags", LAYOUTS)
@pytest.mark.parametrize("n", [1, 32, 128])
def test_generated_spmm_km4_kn2(n, flags):
    A, B = synth_case(300, 256, 0.15, n, seed=41 + n)
    for kn in (2, 4, 8):  # packs of 2 divide all of these
        C = run(sc_amd.Cfmtx.build(A, 4, kn), unit("spmm_km4_kn2"), B, flags)
        assert oracle_check(A, B, C)[0] <= REL_TOL


@pytest.mark.parametrize("flags", LAYOUTS)
@pytest.mark.parametrize("n", [1, 7, 64])
def test_generated_spmm_km3_kn1(n, flags):
    A, B = synth_case(301, 190, 0.2, n, seed=47 + n)
    C = run(sc_amd.Cfmtx.build(A, 3, 1), unit("spmm_km3_kn1"), B, flags)
    assert oracle_check(A, B, C)[0] <= REL_TOL


@pytest.mark.parametrize("flags", LAYOUTS)
def test_generated_small_b_and_spmv(flags):
    A, B = synth_case(256, 200, 0.2, 2, seed=43)
    C = run(sc_amd.Cfmtx.build(A, 4, 1), unit("spmm_small_km4_b2"), B, flags)
    assert oracle_check(A, B, C)[0] <= REL_TOL
    A, B = synth_case(256, 200, 0.2, 1, seed=44)
    C = run(sc_amd.Cfmtx.build(A, 4, 3), unit("spmv_km4"), B, flags)
    assert oracle_check(A, B, C)[0] <= REL_TOL


@pytest.mark.parametrize("flags", LAYOUTS)
def test_generated_dictionary_unit(flags):
    A, B = synth_case(96, 128, 0.3, 64, seed=45)
    cf = sc_amd.Cfmtx.build(A, 4, 1, os.path.join(GOLDEN, "dict4_sub.txt"))
    C = run(cf, unit("spmm_km4_kn1", "spmm_km4_kn1_dict"), B, flags)
    # the format drops slots whose pattern is not in the dictionary: compare
    # with the product of what the format kept
    kept = sc_amd.Csr.from_arrays(96, 128, *_kept_csr(cf))
    assert oracle_check(kept, B, C)[0] <= REL_TOL


def _kept_csr(cf):
    info = cf.info()
    ent = {}
    for p in cf.patterns():
        rows = [r for r, ch in enumerate(p["bits"]) if ch == "1"]
        for q in range(info["npanels"]):
            for j in range(p["rpp"][q], p["rpp"][q + 1]):
                for k, r in enumerate(rows):
                    v = float(p["vals"][j * len(rows) + k])
                    if v != 0:
                        ent[(q * info["km"] + r, int(p["cb"][j]))] = v
    keys = sorted(ent)
    ip = np.zeros(info["m"] + 1, np.int32)
    for r, _ in keys:
        ip[r + 1] += 1
    return np.cumsum(ip).astype(np.int32), np.array([c for _, c in keys], np.int32), \
        np.array([ent[k] for k in keys])


def test_generated_unit_mismatches_are_rejected():
    A, B = synth_case(64, 64, 0.3, 2, seed=46)
    Bt = torch.from_numpy(B).to(DEV)
    E = sc_amd.LibscError
    with pytest.raises(E, match="km=3"):
        sc_amd.Plan(sc_amd.Cfmtx.build(A, 4, 1)).spmm_generated(unit("spmm_km3_kn1"), Bt)
    with pytest.raises(E, match="do not divide"):
        sc_amd.Plan(sc_amd.Cfmtx.build(A, 4, 3)).spmm_generated(unit("spmm_km4_kn2"), Bt)
    with pytest.raises(E, match="N=2"):
        B4 = torch.zeros((64, 4), device=DEV)
        sc_amd.Plan(sc_amd.Cfmtx.build(A, 4, 1)).spmm_generated(unit("spmm_small_km4_b2"), B4)
    with pytest.raises(E, match="no body"):
        sc_amd.Plan(sc_amd.Cfmtx.build(A, 4, 1)).spmm_generated(unit("spmm_km4_kn1", "spmm_km4_kn1_dict"), Bt)
