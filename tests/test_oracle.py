"""Pins the CPU oracle before it is trusted as the checker.

* pattern enumeration: closed form id = 2^bits - 1 - int(bits, 2) and the
  pattern lines of the reference's 47 .cfmtx fixtures;
* builder + writer: byte-exact against the 47 reference fixtures
  (matrices/*-<km>-<kn>.cfmtx, plus the unsuffixed -6-8 copy) and against the
  golden vectors produced by the reference CLI (tests/golden);
* reader: against the reference's own loader compiled from its sources
  (oracle/_ref) on fixtures and golden files;
* CPU SpMM/SpMV: bit-exact on integer-valued inputs, and within the dot
  product error bound of numpy's float64 product on random inputs; a planted
  mistake (a dropped term) must fail the same check.
"""
import glob
import json
import os

import numpy as np
import pytest

import oracle as O
from conftest import FIXTURE_STEM, REF_MATRICES

HERE = os.path.dirname(os.path.abspath(__file__))
GOLDEN = os.path.join(HERE, "golden")
FIX_MTX = os.path.join(REF_MATRICES, FIXTURE_STEM + ".mtx")
needs_ref = pytest.mark.skipif(not os.path.exists(FIX_MTX), reason="reference tree not mounted")


def fixture_files():
    files = sorted(glob.glob(os.path.join(REF_MATRICES, FIXTURE_STEM + "-*.cfmtx")))
    out = []
    for f in files:
        km, kn = map(int, os.path.basename(f)[:-6].split("-")[-2:])
        out.append((f, km, kn))
    out.append((os.path.join(REF_MATRICES, FIXTURE_STEM + ".cfmtx"), 6, 8))
    return out


def golden_cases():
    with open(os.path.join(GOLDEN, "manifest.json")) as f:
        return [c for c in json.load(f) if "cfmtx" in c]


@pytest.mark.parametrize("km", range(1, 7))
def test_pattern_ids_closed_form(km):
    pm = O.patterns_map(km, 1)
    assert len(pm) == 2 ** km - 1
    for key, pid in pm.items():
        bits = "".join("1" if b else "0" for b in key)
        assert pid == 2 ** km - 1 - int(bits, 2)
    # id 0 is all ones, the last id has only the last panel row
    inv = {v: k for k, v in pm.items()}
    assert all(inv[0]) and inv[2 ** km - 2] == tuple([False] * (km - 1) + [True])


def test_pattern_ids_with_kernel_n():
    pm = O.patterns_map(2, 2)
    assert len(pm) == 15 and pm[(True,) * 4] == 0 and pm[(False, False, False, True)] == 14


@needs_ref
def test_fixture_pattern_lines_match_enumeration():
    for f, km, kn in fixture_files():
        with open(f) as fh:
            hdr = fh.readline().split()
            P = int(hdr[3])
            lines = [fh.readline() for _ in range(P)]
        pm = O.patterns_map(km, 1)
        assert P == len(pm)
        for line, (key, pid) in zip(lines, pm.items()):
            assert line == "".join("1" if b else "0" for b in key) + f" {pid} \n"


@needs_ref
def test_oracle_reproduces_every_reference_fixture():
    M, K, ip, ix, data, is_int = O.mtx_to_csr(FIX_MTX)
    assert (M, K, len(ix)) == (512, 512, 104857)
    for f, km, kn in fixture_files():
        pats = O.patterns_map(km, 1)
        cf = O.build(M, K, ip, ix, data.astype(np.float64), km, kn, pats)
        with open(f) as fh:
            assert O.cfmtx_text(cf, pats, is_int) == fh.read(), f


@pytest.mark.parametrize("case", golden_cases(), ids=lambda c: c["tag"])
def test_oracle_reproduces_reference_cli_golden(case):
    d = None
    if case["dictionary"]:
        d = os.path.join(GOLDEN, "cfmtx", case["dictionary"] + ".txt")
    text = O.format_generator(os.path.join(GOLDEN, "cfmtx", case["mtx"]), case["km"], case["kn"],
                              d or "false")
    with open(os.path.join(GOLDEN, "cfmtx", case["cfmtx"])) as f:
        assert text == f.read()


def test_planted_builder_mistake_is_caught():
    """Swapping the ascending-row order of a slot's values (a plausible slip)
    must change the output the fixtures are compared with."""
    case = golden_cases()[0]
    mtx = os.path.join(GOLDEN, "cfmtx", case["mtx"])
    M, K, ip, ix, data, is_int = O.mtx_to_csr(mtx)
    pats = O.patterns_map(case["km"], 1)
    cf = O.build(M, K, ip, ix, data, case["km"], case["kn"], pats)
    good = O.cfmtx_text(cf, pats, is_int)
    pid = next(i for i, (k, _) in enumerate(pats.items()) if sum(k) >= 2 and len(cf["cb"][i]))
    pop = sum(list(pats.keys())[pid])
    v = cf["vals"][pid].copy()
    v[0:pop] = v[0:pop][::-1]
    cf["vals"][pid] = v
    assert O.cfmtx_text(cf, pats, is_int) != good


@needs_ref
def test_oracle_reader_matches_reference_loader():
    if not O.ref_dump_available():
        pytest.skip("oracle/_ref not built")
    files = [f for f, _, _ in fixture_files()[::6]]
    files += [os.path.join(GOLDEN, "cfmtx", c["cfmtx"]) for c in golden_cases()]
    for f in files:
        mine = O.read_cfmtx(f)
        ref = O.ref_read_cfmtx(f)
        assert len(ref) == mine["num_patterns"]
        for i, r in enumerate(ref):
            assert r["km"] == mine["kernel_rows"] and r["kn"] == mine["vector_length"]
            assert r["nrpp"] == mine["nrpp"]
            assert np.array_equal(r["rpp"], mine["rpp"][i])
            assert np.array_equal(r["npp"], mine["npp"][i])
            assert np.array_equal(r["cb"], mine["cb"][i])
            assert np.array_equal(r["vals"].view(np.uint32), mine["nnz"][i].view(np.uint32)), f


def test_cpu_spmm_exact_on_integers():
    rng = np.random.default_rng(1)
    dense = (rng.random((40, 30)) < 0.3) * rng.integers(-4, 5, (40, 30))
    ip = np.concatenate([[0], np.cumsum((dense != 0).sum(1))]).astype(np.int32)
    ix = np.nonzero(dense)[1].astype(np.int32)
    ax = dense[dense != 0].astype(np.float32)
    B = rng.integers(-3, 4, (30, 7)).astype(np.float32)
    C = O.spmm_csr_float(40, 7, ip, ix, ax, B)
    assert np.array_equal(C, (dense @ B).astype(np.float32))
    y = O.spmv_csr_float(40, ip, ix, ax, B[:, 0])
    assert np.array_equal(y, (dense @ B[:, 0]).astype(np.float32))
    c64, cab = O.spmm_f64(40, 7, ip, ix, ax, B)
    assert np.array_equal(c64, dense @ B.astype(np.float64))


def test_cpu_spmm_within_bound_and_detects_dropped_term():
    rng = np.random.default_rng(2)
    dense = (rng.random((64, 80)) < 0.2) * rng.standard_normal((64, 80))
    dense = dense.astype(np.float32)
    ip = np.concatenate([[0], np.cumsum((dense != 0).sum(1))]).astype(np.int32)
    ix = np.nonzero(dense)[1].astype(np.int32)
    ax = dense[dense != 0]
    B = rng.uniform(-1, 1, (80, 16)).astype(np.float32)
    ref = dense.astype(np.float64) @ B.astype(np.float64)
    c64, cab = O.spmm_f64(64, 16, ip, ix, ax, B)
    assert np.allclose(c64, ref, rtol=1e-13, atol=1e-13)
    C = O.spmm_csr_float(64, 16, ip, ix, ax, B)
    assert O.max_rel_err(C, c64, cab) <= 1e-5
    ax_bad = ax.copy()
    ax_bad[5] = 0.0  # a dropped term
    Cbad = O.spmm_csr_float(64, 16, ip, ix, ax_bad, B)
    assert O.max_rel_err(Cbad, c64, cab) > 1e-5
