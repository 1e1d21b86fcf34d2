"""GPU: the demo drivers (lib/demos, built by the libsc Makefile from
demos/demo_gpu.hip and generated units) load a .cfmtx + companion .mtx, run
the trials and print the reference's CSV layout with Correct = 1 on every
trial (max error normalised by |A||B| <= 1e-5 against the fp64 product)."""
import os
import subprocess

import pytest

import sc_amd

pytestmark = pytest.mark.gpu
DEMOS = os.path.join(os.path.dirname(sc_amd.LIB_PATH), "demos")


def make_matrix(tmp_path, m, n, density, seed):
    A = sc_amd.Csr.synth_uniform(m, n, density, 0.05, seed)
    mtx = str(tmp_path / "mat.mtx")
    A.write_mtx(mtx)
    cf = str(tmp_path / "mat-4-1.cfmtx")
    sc_amd.Cfmtx.build(sc_amd.Csr.from_mtx(mtx), 4, 1).write(cf)
    return cf


# fp16 inputs cannot meet the fp32 tolerance; its rows report Correct = 0
APPROXIMATE = {"SpMM hipBlas Half Tensor"}


def run_demo(binary, args, trials):
    out = subprocess.run([os.path.join(DEMOS, binary)] + args, capture_output=True, text=True,
                         timeout=120)
    assert out.returncode == 0, out.stderr
    lines = [l for l in out.stdout.splitlines() if l.strip()]
    header = lines[0].split(",")
    assert header[:6] == ["Operation Name", "Implementation Name", "Number of Trials",
                          "Matrix Name", "Number of Threads", "Number of Subregions"]
    assert header[-5:] == ["kernel_n", "kernel_m", "b_cols", "b_unroll_factor", "number_of_warps"]
    rows = [l.split(",") for l in lines[1:]]
    for r in rows:
        assert len(r) == len(header)
        assert r[2] == str(trials)
        for t in range(trials):
            want = "0" if r[0] in APPROXIMATE else "1"
            assert r[header.index(f"Correct{t}")] == want, (r[0], t, r[header.index(f"Error{t}")])
    return header, rows


@pytest.mark.parametrize("n", [32, 128])
def test_spmm_demo_gpu(tmp_path, n):
    cf = make_matrix(tmp_path, 300, 257, 0.1, 61)
    header, rows = run_demo("spmm_demo_gpu", ["-m", cf, "--header", "--baseline=true", "-n", "SPMM",
                                              "-s", "CSR", "-t", str(n), f"--b_matrix_columns={n}",
                                              "--number_of_warps=2", "--b_unroll_factor=1"], 7)
    # the reference's baseline order (cuBLAS, Half, GemmX, cuSPARSE) on hipBLAS / rocSPARSE
    assert [r[0] for r in rows] == ["SpMM hipBlas", "SpMM hipBlas Half Tensor", "SpMM hipBlas GemmX",
                                    "SpMM rocSparse", "SpMM Serial Float",
                                    "SpMM Format Pack Block Cache less"]
    assert rows[-1][-5:] == ["1", "4", str(n), "1", "2"]


def test_small_b_demo_gpu(tmp_path):
    cf = make_matrix(tmp_path, 200, 150, 0.2, 62)
    _, rows = run_demo("spmm_small_b_col_demo_gpu", ["-m", cf, "--header", "-n", "SPMM", "-s", "CSR",
                                           "-t", "4", "--b_matrix_columns=4", "--number_of_warps=1"], 7)
    assert [r[0] for r in rows] == ["SpMM Format Pack Block Cache less"]


def test_spmv_demo_gpu(tmp_path):
    cf = make_matrix(tmp_path, 250, 250, 0.3, 63)
    _, rows = run_demo("spmv_demo_gpu", ["-m", cf, "--header", "-n", "SPMV", "-s", "CSR"], 20)
    assert [r[0] for r in rows] == ["SpMV Compressed Format"]
    _, rows = run_demo("spmv_demo_gpu", ["-m", cf, "--header", "--baseline=true", "-n", "SPMV", "-s",
                                         "CSR"], 20)
    assert [r[0] for r in rows] == ["SpMV rocSparse GPU", "SpMV hipBlas GPU", "SpMV Serial Float",
                                    "SpMV Compressed Format"]


def test_demo_rejects_mismatched_unit(tmp_path):
    # the small-B demo was generated for b_col = 4: any other N is refused
    cf = make_matrix(tmp_path, 64, 64, 0.2, 64)
    out = subprocess.run([os.path.join(DEMOS, "spmm_small_b_col_demo_gpu"), "-m", cf, "-n", "SPMM",
                          "-s", "CSR", "--b_matrix_columns=2"], capture_output=True, text=True,
                         timeout=120)
    assert out.returncode != 0 and "N=4" in out.stderr
