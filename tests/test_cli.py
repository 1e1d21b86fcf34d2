"""The reference-compatible command lines (format_generator.py and the
main_spmm / main_spmm_small_b_col / main_spmv generators) keep the
reference's argv and outputs.  CPU only: generated HIP is checked as text
here and compiled by the build; its numerics are covered by the GPU tests."""
import json
import os
import re
import shutil
import subprocess
import sys

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CG = os.path.join(ROOT, "sparse-computation_amd", "code_gen")
GOLDEN = os.path.join(HERE, "golden", "cfmtx")


def run(*args, cwd=None):
    return subprocess.run([sys.executable, *args], cwd=cwd, capture_output=True, text=True,
                          check=True)


def test_format_generator_cli_writes_reference_files(tmp_path):
    with open(os.path.join(HERE, "golden", "manifest.json")) as f:
        cases = [c for c in json.load(f) if "cfmtx" in c][:8]
    for c in cases:
        mtx = tmp_path / c["mtx"]
        shutil.copy(os.path.join(GOLDEN, c["mtx"]), mtx)
        args = [os.path.join(CG, "ss_format", "format_generator.py"), str(mtx), str(c["km"]),
                str(c["kn"])]
        if c["dictionary"]:
            args += ["--pattern_dictionary", os.path.join(GOLDEN, c["dictionary"] + ".txt")]
        run(*args)
        out = str(mtx)[:-4] + f"-{c['km']}-{c['kn']}.cfmtx"
        with open(out) as a, open(os.path.join(GOLDEN, c["cfmtx"])) as b:
            assert a.read() == b.read()


def test_format_generator_save_collection_and_non_mtx(tmp_path):
    mtx = tmp_path / "m.mtx"
    shutil.copy(os.path.join(GOLDEN, "real_17x23.mtx"), mtx)
    run(os.path.join(CG, "ss_format", "format_generator.py"), str(mtx), "4", "1",
        "--save_collection", "true")
    a = (tmp_path / "m-4-1.cfmtx").read_text()
    assert a == (tmp_path / "m.cfmtx").read_text()
    assert a == open(os.path.join(GOLDEN, "real_17x23-4-1.cfmtx")).read()
    run(os.path.join(CG, "ss_format", "format_generator.py"), str(tmp_path / "m-4-1.cfmtx"),
        "4", "1")  # not a .mtx: nothing happens
    assert sorted(os.listdir(tmp_path)) == ["m-4-1.cfmtx", "m.cfmtx", "m.mtx"]


def test_python_reader_of_cfmtx():
    sys.path.insert(0, os.path.join(CG, "ss_format"))
    from read_compressed_format import read_compressed_matrix
    m = read_compressed_matrix(os.path.join(GOLDEN, "real_17x23-4-1.cfmtx"))
    assert (m.num_row, m.num_col, m.kernel_rows, m.kernel_cols) == (17, 23, 4, 1)
    assert m.patterns[0] == "1111" and len(m.row_panels_pointer[0]) == 6
    assert len(m.padded_values_data_array[7]) == len(m.indices_array[7])  # pop 1


def _cases(text):
    """Cases of the unit's main dispatch; the one-row layout's own dispatch
    (namespace rows, a single all-ones row pattern) is left out."""
    if "namespace rows {" in text:
        head, rest = text.split("namespace rows {", 1)
        text = head + rest.split("}  // namespace rows", 1)[1]
    return re.findall(r"case (\d+): pattern_(\d+)<V, A>", text)


def _row_cases(text):
    rows = text.split("namespace rows {", 1)[1].split("}  // namespace rows", 1)[0]
    return re.findall(r"case (\d+): pattern_(\d+)<V, A>", rows)


@pytest.mark.parametrize("km,kn", [(4, 1), (4, 2), (6, 3), (1, 1)])
def test_main_spmm_emits_one_body_per_pattern(tmp_path, km, kn):
    out = tmp_path / "k.hip"
    run(os.path.join(CG, "main_spmm.py"), str(out), "format", str(km), str(kn), "1", "2", "i-j")
    text = out.read_text()
    cases = _cases(text)
    assert len(cases) == 2 ** km - 1
    for mask, bits in cases:
        assert int(mask) == sum(1 << r for r, ch in enumerate(bits) if ch == "1")
        assert f"__device__ __forceinline__ void pattern_{bits}(float (&acc)[{km}][V]" in text
        assert f"void wide_{bits}(" in text
    assert f"sc_gen_spmm_km{km}_kn{kn}_record = {{{km}, {kn}, 0, {2 ** km - 1}, 0," in text
    assert f"sc_gen_spmm_km{km}_kn{kn}_launch" in text
    # one-row layout launcher, installed in the record at load
    assert _row_cases(text) == [("1", "1")]
    assert f".rows_launch = (sc_gen_launch_fn)sc_gen_spmm_km{km}_kn{kn}_launch_rows;" in text
    # a pack of kn slots is unrolled, U = max(1, 4 // kn) packs per batch: a
    # full batch of U * kn B-row loads, then a last batch of exactly the t
    # packs left (t = 1 .. U; t * kn loads that may read zeros)
    U = max(1, 4 // kn)
    body = text.split(f"void pattern_{'1' * km}(")[1].split("\n}\n")[0]
    tail = U * (U + 1) // 2
    assert body.count("sc::load_b<V>") == U * kn
    assert body.count("sc::load_b_tail<V>") == tail * kn
    assert body.count("sc::fma_row<V>") == (U + tail) * kn * km


def test_main_spmm_dictionary_and_dense(tmp_path):
    out = tmp_path / "k.hip"
    run(os.path.join(CG, "main_spmm.py"), str(out), "format", "4", "1", "1", "1", "i-j",
        "--pattern_dictionary", os.path.join(GOLDEN, "dict4_sub.txt"))
    assert sorted(int(m) for m, _ in _cases(out.read_text())) == sorted([15, 1, 2, 4, 8, 3])
    r = subprocess.run([sys.executable, os.path.join(CG, "main_spmm.py"), str(out), "dense", "4",
                        "1", "1", "1", "i-j"], capture_output=True, text=True)
    assert r.returncode != 0 and "dense" in r.stderr


def test_small_b_and_spmv_generators_fix_n(tmp_path):
    out = tmp_path / "s.hip"
    run(os.path.join(CG, "main_spmm_small_b_col.py"), str(out), "4", "1", "2")
    text = out.read_text()
    assert "sc_gen_spmm_small_km4_b2_record = {4, 1, 0, 15, 2," in text
    assert "if (N != 2) return hipErrorInvalidValue;" in text
    out = tmp_path / "v.hip"
    run(os.path.join(CG, "main_spmv.py"), str(out), "3", "1")
    text = out.read_text()
    assert "sc_gen_spmv_km3_record = {3, 1, 0, 7, 1," in text
    assert len(_cases(text)) == 7


DEMOS = os.path.join(ROOT, "sparse-computation_amd", "lib", "demos")


def test_demo_command_line_without_gpu():
    exe = os.path.join(DEMOS, "spmm_demo_gpu")
    if not os.path.exists(exe):
        pytest.skip("demos not built")
    r = subprocess.run([exe, "--help"], capture_output=True, text=True)
    assert r.returncode == 0 and "--b_matrix_columns" in r.stdout
    r = subprocess.run([exe, "-n", "SPMM", "-s", "CSR"], capture_output=True, text=True)
    assert r.returncode == 0 and "'matrix' is manditory" in r.stdout
    r = subprocess.run([exe, "-m", "x.cfmtx", "-n", "SPMM", "-s", "COO"], capture_output=True, text=True)
    assert "'storage_format' must be" in r.stdout
    r = subprocess.run([exe, "-m", "x.mtx", "-n", "SPMM", "-s", "CSR"], capture_output=True, text=True)
    assert r.returncode == 1 and "expects a .cfmtx" in r.stderr


@pytest.mark.skipif(not os.path.exists("/opt/rocm/bin/hipcc"), reason="hipcc not installed")
def test_run_script_builds_the_demo(tmp_path):
    mtx = tmp_path / "m.mtx"
    shutil.copy(os.path.join(GOLDEN, "real_64x40.mtx"), mtx)
    env = dict(os.environ, SC_DEMO_BUILD_ONLY="1")
    script = os.path.join(ROOT, "sparse-computation_amd", "run_local_spmm_small_b_col.sh")
    subprocess.run([script, str(mtx), "2"], check=True, capture_output=True, env=env, timeout=600)
    with open(tmp_path / "m-4-1.cfmtx") as a, open(os.path.join(GOLDEN, "real_64x40-4-1.cfmtx")) as b:
        assert a.read() == b.read()
    assert os.access(os.path.join(ROOT, "sparse-computation_amd", "build",
                                  "spmm_small_b_col_demo_gpu"), os.X_OK)


def test_time_analysis_generator_styles(tmp_path):
    # main_time_analysis.py <out> <m> <n> <compact>: pop-count bodies (compact 1)
    # or one body per pattern (compact 0), each with a standalone driver
    sys.path.insert(0, CG)
    import main_time_analysis as ta
    pop = tmp_path / "pop.hip"
    pat = tmp_path / "pat.hip"
    run(os.path.join(CG, "main_time_analysis.py"), str(pop), "4", "1", "1")
    run(os.path.join(CG, "main_time_analysis.py"), str(pat), "4", "1", "0")
    tp, tt = pop.read_text(), pat.read_text()
    for p in (1, 2, 3, 4):
        assert f"void pop{p}_wide(" in tp and f"void pop{p}_narrow(" in tp
    assert "pattern_1111" not in tp and "switch (__builtin_popcount((unsigned)mask))" in tp
    assert len(_cases(tt)) == 15 and "void wide_1011(" in tt
    for t, style in ((tp, "popcount"), (tt, "pattern")):
        assert "int main(int argc, char **argv)" in t and f"sc_gen_ta_{style}_km4_kn1_launch" in t
    assert ta.unit_name(4, 1, True) == "ta_popcount_km4_kn1"


@pytest.mark.skipif(not os.path.exists("/opt/rocm/bin/hipcc"), reason="hipcc not installed")
def test_time_analysis_resource_report(tmp_path):
    out = run(os.path.join(CG, "main_time_analysis.py"), str(tmp_path / "p.hip"), "3", "1", "1",
              "--report").stdout
    lines = out.splitlines()
    i = lines.index("kernel,code_bytes,vgprs,sgprs,scratch_bytes_per_lane,occupancy_waves_per_simd")
    rows = [l.split(",") for l in lines[i + 1:]]
    kernels = {r[0] for r in rows}
    assert "wide_kernel(km=3 V=2 stage)" in kernels and "gather_kernel(km=3 V=1 f32)" in kernels
    for r in rows:
        assert int(r[2]) > 0 and int(r[4]) == 0  # VGPRs used, nothing spilled to scratch
