"""GPU: the time-analysis programs (code_gen/main_time_analysis.py, built by
the libsc Makefile for km 4, kn 1) run both code-generation styles on a
seeded matrix and check the result against the fp64 product (exit status 0,
max error normalised by |A||B| <= 1e-5)."""
import os
import subprocess

import pytest

import sc_amd

pytestmark = pytest.mark.gpu
TA = os.path.join(os.path.dirname(sc_amd.LIB_PATH), "time_analysis")


@pytest.mark.parametrize("style", ["pattern", "popcount"])
@pytest.mark.parametrize("n", [1, 4, 32, 128])
def test_time_analysis_program(style, n):
    exe = os.path.join(TA, f"ta_{style}_km4_kn1")
    out = subprocess.run([exe, "1000", "900", str(n), "0.1", "5"], capture_output=True, text=True,
                         timeout=120)
    assert out.returncode == 0, out.stderr + out.stdout
    head, row = out.stdout.strip().splitlines()[-2:]
    assert head == "style,km,kn,M,K,N,nnz,us_min,us_median,max_rel_err"
    f = row.split(",")
    assert f[0] == style and f[5] == str(n) and float(f[-1]) <= 1e-5
