"""bench.py's command line on the CPU: one GPU only, and every sweep case
runs by name through --config with its own N and coarsening."""
import argparse
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr


def test_sweep_cases_cover_every_configuration():
    names = [c[0] for c in bench.sweep_cases()]
    assert len(names) == len(set(names))
    assert "spmv_512_d30" in names
    assert {f"smallB_512_d20_n{n}" for n in (1, 2, 4)} <= set(names)
    assert sum(n.startswith("largeB_512_d10_") for n in names) == 3 * 6 * 8
    assert sum(n.startswith("ffn_") for n in names) == 12
    assert {f"structured_4096_d10_n{n}" for n in (1, 32, 128)} <= set(names)


def test_config_by_case_name_takes_its_shape():
    args = argparse.Namespace(config="smallB_512_d20_n4", n=128, km=1, kn=1)
    A, name = bench.workload(args)
    assert name == "smallB_512_d20_n4"
    assert (args.n, args.km, args.kn) == (4, 4, 2)
    assert A.shape == (512, 512)
    args = argparse.Namespace(config="no_such_case", n=128, km=4, kn=1)
    try:
        bench.workload(args)
    except SystemExit as e:
        assert "unknown --config" in str(e)
    else:
        raise AssertionError("an unknown configuration was accepted")
