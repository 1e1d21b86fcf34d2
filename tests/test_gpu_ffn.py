"""GPU parity on the transformer FFN configuration: A 2048x512 and 512x2048
fp32 at 50/70/80/90/95/98 % sparsity (uniform random masks, values
N(0, 0.02^2)), B dense U(-1, 1) with N = 128, coarsen factors km 4 x kn 1,
the seeds the sweep times (bench.py sweep_cases).  Every case runs on the
default plan (which picks the one-row or the pattern layout per launch) and
on the pattern layout alone, against the fp64 oracle: max relative error
<= 1e-5 normalised by (|A| |B|)_ij.
"""
import numpy as np
import pytest

import sc_amd
from cases import REL_TOL, oracle_check

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

DEV = "cuda:0"
BASE = 0x5EED0000
N = 128


def ffn_matrix(shape, sparsity):
    m, k = shape
    seed = BASE + (3000 if m > k else 3100) + sparsity
    return sc_amd.Csr.synth_uniform(m, k, 1 - sparsity / 100, 0.02, seed)


@pytest.mark.parametrize("sparsity", [50, 70, 80, 90, 95, 98])
@pytest.mark.parametrize("shape", [(2048, 512), (512, 2048)])
def test_ffn_config(shape, sparsity):
    A = ffn_matrix(shape, sparsity)
    m, k = shape
    assert A.nnz == round((1 - sparsity / 100) * m * k)
    B = sc_amd.synth_dense(k * N, BASE + 500 + N).reshape(k, N)
    cf = sc_amd.Cfmtx.build(A, 4, 1)
    Bt = torch.from_numpy(B).to(DEV)
    for flags in (0, sc_amd.PLAN_PATTERNS):
        plan = sc_amd.Plan(cf, flags)
        Ct = torch.full((m, N), float("nan"), device=DEV)  # must be overwritten
        plan.spmm(Bt, Ct)
        torch.cuda.synchronize()
        err, _ = oracle_check(A, B, Ct.cpu().numpy())
        assert err <= REL_TOL, (shape, sparsity, flags, plan.describe(N), err)
