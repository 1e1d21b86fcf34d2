"""Vendor-library baselines (libsc_vendor.so: rocSPARSE, hipBLAS) compute the
same product as the pattern kernels: the MI355X rows that stand in for the
reference demo's cuSPARSE / cuBLAS rows
(example_cuda/spmm_demo_gpu_utils.h:437-940).  These are baselines, so the
check is that they multiply the same A and B, not that they match bit for
bit."""
import numpy as np
import pytest

from cases import REL_TOL, oracle_check, synth_case

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def V():
    from sc_amd import vendor
    return vendor


def _run(V, A, B, kind, alg=0):
    dev = torch.device("cuda:0")
    m, k = A.shape
    n = B.shape[1]
    h = V.Vendor(A, kind, n, alg)
    Bt = torch.from_numpy(np.ascontiguousarray(B)).to(dev)
    if kind == V.ROCSPARSE_SPMV:
        Bt = Bt.reshape(k)
    Ct = torch.full((m, n) if kind != V.ROCSPARSE_SPMV else (m,), float("nan"), device=dev)
    h.bind(Bt, Ct)
    h.run()
    h.fetch()
    torch.cuda.synchronize()
    return Ct.cpu().numpy().reshape(m, n), h


@pytest.mark.parametrize("alg", [0, 1, 2, 3, 4])
@pytest.mark.parametrize("n", [1, 4, 32, 128])
def test_rocsparse_spmm_matches_oracle(V, alg, n):
    A, B = synth_case(300, 257, 0.2, n, 7100 + n)
    C, _ = _run(V, A, B, V.ROCSPARSE_SPMM, alg)
    err, _ = oracle_check(A, B, C)
    assert err <= REL_TOL, err


@pytest.mark.parametrize("alg", [0, 1, 2, 3])
def test_rocsparse_spmv_matches_oracle(V, alg):
    A, B = synth_case(512, 512, 0.3, 1, 7200)
    C, _ = _run(V, A, B, V.ROCSPARSE_SPMV, alg)
    err, _ = oracle_check(A, B, C)
    assert err <= REL_TOL, err


@pytest.mark.parametrize("kind", ["HIPBLAS_SGEMM", "HIPBLAS_GEMMEX"])
def test_hipblas_fp32_matches_oracle(V, kind):
    A, B = synth_case(256, 384, 0.1, 64, 7300)
    C, h = _run(V, A, B, getattr(V, kind))
    err, _ = oracle_check(A, B, C)
    assert err <= REL_TOL, err
    assert h.device_bytes() == 256 * 384 * 4


def test_hipblas_half_is_an_fp16_product(V):
    # fp16 inputs: a relative error of a few 2^-11 of |A||B|, not fp32 accuracy
    A, B = synth_case(256, 384, 0.1, 64, 7400)
    C, _ = _run(V, A, B, V.HIPBLAS_HALF)
    err, _ = oracle_check(A, B, C)
    assert 1e-6 < err <= 5e-3, err


def test_vendor_rejects_bad_arguments(V):
    A, _ = synth_case(64, 64, 0.2, 1, 7500)
    with pytest.raises(V.VendorError, match="SpMV needs N == 1"):
        V.Vendor(A, V.ROCSPARSE_SPMV, 4)
    with pytest.raises(V.VendorError, match="unknown vendor kind"):
        V.Vendor(A, 17, 4)
    h = V.Vendor(A, V.ROCSPARSE_SPMM, 4)
    with pytest.raises(V.VendorError, match="not bound"):
        h.run()
