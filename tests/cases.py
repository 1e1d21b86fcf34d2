"""Shared test inputs: seeded matrices and dense operands, and the parity
check of a GPU result against the CPU oracle."""
from __future__ import annotations

import numpy as np

import oracle as O
import sc_amd

# max relative error normalised by (|A| |B|)_ij, the forward-error scale of a
# dot product; the path's fp32 tolerance against the fp64 check
REL_TOL = 1e-5


def synth_case(m, k, density, n, seed, sigma=0.05, structured=False):
    if structured:
        A = sc_amd.Csr.synth_blocks(m, k, density, sigma, seed)
    else:
        A = sc_amd.Csr.synth_uniform(m, k, density, sigma, seed)
    B = sc_amd.synth_dense(k * n, seed + 500).reshape(k, n)
    return A, B


def csr_f32(A):
    ip, ix, dx = A.arrays()
    return ip, ix, dx.astype(np.float32)


def oracle_check_acc(A, B, C_gpu, C0):
    """Max relative error of an accumulating launch (C = C0 + A*B): C itself
    against c64 + C0, normalised by (|A| |B|)_ij + |C0_ij|, the forward-error
    scale of the dot product plus the one extra addition."""
    m, _ = A.shape
    n = B.shape[1]
    ip, ix, ax = csr_f32(A)
    c64, cab = O.spmm_f64(m, n, ip, ix, ax, B)
    c0 = np.asarray(C0, np.float64).reshape(m, n)
    return O.max_rel_err(np.asarray(C_gpu).reshape(m, n), c64 + c0, cab + np.abs(c0))


def oracle_check(A, B, C_gpu, tol=REL_TOL):
    """(max_rel_err, max elementwise rel err with floor 1e-6 max|C|)."""
    m, _ = A.shape
    n = B.shape[1]
    ip, ix, ax = csr_f32(A)
    c64, cab = O.spmm_f64(m, n, ip, ix, ax, B)
    err = O.max_rel_err(np.asarray(C_gpu).reshape(m, n), c64, cab)
    floor = 1e-6 * max(1e-30, float(np.abs(c64).max()) if c64.size else 1.0)
    elem = float(np.max(np.abs(np.asarray(C_gpu).reshape(m, n) - c64) /
                        np.maximum(np.abs(c64), floor))) if c64.size else 0.0
    return err, elem
