"""CPU oracle for the enumerate-and-sparse-coarsen path (Python side).

TEST INFRASTRUCTURE ONLY.  Only tests/, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` import this module, and only as the
checker (or the timed CPU baseline).  The product never imports it.

The heavy loops live in ``sc_oracle.c`` (built into ``oracle/_build``); this
module wraps them with ctypes and restates the small Python pieces of the
reference directly:

* ``patterns_map``            -- code_gen/pattern_utiles/pattern_dictionary.py:29-37
* ``read_pattern_dictionary`` -- code_gen/pattern_utiles/pattern_dictionary.py:49-60
* ``cfmtx_text``              -- code_gen/ss_format/format_generator.py:132-160
* ``mtx_to_csr``              -- format_generator.py:214-215 (scipy.io.mmread(path).tocsr(),
                                 the reference's own third-party call; scipy 1.15.3 here)

Pinning of each function is listed in the header of ``sc_oracle.c``; the value
text of ``cfmtx_text`` is CPython's ``repr(float)`` (numpy 2.2.6's
``str(np.float64)`` prints the same text, checked in the tests).
"""
from __future__ import annotations

import ctypes as C
import ctypes as _ct
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "libsc_oracle.so")
REF_DUMP = os.path.join(HERE, "_ref", "ref_cfmtx_dump")

_lib = None


def build() -> None:
    """Compile sc_oracle.c (and the reference loaders when present)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        i32p = C.POINTER(C.c_int32)
        L.or_pattern_masks.argtypes = [C.c_int, C.c_int, i32p]
        L.or_pattern_masks.restype = C.c_int
        L.or_build.argtypes = [C.c_int32, C.c_int32, i32p, i32p, C.POINTER(C.c_double), C.c_int32,
                               C.c_int32, C.c_int32, i32p, i32p, i32p]
        L.or_build.restype = C.POINTER(_OrCfmtx)
        L.or_cfmtx_free.argtypes = [C.POINTER(_OrCfmtx)]
        L.or_read_cfmtx.argtypes = [C.c_char_p]
        L.or_read_cfmtx.restype = C.POINTER(_OrRead)
        L.or_read_free.argtypes = [C.POINTER(_OrRead)]
        fp = C.POINTER(C.c_float)
        L.or_spmm_csr_float.argtypes = [C.c_int, C.c_int, i32p, i32p, fp, fp, fp]
        L.or_spmv_csr_float.argtypes = [C.c_int, i32p, i32p, fp, fp, fp]
        L.or_spmm_f64.argtypes = [C.c_int, C.c_int, i32p, i32p, fp, fp, C.POINTER(C.c_double),
                                  C.POINTER(C.c_double)]
        _lib = L
    return _lib


class _OrCfmtx(C.Structure):
    _fields_ = [("num_row", C.c_int32), ("num_col", C.c_int32), ("kernel_rows", C.c_int32),
                ("vector_length", C.c_int32), ("npat", C.c_int32), ("npanels", C.c_int32),
                ("rpp", C.POINTER(C.c_int32)), ("ncb", C.POINTER(C.c_int64)),
                ("cb", C.POINTER(C.POINTER(C.c_int32))), ("nval", C.POINTER(C.c_int64)),
                ("val", C.POINTER(C.POINTER(C.c_double))),
                ("pad", C.POINTER(C.POINTER(C.c_uint8)))]


class _OrRead(C.Structure):
    _fields_ = [("num_rows", C.c_int32), ("num_columns", C.c_int32), ("kernel_rows", C.c_int32),
                ("num_patterns", C.c_int32), ("vector_length", C.c_int32), ("nrpp", C.c_int32),
                ("pop", C.POINTER(C.c_int32)), ("rpp", C.POINTER(C.c_int32)),
                ("npp", C.POINTER(C.c_int32)), ("ncb", C.POINTER(C.c_int64)),
                ("cb", C.POINTER(C.POINTER(C.c_int32))), ("nnz", C.POINTER(C.c_int64)),
                ("val", C.POINTER(C.POINTER(C.c_float)))]


def _ptr(a, ctype):
    return a.ctypes.data_as(C.POINTER(ctype))


# --------------------------------------------------------------------------
# Pattern enumeration
# --------------------------------------------------------------------------

def patterns_map(kernel_m: int, kernel_n: int = 1) -> dict:
    """build_patterns_map (pattern_dictionary.py:29-37): tuple(bool) -> id."""
    bits = kernel_m * kernel_n
    masks = np.zeros(2 ** bits - 1, dtype=np.int32)
    n = lib().or_pattern_masks(kernel_m, kernel_n, _ptr(masks, C.c_int32))
    assert n == len(masks)
    out = {}
    for pid, m in enumerate(masks.tolist()):
        out[tuple(bool((m >> c) & 1) for c in range(bits))] = pid
    return out


def read_pattern_dictionary(path: str) -> dict:
    """read_pattern_dictionary (pattern_dictionary.py:49-60) followed by the
    conversion to the ``patterns`` dict in format_generator.py:200-205."""
    id_to_bin = {}
    with open(path) as f:
        f.readline().split()
        for line in f:
            value, key = line.split()
            id_to_bin[int(key)] = value
    return {tuple(c == "1" for c in v): int(k) for k, v in id_to_bin.items()}


# --------------------------------------------------------------------------
# Builder + writer
# --------------------------------------------------------------------------

def mtx_to_csr(path: str):
    """scipy.io.mmread(path).tocsr() exactly as format_generator.py:214-215.

    Returns (M, K, indptr int32, indices int32, data, is_integer)."""
    from scipy.io import mmread
    A = mmread(path).tocsr()
    data = A.data
    is_int = np.issubdtype(data.dtype, np.integer)
    return (A.shape[0], A.shape[1], A.indptr.astype(np.int32), A.indices.astype(np.int32),
            data, is_int)


def build(M, K, indptr, indices, data, km, kn, patterns: dict):
    """csr_to_compressed_format_converter + transform_row_panel
    (format_generator.py:36-129) through sc_oracle.c.

    Returns dict with rpp (list of int lists), cb, vals (float64 lists),
    pad (bool lists) per pattern id, or None where the reference raises."""
    keys = list(patterns.items())
    key_mask = np.array([sum(1 << c for c, b in enumerate(k) if b) for k, _ in keys], np.int32)
    key_len = np.array([len(k) for k, _ in keys], np.int32)
    key_id = np.array([v for _, v in keys], np.int32)
    indptr = np.ascontiguousarray(indptr, np.int32)
    indices = np.ascontiguousarray(indices, np.int32)
    data = np.ascontiguousarray(data, np.float64)
    L = lib()
    r = L.or_build(M, K, _ptr(indptr, C.c_int32), _ptr(indices, C.c_int32),
                   _ptr(data, C.c_double), km, kn, len(keys), _ptr(key_mask, C.c_int32),
                   _ptr(key_len, C.c_int32), _ptr(key_id, C.c_int32))
    if not r:
        return None
    f = r.contents
    npan = f.npanels
    out = {"num_row": f.num_row, "num_col": f.num_col, "kernel_rows": f.kernel_rows,
           "vector_length": f.vector_length, "rpp": [], "cb": [], "vals": [], "pad": []}
    for p in range(f.npat):
        out["rpp"].append([f.rpp[p * (npan + 1) + j] for j in range(npan + 1)])
        n = f.ncb[p]
        out["cb"].append(np.ctypeslib.as_array(f.cb[p], (n,)).copy() if n else np.zeros(0, np.int32))
        n = f.nval[p]
        out["vals"].append(np.ctypeslib.as_array(f.val[p], (n,)).copy() if n else np.zeros(0))
        out["pad"].append(np.ctypeslib.as_array(f.pad[p], (n,)).astype(bool) if n
                          else np.zeros(0, bool))
    L.or_cfmtx_free(r)
    return out


def _value_text(v: float, pad: bool) -> str:
    # format_generator.py:80-81 vstacks a float64 csr_matrix of padding rows
    # onto the input, which upcasts integer and pattern fields to float64:
    # every real value prints as a float (an integer field's 7 as "7.0").
    if pad:
        return "0"
    return repr(float(v))


def cfmtx_text(cf: dict, patterns: dict, is_int: bool = False) -> str:
    """format_writer (format_generator.py:132-160) as a string.  `is_int` is
    accepted for the field kind of the .mtx but does not change the text."""
    out = [f"{cf['num_row']} {cf['num_col']} {cf['kernel_rows']} {len(patterns)} "
           f"{cf['vector_length']}\n"]
    for key, val in patterns.items():
        out.append("".join(str(int(x)) for x in key) + f" {val} \n")
    for i in range(len(patterns)):
        out.append(" ".join(str(x) for x in cf["rpp"][i]) + "\n")
        out.append(" ".join(str(int(x)) for x in cf["cb"][i]) + "\n")
        out.append(" ".join(_value_text(v, p)
                            for v, p in zip(cf["vals"][i].tolist(), cf["pad"][i].tolist())) + "\n")
    return "".join(out)


def format_generator(path: str, km: int, kn: int, pattern_dictionary: str = "false") -> str:
    """The whole of format_generator.py's __main__ (:175-225) for one .mtx,
    returning the .cfmtx text instead of writing it."""
    if pattern_dictionary != "false":
        patterns = read_pattern_dictionary(pattern_dictionary)
    else:
        patterns = patterns_map(km, 1)
    M, K, ip, ix, data, is_int = mtx_to_csr(path)
    cf = build(M, K, ip, ix, data.astype(np.float64), km, kn, patterns)
    if cf is None:
        raise ZeroDivisionError("pattern with no ones")
    return cfmtx_text(cf, patterns, is_int)


# --------------------------------------------------------------------------
# Reader
# --------------------------------------------------------------------------

def read_cfmtx(path: str):
    """readCFMTXFile (utils/Sparse_io.cpp:84-182): per pattern RPP, NPP, CB,
    NNZ (float32), plus the header fields.  None if unopenable/invalid."""
    L = lib()
    r = L.or_read_cfmtx(path.encode())
    if not r:
        return None
    f = r.contents
    P, nrpp = f.num_patterns, f.nrpp
    out = {"num_rows": f.num_rows, "num_columns": f.num_columns, "kernel_rows": f.kernel_rows,
           "num_patterns": P, "vector_length": f.vector_length, "nrpp": nrpp,
           "pop": [f.pop[i] for i in range(P)], "rpp": [], "npp": [], "cb": [], "nnz": []}
    for i in range(P):
        out["rpp"].append(np.array([f.rpp[i * nrpp + j] for j in range(nrpp)], np.int32))
        out["npp"].append(np.array([f.npp[i * nrpp + j] for j in range(nrpp)], np.int32))
        n = f.ncb[i]
        out["cb"].append(np.ctypeslib.as_array(f.cb[i], (n,)).copy() if n else np.zeros(0, np.int32))
        n = f.nnz[i]
        out["nnz"].append(np.ctypeslib.as_array(f.val[i], (n,)).copy() if n
                          else np.zeros(0, np.float32))
    L.or_read_free(r)
    return out


def ref_dump_available() -> bool:
    return os.path.exists(REF_DUMP)


def ref_read_cfmtx(path: str):
    """The reference's own readCompressedFormatMatrix, compiled from
    /root/reference into oracle/_ref (only where the reference is mounted)."""
    out = subprocess.run([REF_DUMP, "cfmtx", path], check=True, capture_output=True, text=True)
    return _parse_ref_dump(out.stdout)


def ref_read_csr(path: str):
    """The reference's readCSRMatrix (companion .mtx of a .cfmtx path)."""
    out = subprocess.run([REF_DUMP, "csr", path], check=True, capture_output=True, text=True)
    lines = out.stdout.splitlines()
    m, n, nnz = map(int, lines[0].split())
    p = np.array(lines[1].split(), np.int64)
    i = np.array(lines[2].split(), np.int64) if nnz else np.zeros(0, np.int64)
    x = (np.array([int(t, 16) for t in lines[3].split()], np.uint64).view(np.float64)
         if nnz else np.zeros(0))
    return {"m": m, "n": n, "nnz": nnz, "p": p, "i": i, "x": x}


def _parse_ref_dump(text: str):
    lines = text.splitlines()
    P = int(lines[0].split()[0])
    pos = 1
    pats = []
    for _ in range(P):
        km, kn, m, n, pm, nrpp, nnz, ncb = map(int, lines[pos].split())
        rpp = np.array(lines[pos + 1].split(), np.int64)
        npp = np.array(lines[pos + 2].split(), np.int64)
        cb = np.array(lines[pos + 3].split(), np.int64)
        vals = np.array([int(t, 16) for t in lines[pos + 4].split()], np.uint32).view(np.float32)
        pats.append({"km": km, "kn": kn, "m": m, "n": n, "pm": pm, "nrpp": nrpp, "nnz": nnz,
                     "rpp": rpp, "npp": npp, "cb": cb, "vals": vals})
        pos += 5
    return pats


# --------------------------------------------------------------------------
# CPU SpMM / SpMV
# --------------------------------------------------------------------------

def spmm_csr_float(M, N, indptr, indices, vals_f32, B, C=None):
    """spmm_csr_float (example_cuda/spmm_demo_gpu_utils.h:25-36): C += A*B."""
    ip = np.ascontiguousarray(indptr, np.int32)
    ix = np.ascontiguousarray(indices, np.int32)
    ax = np.ascontiguousarray(vals_f32, np.float32)
    B = np.ascontiguousarray(B, np.float32)
    out = np.zeros((M, N), np.float32) if C is None else C
    lib().or_spmm_csr_float(M, N, _ptr(ip, _ct.c_int32), _ptr(ix, _ct.c_int32),
                            _ptr(ax, _ct.c_float), _ptr(B, _ct.c_float), _ptr(out, _ct.c_float))
    return out


def spmv_csr_float(M, indptr, indices, vals_f32, x, y=None):
    """spmv_csr_float (example_cuda/spmv_demo_gpu_utils.h:86-98): y += A*x."""
    ip = np.ascontiguousarray(indptr, np.int32)
    ix = np.ascontiguousarray(indices, np.int32)
    ax = np.ascontiguousarray(vals_f32, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    if y is None:
        y = np.zeros(M, np.float32)
    lib().or_spmv_csr_float(M, _ptr(ip, C.c_int32), _ptr(ix, C.c_int32), _ptr(ax, C.c_float),
                            _ptr(x, C.c_float), _ptr(y, C.c_float))
    return y


def spmm_f64(M, N, indptr, indices, vals_f32, B):
    """fp64 product of the fp32 operands and the |A|*|B| bound."""
    ip = np.ascontiguousarray(indptr, np.int32)
    ix = np.ascontiguousarray(indices, np.int32)
    ax = np.ascontiguousarray(vals_f32, np.float32)
    B = np.ascontiguousarray(B, np.float32)
    c64 = np.zeros((M, N), np.float64)
    cab = np.zeros((M, N), np.float64)
    lib().or_spmm_f64(M, N, _ptr(ip, C.c_int32), _ptr(ix, C.c_int32), _ptr(ax, C.c_float),
                      _ptr(B, C.c_float), _ptr(c64, C.c_double), _ptr(cab, C.c_double))
    return c64, cab


def max_rel_err(C_test, c64, cab):
    """max |C - C64| / (|A|*|B|), with zero bound entries requiring C == 0."""
    d = np.abs(C_test.astype(np.float64) - c64)
    nz = cab > 0
    err = float(np.max(d[nz] / cab[nz])) if nz.any() else 0.0
    if (~nz).any() and float(np.max(d[~nz])) > 0:
        return float("inf")
    return err
