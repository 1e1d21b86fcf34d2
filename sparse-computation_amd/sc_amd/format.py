"""Host objects of the path: CSR matrices, .mtx files and the .cfmtx format.

Mirrors the reference's host surface (include/Sparse_io.h:16-30,
include/compressed_format/CompressedFormat.h:88-279,
code_gen/ss_format/format_generator.py) on top of libsc.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from ._lib import check, lib

VALUES_REAL, VALUES_INTEGER, VALUES_PATTERN = 0, 1, 2
MTX_SCIPY, MTX_SYMLIB = 0, 1


def _arr(a, dtype):
    a = np.ascontiguousarray(a, dtype=dtype)
    return a, a.ctypes.data_as(C.POINTER(np.ctypeslib.as_ctypes_type(dtype)))


class Csr:
    """CSR matrix owned by libsc (sym_lib::CSR / scipy CSR of the reference)."""

    def __init__(self, handle):
        self._h = C.c_void_p(handle) if not isinstance(handle, C.c_void_p) else handle
        self._free = lib().sc_csr_free

    def __del__(self):
        # the free function is bound at creation: at interpreter exit this
        # module's globals may already be gone
        free = getattr(self, "_free", None)
        if free is not None and getattr(self, "_h", None) and self._h.value:
            free(self._h)
            self._h = C.c_void_p(None)

    @classmethod
    def from_mtx(cls, path: str, mode: int = MTX_SCIPY) -> "Csr":
        h = C.c_void_p()
        check(lib().sc_mtx_read(path.encode(), mode, C.byref(h)))
        return cls(h)

    @classmethod
    def from_arrays(cls, m, n, indptr, indices, data, kind=VALUES_REAL) -> "Csr":
        ip, ipp = _arr(indptr, np.int32)
        ix, ixp = _arr(indices, np.int32)
        dx, dxp = _arr(data, np.float64)
        h = C.c_void_p()
        check(lib().sc_csr_create(int(m), int(n), ipp, ixp, dxp, kind, C.byref(h)))
        return cls(h)

    @classmethod
    def synth_uniform(cls, m, n, density, sigma, seed) -> "Csr":
        h = C.c_void_p()
        check(lib().sc_synth_uniform(m, n, density, sigma, seed, C.byref(h)))
        return cls(h)

    @classmethod
    def synth_blocks(cls, m, n, density, sigma, seed) -> "Csr":
        h = C.c_void_p()
        check(lib().sc_synth_blocks(m, n, density, sigma, seed, C.byref(h)))
        return cls(h)

    @property
    def shape(self):
        m, n, nnz, kind = C.c_int32(), C.c_int32(), C.c_int64(), C.c_int32()
        check(lib().sc_csr_info(self._h, C.byref(m), C.byref(n), C.byref(nnz), C.byref(kind)))
        return m.value, n.value

    @property
    def nnz(self) -> int:
        nnz = C.c_int64()
        check(lib().sc_csr_info(self._h, None, None, C.byref(nnz), None))
        return nnz.value

    @property
    def kind(self) -> int:
        k = C.c_int32()
        check(lib().sc_csr_info(self._h, None, None, None, C.byref(k)))
        return k.value

    def arrays(self):
        """(indptr int32, indices int32, data float64) copies."""
        m, _ = self.shape
        nnz = self.nnz
        ip, ix, dx = C.POINTER(C.c_int32)(), C.POINTER(C.c_int32)(), C.POINTER(C.c_double)()
        check(lib().sc_csr_arrays(self._h, C.byref(ip), C.byref(ix), C.byref(dx)))
        indptr = np.ctypeslib.as_array(ip, (m + 1,)).copy()
        if nnz == 0:
            return indptr, np.zeros(0, np.int32), np.zeros(0, np.float64)
        return (indptr, np.ctypeslib.as_array(ix, (nnz,)).copy(),
                np.ctypeslib.as_array(dx, (nnz,)).copy())

    def write_mtx(self, path: str) -> None:
        check(lib().sc_mtx_write(self._h, path.encode()))


class Cfmtx:
    """Compressed format (MixedFormat<float> of per-pattern CompressedFormat)."""

    def __init__(self, handle):
        self._h = C.c_void_p(handle) if not isinstance(handle, C.c_void_p) else handle
        self._free = lib().sc_cfmtx_free

    def __del__(self):
        # the free function is bound at creation: at interpreter exit this
        # module's globals may already be gone
        free = getattr(self, "_free", None)
        if free is not None and getattr(self, "_h", None) and self._h.value:
            free(self._h)
            self._h = C.c_void_p(None)

    @classmethod
    def build(cls, csr: Csr, km: int, kn: int, dictionary: str | None = None) -> "Cfmtx":
        h = C.c_void_p()
        check(lib().sc_cfmtx_build(csr._h, km, kn, dictionary.encode() if dictionary else None,
                                   C.byref(h)))
        return cls(h)

    @classmethod
    def read(cls, path: str) -> "Cfmtx":
        h = C.c_void_p()
        check(lib().sc_cfmtx_read(path.encode(), C.byref(h)))
        return cls(h)

    def write(self, path: str) -> None:
        check(lib().sc_cfmtx_write(self._h, path.encode()))

    def text(self) -> str:
        n = C.c_int64()
        check(lib().sc_cfmtx_text(self._h, None, 0, C.byref(n)))
        buf = C.create_string_buffer(n.value + 1)
        check(lib().sc_cfmtx_text(self._h, buf, n.value + 1, C.byref(n)))
        return buf.raw[: n.value].decode()

    def info(self) -> dict:
        v = [C.c_int32() for _ in range(6)]
        check(lib().sc_cfmtx_info(self._h, *[C.byref(x) for x in v]))
        return dict(zip(("m", "n", "km", "npat", "kn", "npanels"), (x.value for x in v)))

    def pattern(self, i: int) -> dict:
        bits, pid, pop = C.c_char_p(), C.c_int32(), C.c_int32()
        rpp, cb, vals = C.POINTER(C.c_int32)(), C.POINTER(C.c_int32)(), C.POINTER(C.c_float)()
        nr, nc, nv = C.c_int64(), C.c_int64(), C.c_int64()
        check(lib().sc_cfmtx_pattern(self._h, i, C.byref(bits), C.byref(pid), C.byref(pop),
                                     C.byref(rpp), C.byref(nr), C.byref(cb), C.byref(nc),
                                     C.byref(vals), C.byref(nv)))

        def view(p, n, dt):
            return np.ctypeslib.as_array(p, (n,)).copy() if n else np.zeros(0, dt)

        return {"bits": bits.value.decode(), "id": pid.value, "pop": pop.value,
                "rpp": view(rpp, nr.value, np.int32), "cb": view(cb, nc.value, np.int32),
                "vals": view(vals, nv.value, np.float32)}

    def patterns(self):
        return [self.pattern(i) for i in range(self.info()["npat"])]


def load_cfmtx_matrices(path: str):
    """loadCfmtxMatrices (utils/Sparse_io.cpp:186-196): (Csr, Cfmtx)."""
    a, c = C.c_void_p(), C.c_void_p()
    check(lib().sc_load_cfmtx_matrices(path.encode(), C.byref(a), C.byref(c)))
    return Csr(a), Cfmtx(c)


def read_csr_matrix(path: str) -> Csr:
    """readCSRMatrix (utils/Sparse_io.cpp:198-206)."""
    a = C.c_void_p()
    check(lib().sc_read_csr_matrix(path.encode(), C.byref(a)))
    return Csr(a)


def read_compressed_format_matrix(path: str) -> Cfmtx:
    """readCompressedFormatMatrix (utils/Sparse_io.cpp:208-215)."""
    if not path.endswith(".cfmtx"):
        raise ValueError(f"readCompressedFormatMatrix expects a .cfmtx path: {path}")
    return Cfmtx.read(path)


def companion_mtx_path(path: str) -> str:
    """companionMtxPathFromCFMTX (utils/Sparse_io.cpp:28-46)."""
    buf = C.create_string_buffer(len(path.encode()) + 8)
    check(lib().sc_companion_mtx_path(path.encode(), buf, len(buf)))
    return buf.value.decode()


def patterns(km: int, kn: int = 1):
    """Bit strings of ids 0..2**(km*kn)-2 (build_patterns_map order)."""
    bits = km * kn
    n = C.c_int32()
    buf = C.create_string_buffer((bits + 1) * ((1 << bits) - 1))
    check(lib().sc_patterns(km, kn, buf, len(buf), C.byref(n)))
    raw = buf.raw
    return [raw[i * (bits + 1): i * (bits + 1) + bits].decode() for i in range(n.value)]


def synth_dense(count: int, seed: int) -> np.ndarray:
    out = np.empty(count, np.float32)
    check(lib().sc_synth_dense(out.ctypes.data_as(C.POINTER(C.c_float)), count, seed))
    return out


def synth_raw(seed: int, count: int) -> np.ndarray:
    out = np.empty(count, np.uint64)
    check(lib().sc_synth_raw(seed, out.ctypes.data_as(C.POINTER(C.c_uint64)), count))
    return out
