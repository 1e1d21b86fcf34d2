"""ctypes binding of libsc_vendor.so (include/sc_vendor.h): rocSPARSE and
hipBLAS on the same matrix as the pattern kernels, the MI355X counterparts of
the cuSPARSE / cuBLAS rows of the reference's demos
(example_cuda/spmm_demo_gpu_utils.h:437-940).  Baselines only: nothing in
the pattern-kernel path uses this module."""
from __future__ import annotations

import ctypes as C
import os

from ._lib import PKG_ROOT, lib as _libsc
from .format import Csr

VENDOR_PATH = os.path.join(PKG_ROOT, "lib", "libsc_vendor.so")

ROCSPARSE_SPMM = 0
ROCSPARSE_SPMV = 1
HIPBLAS_SGEMM = 2
HIPBLAS_GEMMEX = 3
HIPBLAS_HALF = 4

KIND_NAMES = {
    ROCSPARSE_SPMM: "rocSPARSE SpMM",
    ROCSPARSE_SPMV: "rocSPARSE SpMV",
    HIPBLAS_SGEMM: "hipBLAS Sgemm",
    HIPBLAS_GEMMEX: "hipBLAS GemmEx",
    HIPBLAS_HALF: "hipBLAS Half",
}
SPMM_ALGS = {0: "default", 1: "csr_row_split_lds", 2: "csr_row_split_shfl", 3: "csr_nnz_split",
             4: "csr_merge_path"}

_v = None
vp = C.c_void_p


class VendorError(RuntimeError):
    pass


def vlib():
    global _v
    if _v is None:
        _libsc()  # torch's HIP runtime and libsc first
        if not os.path.exists(VENDOR_PATH):
            raise VendorError(f"{VENDOR_PATH} is not built (make -C sparse-computation_amd/csrc vendor)")
        L = C.CDLL(VENDOR_PATH)
        sigs = {
            "sc_vendor_last_error": ([], C.c_char_p),
            "sc_vendor_create": ([vp, C.c_int32, C.c_int32, C.c_int32, C.POINTER(vp)], C.c_int),
            "sc_vendor_bind": ([vp, vp, vp, vp], C.c_int),
            "sc_vendor_run": ([vp, vp], C.c_int),
            "sc_vendor_fetch": ([vp, vp], C.c_int),
            "sc_vendor_device_bytes": ([vp], C.c_int64),
            "sc_vendor_destroy": ([vp], None),
        }
        for name, (args, res) in sigs.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = res
        _v = L
    return _v


def _check(rc):
    if rc != 0:
        raise VendorError(f"libsc_vendor error {rc}: {vlib().sc_vendor_last_error().decode()}")


class Vendor:
    """One vendor-library product C = A*B (or y = A*x) bound to one N."""

    def __init__(self, csr: Csr, kind: int, N: int, alg: int = 0):
        self.kind, self.N, self.alg = kind, N, alg
        self.m, self.k = csr.shape
        h = vp()
        _check(vlib().sc_vendor_create(csr._h, kind, N, alg, C.byref(h)))
        self._csr = csr  # keeps the host matrix alive while the handle exists
        self._destroy = vlib().sc_vendor_destroy
        self.handle = h
        self._bound = None

    def __del__(self):
        # the destroy function is bound at creation: at interpreter exit this
        # module's globals may already be gone
        h = getattr(self, "handle", None)
        destroy = getattr(self, "_destroy", None)
        if h and destroy is not None:
            destroy(h)
            self.handle = None

    @property
    def name(self) -> str:
        n = KIND_NAMES[self.kind]
        if self.kind == ROCSPARSE_SPMM:
            n += f" ({SPMM_ALGS.get(self.alg, self.alg)})"
        return n

    def bind(self, B, C_out, stream=None):
        """Attach device tensors B (K x N, or K) and C (M x N, or M), fp32."""
        import torch
        for t, rows, nm in ((B, self.k, "B"), (C_out, self.m, "C")):
            if t.dtype != torch.float32 or not t.is_cuda or not t.is_contiguous():
                raise ValueError(f"{nm} must be a contiguous fp32 device tensor")
            if t.shape[0] != rows or t.numel() != rows * self.N:
                raise ValueError(f"{nm} has shape {tuple(t.shape)}, expected ({rows}, {self.N})")
        s = (stream or torch.cuda.current_stream()).cuda_stream
        _check(vlib().sc_vendor_bind(self.handle, B.data_ptr(), C_out.data_ptr(), s))
        self._bound = (B, C_out, s)

    def run(self):
        _check(vlib().sc_vendor_run(self.handle, self._bound[2] if self._bound else None))

    def fetch(self):
        _check(vlib().sc_vendor_fetch(self.handle, self._bound[2] if self._bound else None))

    def device_bytes(self) -> int:
        return int(vlib().sc_vendor_device_bytes(self.handle))
