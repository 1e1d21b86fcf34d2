"""GPU side of the path: a plan (the .cfmtx resident on one device) and the
pattern kernels, called through libsc's C ABI with torch tensors for the
dense operands.  There is no CPU fallback: without a HIP device the calls
raise."""
from __future__ import annotations

import ctypes as C

from ._lib import check, lib, torch
from .format import Cfmtx

PLAN_DROP_PADDING = 1
PLAN_TILED = 2
PLAN_CHUNKED = 4
PLAN_F16_VALUES = 8
PLAN_ROWS = 16
PLAN_PATTERNS = 32
PLAN_BANDS = 64
ACCUMULATE = 1


def _stream_handle(stream):
    if stream is None:
        return C.c_void_p(torch.cuda.current_stream().cuda_stream)
    if isinstance(stream, int):
        return C.c_void_p(stream)
    return C.c_void_p(stream.cuda_stream)


class GeneratedUnit:
    """A kernel unit emitted by code_gen/main_spmm.py, main_spmm_small_b_col.py
    or main_spmv.py and compiled to a shared object: its record (km, kn,
    masks, N variant) and launcher, looked up as sc_gen_<name>_record /
    sc_gen_<name>_launch."""

    def __init__(self, so_path: str, name: str):
        self.lib = C.CDLL(so_path)
        self.name = name
        self.record = C.c_void_p.in_dll(self.lib, f"sc_gen_{name}_record")
        self.record_ptr = C.cast(C.addressof(self.record), C.c_void_p)
        self.launch = C.cast(getattr(self.lib, f"sc_gen_{name}_launch"), C.c_void_p)

    def info(self) -> dict:
        f = (C.c_int32 * 5).from_address(C.addressof(self.record))
        return dict(zip(("km", "kn", "waves", "npatterns", "variant"), list(f)))


class Plan:
    """SpMMMixePatternGeneralCacheLess / SpMVMixePatternDecomposeByRowSeperated
    of the reference (the generated classes of example_cuda/*_utils.h): the
    format uploaded once, then launched on caller-owned B/C."""

    def __init__(self, cf: Cfmtx, flags: int = 0):
        h = C.c_void_p()
        check(lib().sc_plan_create(cf._h, flags, C.byref(h)))
        self._h = h
        self._free = lib().sc_plan_destroy
        # sc_plan_create uploads to the current HIP device
        self.device = torch.cuda.current_device()

    def __del__(self):
        # the free function is bound at creation: at interpreter exit this
        # module's globals may already be gone
        free = getattr(self, "_free", None)
        if free is not None and getattr(self, "_h", None) and self._h.value:
            free(self._h)
            self._h = C.c_void_p(None)

    def info(self) -> dict:
        v32 = [C.c_int32() for _ in range(4)]
        v64 = [C.c_int64() for _ in range(3)]
        check(lib().sc_plan_info(self._h, *[C.byref(x) for x in v32], *[C.byref(x) for x in v64]))
        return dict(zip(("m", "n", "km", "npanels", "nslots", "nvals", "nsegs"),
                        [x.value for x in v32 + v64]))

    def describe(self, N: int) -> str:
        """Kernel and launch geometry sc_spmm uses for N columns."""
        buf = C.create_string_buffer(256)
        check(lib().sc_plan_describe(self._h, N, buf, len(buf)))
        return buf.value.decode()

    def _check_device(self, t, name):
        if not t.is_cuda or t.device.index != self.device:
            raise ValueError(f"{name} must be on the plan's device cuda:{self.device}, got {t.device}")

    def _check_operand(self, t, rows, cols, name, dtype=None):
        dtype = torch.float32 if dtype is None else dtype
        if not (t.is_cuda and t.dtype == dtype and t.is_contiguous()):
            raise ValueError(f"{name} must be a contiguous {dtype} tensor on the GPU")
        self._check_device(t, name)
        if t.numel() != rows * cols:
            raise ValueError(f"{name} must hold {rows}x{cols} elements, got {tuple(t.shape)}")

    def spmm(self, B, C_out=None, accumulate=False, waves=0, stream=None):
        """C = A @ B (B: K x N row-major float32 CUDA tensor)."""
        info = self.info()
        N = B.shape[1] if B.dim() == 2 else 1
        self._check_operand(B, info["n"], N, "B")
        if C_out is None:
            C_out = torch.empty((info["m"], N), dtype=torch.float32, device=B.device)
        self._check_operand(C_out, info["m"], N, "C")
        check(lib().sc_spmm(self._h, C.c_void_p(B.data_ptr()), C.c_void_p(C_out.data_ptr()), N,
                            ACCUMULATE if accumulate else 0, waves, _stream_handle(stream)))
        return C_out

    def spmm_noalloc(self, B, C_out, accumulate=False, waves=0, stream=None):
        """C = A @ B through sc_spmm_noalloc: the split-K kernels use the
        library's static per-device scratch, nothing is allocated (C_out must
        be given)."""
        info = self.info()
        N = B.shape[1] if B.dim() == 2 else 1
        self._check_operand(B, info["n"], N, "B")
        self._check_operand(C_out, info["m"], N, "C")
        check(lib().sc_spmm_noalloc(self._h, C.c_void_p(B.data_ptr()), C.c_void_p(C_out.data_ptr()), N,
                                    ACCUMULATE if accumulate else 0, waves, _stream_handle(stream)))
        return C_out

    def spmm_ptr(self, b_ptr: int, c_ptr: int, N: int, flags: int = 0, waves: int = 0,
                 stream=None) -> None:
        """Raw-pointer form (no shape checks): for timing loops."""
        check(lib().sc_spmm(self._h, C.c_void_p(b_ptr), C.c_void_p(c_ptr), N, flags, waves,
                            _stream_handle(stream)))

    def spmm_generated(self, unit: GeneratedUnit, B, C_out=None, accumulate=False, waves=0,
                       stream=None):
        """C = A @ B through a generated kernel unit (checked against the plan)."""
        info = self.info()
        N = B.shape[1] if B.dim() == 2 else 1
        self._check_operand(B, info["n"], N, "B")
        if C_out is None:
            C_out = torch.empty((info["m"], N), dtype=torch.float32, device=B.device)
        self._check_operand(C_out, info["m"], N, "C")
        check(lib().sc_spmm_generated(self._h, unit.record_ptr, unit.launch,
                                      C.c_void_p(B.data_ptr()), C.c_void_p(C_out.data_ptr()), N,
                                      ACCUMULATE if accumulate else 0, waves,
                                      _stream_handle(stream)))
        return C_out

    def spmm_f16(self, B, C_out=None, accumulate=False, waves=0, stream=None):
        """C = A @ B in binary16 (B: K x N float16 CUDA tensor, N in 1, 2, 4;
        the plan must be created with PLAN_F16_VALUES).  fp32 accumulation."""
        info = self.info()
        N = B.shape[1] if B.dim() == 2 else 1
        if B.dtype != torch.float16 or not B.is_cuda or not B.is_contiguous() or B.shape[0] != info["n"]:
            raise ValueError(f"B must be a contiguous ({info['n']}, N) float16 device tensor")
        self._check_device(B, "B")
        if C_out is None:
            C_out = torch.empty((info["m"], N), dtype=torch.float16, device=B.device)
        if (C_out.dtype != torch.float16 or not C_out.is_cuda or not C_out.is_contiguous()
                or C_out.shape[0] != info["m"] or C_out.numel() != info["m"] * N):
            raise ValueError(f"C must be a contiguous ({info['m']}, {N}) float16 device tensor")
        self._check_device(C_out, "C")
        check(lib().sc_spmm_f16(self._h, C.c_void_p(B.data_ptr()), C.c_void_p(C_out.data_ptr()), N,
                                ACCUMULATE if accumulate else 0, waves, _stream_handle(stream)))
        return C_out

    def spmv(self, x, y=None, accumulate=False, stream=None):
        """y = A @ x (x: length-K float32 CUDA tensor)."""
        info = self.info()
        self._check_operand(x, info["n"], 1, "x")
        if y is None:
            y = torch.empty(info["m"], dtype=torch.float32, device=x.device)
        self._check_operand(y, info["m"], 1, "y")
        check(lib().sc_spmv(self._h, C.c_void_p(x.data_ptr()), C.c_void_p(y.data_ptr()),
                            ACCUMULATE if accumulate else 0, _stream_handle(stream)))
        return y
