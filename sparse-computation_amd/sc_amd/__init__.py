"""sc_amd -- Python binding of libsc, the MI355X implementation of the
enumerate-and-sparse-coarsen SpMM/SpMV path.

Host: ``Csr`` (.mtx / arrays / seeded synthetic matrices), ``Cfmtx`` (build,
write byte-exact, read), ``load_cfmtx_matrices``.  Device: ``Plan`` (upload
once) with ``spmm`` / ``spmv`` on torch tensors.  All work is done by
``lib/libsc.so``; nothing here computes a result itself.
"""
from ._lib import EXPORTS, LIB_PATH, LibscError, lib  # noqa: F401
from .device import (ACCUMULATE, PLAN_BANDS, PLAN_CHUNKED, PLAN_DROP_PADDING, PLAN_F16_VALUES,  # noqa: F401
                     PLAN_PATTERNS, PLAN_ROWS, PLAN_TILED, GeneratedUnit, Plan)
from .format import (MTX_SCIPY, MTX_SYMLIB, VALUES_INTEGER, VALUES_PATTERN,  # noqa: F401
                     VALUES_REAL, Cfmtx, Csr, companion_mtx_path, load_cfmtx_matrices,
                     patterns, read_compressed_format_matrix, read_csr_matrix, synth_dense,
                     synth_raw)
