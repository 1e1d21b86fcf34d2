/*
 * sc_api.h -- C ABI of libsc, the MI355X (gfx950) implementation of the
 * enumerate-and-sparse-coarsen SpMM/SpMV path of hosseinal/sparse-computation.
 *
 * Every entry point returns an int status (SC_OK == 0); on failure
 * sc_last_error() returns a thread-local message.  No C++ exception crosses
 * this boundary.  Objects are opaque and owned by the caller, who frees them
 * with the matching *_free / *_destroy call.  Device pointers are plain
 * `const float *` / `float *` allocated by the caller (hipMalloc, torch, ...);
 * streams are passed as `void *` holding a hipStream_t (NULL = null stream).
 *
 * Each declaration names the reference interface it replaces (file:line in
 * the reference tree).
 */
#ifndef SC_API_H
#define SC_API_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SC_ABI_VERSION 2

/* status codes */
#define SC_OK 0
#define SC_ERR_ARG 1         /* invalid argument */
#define SC_ERR_IO 2          /* file cannot be opened / written */
#define SC_ERR_FORMAT 3      /* malformed .mtx / .cfmtx / dictionary text */
#define SC_ERR_HIP 4         /* HIP runtime error */
#define SC_ERR_UNSUPPORTED 5 /* valid input outside what this build handles */
#define SC_ERR_NOMEM 6       /* host allocation failed */
#define SC_ERR_INTERNAL 7

/* value kinds of a matrix (they decide how .cfmtx values are printed) */
#define SC_VALUES_REAL 0
#define SC_VALUES_INTEGER 1
#define SC_VALUES_PATTERN 2

/* .mtx reader modes */
#define SC_MTX_SCIPY 0  /* scipy.io.mmread(p).tocsr(): duplicates summed   */
#define SC_MTX_SYMLIB 1 /* sym_lib reader of the demos: duplicates kept     */

typedef struct sc_csr sc_csr;     /* CSR matrix (host)                        */
typedef struct sc_cfmtx sc_cfmtx; /* compressed format (host)                 */
typedef struct sc_plan sc_plan;   /* compressed format resident on one GPU    */

/* Message of the last failed call on this thread ("" if none). */
const char *sc_last_error(void);
int sc_abi_version(void);

/* ---------------------------------------------------------------- patterns */

/* build_patterns_map(kernel_m, kernel_n) / generate_pattern_dictionary(m, n)
 * (code_gen/pattern_utiles/pattern_dictionary.py:29-46).  Writes the bit
 * string of every id 0 .. 2^(km*kn)-2 into `bits` (km*kn chars + NUL each,
 * stride km*kn+1); returns the count through *npat. */
int sc_patterns(int32_t km, int32_t kn, char *bits, int64_t bits_len, int32_t *npat);

/* ---------------------------------------------------------------- CSR / mtx */

/* readCSRMatrixFromMTX (utils/Sparse_io.cpp:48-82) with mode SC_MTX_SYMLIB;
 * scipy.io.mmread(path).tocsr() (code_gen/ss_format/format_generator.py:214-215)
 * with mode SC_MTX_SCIPY. */
int sc_mtx_read(const char *path, int32_t mode, sc_csr **out);
/* Write a coordinate general .mtx (values as Python repr of the double). */
int sc_mtx_write(const sc_csr *A, const char *path);
/* Copy caller arrays into a new CSR (columns sorted and unique per row). */
int sc_csr_create(int32_t m, int32_t n, const int32_t *indptr, const int32_t *indices,
                  const double *data, int32_t value_kind, sc_csr **out);
int sc_csr_info(const sc_csr *A, int32_t *m, int32_t *n, int64_t *nnz, int32_t *value_kind);
/* Borrowed views, valid until sc_csr_free. */
int sc_csr_arrays(const sc_csr *A, const int32_t **indptr, const int32_t **indices,
                  const double **data);
void sc_csr_free(sc_csr *A);

/* ---------------------------------------------------------------- .cfmtx */

/* csr_to_compressed_format_converter + transform_row_panel
 * (code_gen/ss_format/format_generator.py:36-129).  km = row coarsen factor,
 * kn = column pack (0 = 32 // pop).  dictionary_path NULL = enumerate all
 * 2^km-1 patterns (format_generator.py:207-208); otherwise a
 * --pattern_dictionary file (:200-205). */
int sc_cfmtx_build(const sc_csr *A, int32_t km, int32_t kn, const char *dictionary_path,
                   sc_cfmtx **out);
/* format_writer (format_generator.py:132-160), byte-exact. */
int sc_cfmtx_write(const sc_cfmtx *cf, const char *path);
/* readCFMTXFile / readCompressedFormatMatrix (utils/Sparse_io.cpp:84-182, :208-215). */
int sc_cfmtx_read(const char *path, sc_cfmtx **out);
/* loadCfmtxMatrices (utils/Sparse_io.cpp:186-196, include/Sparse_io.h:24):
 * the .cfmtx and its companion .mtx (sym_lib reader).  Path must end in .cfmtx. */
int sc_load_cfmtx_matrices(const char *cfmtx_path, sc_csr **csr, sc_cfmtx **cf);
/* readCSRMatrix (utils/Sparse_io.cpp:198-206): the companion .mtx only. */
int sc_read_csr_matrix(const char *cfmtx_path, sc_csr **csr);
/* companionMtxPathFromCFMTX (utils/Sparse_io.cpp:28-46). */
int sc_companion_mtx_path(const char *cfmtx_path, char *buf, size_t buflen);

/* Header of a .cfmtx: M, K, km, number of patterns, kn (as written), and
 * the number of row panels ceil(M/km). */
int sc_cfmtx_info(const sc_cfmtx *cf, int32_t *m, int32_t *n, int32_t *km, int32_t *npat,
                  int32_t *kn, int32_t *npanels);
/* Pattern i (data-block order): its bit string, printed id and pop, and
 * borrowed views of RPP (npanels+1), CB and the fp32 values (what the
 * reference's CompressedFormat<float> holds: CompressedFormat.h:88-107). */
int sc_cfmtx_pattern(const sc_cfmtx *cf, int32_t i, const char **bits, int32_t *id, int32_t *pop,
                     const int32_t **rpp, int64_t *nrpp, const int32_t **cb, int64_t *ncb,
                     const float **vals, int64_t *nvals);
/* Serialised text of a built .cfmtx (length through *len; buffer may be NULL
 * to query the length). */
int sc_cfmtx_text(const sc_cfmtx *cf, char *buf, int64_t buflen, int64_t *len);
void sc_cfmtx_free(sc_cfmtx *cf);

/* ---------------------------------------------------------------- GPU path */

/* Plan flags */
#define SC_PLAN_DROP_PADDING 1 /* omit the zero-valued padding slots on the device */
#define SC_PLAN_TILED 2        /* also build the split-K LDS-staged copy (opt-in)   */
#define SC_PLAN_CHUNKED 4      /* build the K-block-major copy of the chunk kernel
                                  (B column chunks resident in LDS, N % 32 == 0)   */
#define SC_PLAN_F16_VALUES 8   /* also keep a binary16 copy of the values (sc_spmm_f16) */
#define SC_PLAN_ROWS 16        /* lay the slots out as one-row panels (kernel_m 1):
                                  one workgroup per row instead of per km rows  */
#define SC_PLAN_PATTERNS 32    /* keep only the km-row pattern layout           */
#define SC_PLAN_BANDS 64       /* kernel_m 4 files: also build the band layout (B
                                  staged in LDS once per band of panels and K
                                  range of up to 512 rows, 4-column windows of
                                  each panel on the matrix cores, split K over
                                  the ranges with a plan-owned workspace; the
                                  format's zero padding slots are skipped; K up
                                  to 8192); sc_spmm runs it at N a multiple of
                                  64 up to 256                                 */
/* Without SC_PLAN_ROWS, SC_PLAN_PATTERNS, SC_PLAN_TILED or SC_PLAN_CHUNKED a
 * plan of a kernel_m > 1 file holds both layouts, and sc_spmm / sc_spmv run
 * the one-row layout while its B-row gathers (4 * stored entries * N bytes)
 * total under 128 MiB, the km-row pattern layout above; sc_spmm_f16 follows
 * the same rule when the rows fit its LDS staging.  sc_spmm_generated always
 * runs the pattern layout.
 * Concurrency: a plan holds no launch state unless it was built with
 * SC_PLAN_TILED or SC_PLAN_BANDS, so its launches may run at once on distinct
 * streams.  The split-K kernels of those two flags keep partial sums and
 * arrival counters in the plan's workspace: launches of such a plan must be
 * ordered (one stream, or events between streams). */

/* allocateAndCopyMixedFormat (example_cuda/spmm_demo_gpu_utils.h:207-245) and
 * the constructors of the generated classes SpMMMixePatternGeneralCacheLess /
 * SpMVMixePatternDecomposeByRowSeperated: validate the format, flatten it
 * into panel-major segments and upload it to the current HIP device.
 * Every (panel, pattern) block of slots must use columns < K and hold
 * pop values per slot; out-of-range formats are rejected here, so a kernel
 * never reads outside the plan. */
int sc_plan_create(const sc_cfmtx *cf, int32_t flags, sc_plan **out);
/* Plan geometry: rows, cols, km, panels, device slots and values, segments. */
int sc_plan_info(const sc_plan *plan, int32_t *m, int32_t *n, int32_t *km, int32_t *npanels,
                 int64_t *nslots, int64_t *nvals, int64_t *nsegs);
/* Which kernel sc_spmm runs for this plan and N, and its launch geometry, as
 * text (e.g. "wide_kernel km=4 V=2 stage=1 waves=4 grid=1024").  Diagnostic;
 * no counterpart in the reference. */
int sc_plan_describe(const sc_plan *plan, int32_t N, char *buf, size_t buflen);
/* The pattern kernels: SpMMFullRowPanelGeneralKernel{km}With{kn}BlockCacheLess
 * (example_cuda/spmm_demo_gpu_utils.h:1357-1664, large N) and
 * SpmvComplexPatternDecomposeByRowSeperated (spmm_small_b_col_demo_gpu_utils.h
 * :1061-2986 for small N, spmv_demo_gpu_utils.h:632-904 for N = 1).
 * C = A*B with B row-major K x N and C row-major M x N, both on the plan's
 * device.  C is overwritten (the reference accumulates into a pre-zeroed C;
 * pass SC_ACCUMULATE for C += A*B).  waves_per_panel 0 = automatic. */
#define SC_ACCUMULATE 1
int sc_spmm(const sc_plan *plan, const float *dB, float *dC, int32_t N, int32_t flags,
            int32_t waves_per_panel, void *hip_stream);
/* No counterpart in the reference.  For callers that cannot allocate device
 * memory: code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc.  sc_spmm with the split-K kernels' partial sums and
 * arrival counters (SC_PLAN_BANDS, SC_PLAN_TILED) in the library's static
 * per-device scratch instead of the plan's workspace; allocates nothing.
 * The scratch is 16 MiB of partial sums plus 16 KiB of counters, held on each
 * GPU the library runs on until the process ends; the launches are the ones
 * sc_spmm makes on the same plan (so results equal sc_spmm's), and a launch
 * whose partial sums or counters need more is refused with
 * SC_ERR_UNSUPPORTED (the band kernel at N = 128 on a 4096-row plan with K =
 * 4096 fits).  Every call on one GPU shares that GPU's scratch: calls that
 * overlap on one GPU (other streams, other threads) race. */
int sc_spmm_noalloc(const sc_plan *plan, const float *dB, float *dC, int32_t N, int32_t flags,
                    int32_t waves_per_panel, void *hip_stream);
/* y = A*x (N = 1). */
int sc_spmv(const sc_plan *plan, const float *dx, float *dy, int32_t flags, void *hip_stream);
/* The binary16 small-B path: C = A*B with A's values (the plan's binary16
 * copy: create the plan with SC_PLAN_F16_VALUES), B (K x N) and C (M x N) in
 * IEEE binary16, N = 1, 2 or 4, fp32 accumulation, C rounded once to nearest
 * even.  Replaces the reference's fp16 small-B kernels
 * (SpmvComplexPatternDecomposeByRowSeperatedHalf, PatternWith{pop}NNZByRowPanelFullHALF:
 * example_cuda/spmm_small_b_col_demo_gpu_utils.h:2987-5017, generator
 * code_gen/spmm_small_b_col/spmm_small_b_col_format_code_generator.py:326-435),
 * which accumulate in binary16. */
int sc_spmm_f16(const sc_plan *plan, const void *dB, void *dC, int32_t N, int32_t flags,
                int32_t waves_per_panel, void *hip_stream);
void sc_plan_destroy(sc_plan *plan);

/* ------------------------------------------------------- generated kernels */

/* sc_gen_<name>_launch of a generated unit. */
typedef int (*sc_gen_launch_fn)(const void *view, const float *B, float *C, int N, int accumulate,
                                int waves, void *hip_stream);

/* Parameters a generated kernel unit was emitted with by code_gen/main_spmm.py,
 * main_spmm_small_b_col.py or main_spmv.py (exported as sc_gen_<name>_record).
 * The reference bakes the same parameters into its generated headers
 * (code_gen/spmm/spmm_format_code_generator.py:7-223) but never checks them
 * against the loaded matrix. */
typedef struct sc_gen_record {
  int32_t km;             /* rows per panel                                    */
  int32_t kn;             /* slots per unrolled pack (segments must be multiples) */
  int32_t waves;          /* waves per panel, 0 = chosen at launch             */
  int32_t npatterns;      /* number of pattern bodies                          */
  int32_t variant;        /* 0 = any N, otherwise the only N accepted          */
  const uint32_t *masks;  /* row mask of each body (bit r = panel row r)       */
  /* sc_gen_<name>_launch_rows: the unit's kernel_m 1 body on a plan's one-row
   * layout of the same slots, or NULL */
  sc_gen_launch_fn rows_launch;
} sc_gen_record;

/* Launch a generated unit on a plan after checking that the unit fits it:
 * same km, a pack that divides every segment, a body for every pattern the
 * plan holds and, for fixed-N units, the same N.  A plan that holds the
 * one-row layout too (created without SC_PLAN_PATTERNS) runs under sc_spmm's
 * rule: launches whose one-row B gathers stay under 128 MiB run the unit's
 * kernel_m 1 body (rec->rows_launch) on that layout.  Replaces the launch in
 * the generated classes' execute() (spmm_demo_gpu_utils.h:1700-1720). */
int sc_spmm_generated(const sc_plan *plan, const sc_gen_record *rec, sc_gen_launch_fn launch,
                      const float *dB, float *dC, int32_t N, int32_t flags,
                      int32_t waves_per_panel, void *hip_stream);

#ifdef __cplusplus
}
#endif

#endif /* SC_API_H */
