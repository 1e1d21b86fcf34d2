/*
 * sc_vendor.h -- vendor-library baselines for the pattern kernels
 * (libsc_vendor.so: rocSPARSE and hipBLAS on the same CSR matrix).
 *
 * These are the MI355X counterparts of the baseline rows the reference's
 * demos print next to the pattern kernel: SpMMcuSparse, SpMMcuBlas,
 * SpMMcuBlasGemmX, SpMMcuBlasHalf (example_cuda/spmm_demo_gpu_utils.h
 * :437-940) and the cuSPARSE / cuBLAS SpMV rows
 * (example_cuda/spmv_demo_gpu.cu:104-120).  They are measured, not used by
 * the product path.
 *
 * Layout: B row-major K x N, C row-major M x N, fp32 device buffers, as for
 * sc_spmm.  A handle is bound to one N and to one pair of B/C buffers:
 * sc_vendor_bind does every untimed step (descriptor set-up, rocSPARSE
 * preprocessing, fp16 conversion of B), sc_vendor_run issues only the
 * library call the reference times, sc_vendor_fetch leaves C in dC as fp32
 * (a conversion for the fp16 kind, nothing otherwise).
 */
#ifndef SC_VENDOR_H
#define SC_VENDOR_H

#include <stdint.h>

#include "sc_api.h"

#ifdef __cplusplus
extern "C" {
#endif

/* kinds */
#define SC_VENDOR_ROCSPARSE_SPMM 0   /* rocsparse_spmm, CSR fp32 (SpMMcuSparse :437-549)      */
#define SC_VENDOR_ROCSPARSE_SPMV 1   /* rocsparse_spmv, CSR fp32 (cuSPARSE SpMV row), N = 1   */
#define SC_VENDOR_HIPBLAS_SGEMM 2    /* dense A, hipblasSgemm (SpMMcuBlas :551-679)           */
#define SC_VENDOR_HIPBLAS_GEMMEX 3   /* dense A, hipblasGemmEx fp32 (SpMMcuBlasGemmX :790-941) */
#define SC_VENDOR_HIPBLAS_HALF 4     /* dense A and B in fp16, fp32 compute, fp16 C
                                        (SpMMcuBlasHalf :681-788)                              */

/* rocSPARSE algorithm for the SPMM/SPMV kinds (ignored by the others):
 * 0 = default, 1 = CSR row split (LDS), 2 = CSR row split (shuffles),
 * 3 = CSR nnz split (merge), 4 = CSR merge path.  SPMV: 0 = default,
 * 1 = adaptive, 2 = stream, 3 = LRB. */
typedef struct sc_vendor sc_vendor;

/* Message of the last failed sc_vendor_* call on this thread. */
const char *sc_vendor_last_error(void);

/* Upload A (fp32 values; dense M x K copy for the hipBLAS kinds) to the
 * current device and create the library handle. */
int sc_vendor_create(const sc_csr *A, int32_t kind, int32_t N, int32_t alg, sc_vendor **out);
/* Attach B and C (untimed set-up; see above). */
int sc_vendor_bind(sc_vendor *h, const float *dB, float *dC, void *hip_stream);
/* The library call alone: C = A * B. */
int sc_vendor_run(sc_vendor *h, void *hip_stream);
/* Leave the fp32 result in the bound dC. */
int sc_vendor_fetch(sc_vendor *h, void *hip_stream);
/* Device bytes the handle holds (A copy, workspace, fp16 buffers). */
int64_t sc_vendor_device_bytes(const sc_vendor *h);
void sc_vendor_destroy(sc_vendor *h);

#ifdef __cplusplus
}
#endif

#endif /* SC_VENDOR_H */
