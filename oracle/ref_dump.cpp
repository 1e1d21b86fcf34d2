// ref_dump.cpp -- test-only driver around the reference's own .cfmtx/.mtx
// loaders, compiled from their sources under /root/reference by
// oracle/Makefile into oracle/_ref/ref_cfmtx_dump.  It is the checker for the
// product's reader, never part of the product.
//
//   ref_cfmtx_dump cfmtx <file.cfmtx>  -> readCompressedFormatMatrix
//                                         (utils/Sparse_io.cpp:208-215)
//   ref_cfmtx_dump csr   <file.cfmtx>  -> readCSRMatrix on the companion .mtx
//                                         (utils/Sparse_io.cpp:198-206)
//
// Output (text): floats as the hex of their bit patterns so nothing is lost.
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>

#include "Sparse_io.h"

static unsigned f2u(float f) {
  unsigned u;
  std::memcpy(&u, &f, 4);
  return u;
}
static unsigned long long d2u(double d) {
  unsigned long long u;
  std::memcpy(&u, &d, 8);
  return u;
}

int main(int argc, char **argv) {
  if (argc != 3) {
    std::fprintf(stderr, "usage: %s cfmtx|csr <path.cfmtx>\n", argv[0]);
    return 2;
  }
  std::string mode = argv[1], path = argv[2];
  using namespace swiftware::compression;
  if (mode == "cfmtx") {
    MixedFormat<float> *mf = readCompressedFormatMatrix(path);
    if (!mf) return 1;
    std::printf("%zu\n", mf->cf.size());
    for (auto *c : mf->cf) {
      std::printf("%zu %zu %zu %zu %zu %zu %zu %zu\n", c->km, c->kn, c->m, c->n, c->pm, c->nrpp,
                  c->nnz, c->CB.size());
      for (size_t j = 0; j < c->nrpp; ++j) std::printf(j ? " %d" : "%d", c->RPP[j]);
      std::printf("\n");
      for (size_t j = 0; j < c->nrpp; ++j) std::printf(j ? " %d" : "%d", c->NPP[j]);
      std::printf("\n");
      for (size_t j = 0; j < c->CB.size(); ++j) std::printf(j ? " %d" : "%d", c->CB[j]);
      std::printf("\n");
      for (size_t j = 0; j < c->nnz; ++j) std::printf(j ? " %08x" : "%08x", f2u(c->NNZ[j]));
      std::printf("\n");
    }
    // MixedFormat's destructor frees an uninitialised Dense pointer
    // (CompressedFormat.h:270-278), so the object is deliberately leaked.
    return 0;
  }
  if (mode == "csr") {
    sym_lib::CSR *A = readCSRMatrix(path);
    if (!A) return 1;
    std::printf("%zu %zu %zu\n", A->m, A->n, A->nnz);
    for (size_t j = 0; j <= A->m; ++j) std::printf(j ? " %d" : "%d", A->p[j]);
    std::printf("\n");
    for (size_t j = 0; j < A->nnz; ++j) std::printf(j ? " %d" : "%d", A->i[j]);
    std::printf("\n");
    for (size_t j = 0; j < A->nnz; ++j) std::printf(j ? " %016llx" : "%016llx", d2u(A->x[j]));
    std::printf("\n");
    return 0;
  }
  return 2;
}
