// sc_capi.cpp -- C ABI over the host format code (CSR, .mtx, .cfmtx,
// pattern enumeration, synthetic inputs).  The GPU entry points live in
// sc_plan.hip.
#include <cstring>
#include <memory>

#include "sc_errors.hpp"
#include "sc_format.hpp"
#include "sc_synth.h"

struct sc_csr {
  sc::Csr A;
};
struct sc_cfmtx {
  sc::Cfmtx cf;
};

namespace sc {

static thread_local std::string g_last_error;

void set_last_error(const std::string &msg) { g_last_error = msg; }
void clear_last_error() { g_last_error.clear(); }

static void need(bool ok, const char *what) {
  if (!ok) throw Error{SC_ERR_ARG, what};
}

}  // namespace sc

extern "C" {

const char *sc_last_error(void) { return sc::g_last_error.c_str(); }
int sc_abi_version(void) { return SC_ABI_VERSION; }

int sc_patterns(int32_t km, int32_t kn, char *bits, int64_t bits_len, int32_t *npat) {
  SC_GUARD([&] {
    auto v = sc::enumerate_patterns(km, kn);
    const int64_t stride = (int64_t)km * kn + 1;
    if (npat) *npat = (int32_t)v.size();
    if (bits) {
      sc::need(bits_len >= stride * (int64_t)v.size(), "pattern buffer too small");
      for (size_t i = 0; i < v.size(); ++i) std::memcpy(bits + i * stride, v[i].c_str(), (size_t)stride);
    }
  });
}

int sc_mtx_read(const char *path, int32_t mode, sc_csr **out) {
  SC_GUARD([&] {
    sc::need(path && out, "null argument");
    sc::need(mode == SC_MTX_SCIPY || mode == SC_MTX_SYMLIB, "unknown .mtx reader mode");
    auto p = std::make_unique<sc_csr>();
    p->A = sc::read_mtx(path, (sc::MtxMode)mode);
    *out = p.release();
  });
}

int sc_mtx_write(const sc_csr *A, const char *path) {
  SC_GUARD([&] {
    sc::need(A && path, "null argument");
    sc::write_mtx(A->A, path);
  });
}

int sc_csr_create(int32_t m, int32_t n, const int32_t *indptr, const int32_t *indices,
                  const double *data, int32_t value_kind, sc_csr **out) {
  SC_GUARD([&] {
    sc::need(out && indptr && m >= 0 && n >= 0, "bad CSR arguments");
    sc::need(value_kind >= 0 && value_kind <= 2, "bad value kind");
    auto p = std::make_unique<sc_csr>();
    p->A.m = m;
    p->A.n = n;
    p->A.kind = (sc::ValueKind)value_kind;
    p->A.indptr.assign(indptr, indptr + (size_t)m + 1);
    const int64_t nnz = p->A.indptr.back();
    sc::need(p->A.indptr[0] == 0 && nnz >= 0, "CSR row pointer must start at 0");
    if (nnz) sc::need(indices && data, "null CSR arrays");
    p->A.indices.assign(indices, indices + nnz);
    p->A.data.assign(data, data + nnz);
    *out = p.release();
  });
}

int sc_csr_info(const sc_csr *A, int32_t *m, int32_t *n, int64_t *nnz, int32_t *value_kind) {
  SC_GUARD([&] {
    sc::need(A, "null CSR");
    if (m) *m = A->A.m;
    if (n) *n = A->A.n;
    if (nnz) *nnz = A->A.nnz();
    if (value_kind) *value_kind = A->A.kind;
  });
}

int sc_csr_arrays(const sc_csr *A, const int32_t **indptr, const int32_t **indices,
                  const double **data) {
  SC_GUARD([&] {
    sc::need(A, "null CSR");
    if (indptr) *indptr = A->A.indptr.data();
    if (indices) *indices = A->A.indices.data();
    if (data) *data = A->A.data.data();
  });
}

void sc_csr_free(sc_csr *A) { delete A; }

int sc_cfmtx_build(const sc_csr *A, int32_t km, int32_t kn, const char *dictionary_path,
                   sc_cfmtx **out) {
  SC_GUARD([&] {
    sc::need(A && out, "null argument");
    auto p = std::make_unique<sc_cfmtx>();
    if (dictionary_path) {
      auto dict = sc::read_pattern_dictionary(dictionary_path);
      p->cf = sc::build_cfmtx(A->A, km, kn, &dict);
    } else {
      p->cf = sc::build_cfmtx(A->A, km, kn, nullptr);
    }
    *out = p.release();
  });
}

int sc_cfmtx_write(const sc_cfmtx *cf, const char *path) {
  SC_GUARD([&] {
    sc::need(cf && path, "null argument");
    sc::write_cfmtx(cf->cf, path);
  });
}

int sc_cfmtx_text(const sc_cfmtx *cf, char *buf, int64_t buflen, int64_t *len) {
  SC_GUARD([&] {
    sc::need(cf, "null argument");
    std::string s = sc::cfmtx_text(cf->cf);
    if (len) *len = (int64_t)s.size();
    if (buf) {
      sc::need(buflen >= (int64_t)s.size(), "text buffer too small");
      std::memcpy(buf, s.data(), s.size());
    }
  });
}

static bool ends_with(const std::string &s, const std::string &suf) {
  return s.size() >= suf.size() && s.compare(s.size() - suf.size(), suf.size(), suf) == 0;
}

int sc_cfmtx_read(const char *path, sc_cfmtx **out) {
  SC_GUARD([&] {
    sc::need(path && out, "null argument");
    auto p = std::make_unique<sc_cfmtx>();
    p->cf = sc::read_cfmtx(path);
    *out = p.release();
  });
}

int sc_load_cfmtx_matrices(const char *cfmtx_path, sc_csr **csr, sc_cfmtx **cf) {
  SC_GUARD([&] {
    sc::need(cfmtx_path && csr && cf, "null argument");
    std::string path = cfmtx_path;
    if (!ends_with(path, ".cfmtx"))
      throw sc::Error{SC_ERR_ARG, "loadCfmtxMatrices expects a .cfmtx path: " + path};
    auto c = std::make_unique<sc_cfmtx>();
    c->cf = sc::read_cfmtx(path);
    auto a = std::make_unique<sc_csr>();
    a->A = sc::read_mtx(sc::companion_mtx_path(path), sc::MTX_SYMLIB);
    *cf = c.release();
    *csr = a.release();
  });
}

int sc_read_csr_matrix(const char *cfmtx_path, sc_csr **csr) {
  SC_GUARD([&] {
    sc::need(cfmtx_path && csr, "null argument");
    std::string path = cfmtx_path;
    if (!ends_with(path, ".cfmtx"))
      throw sc::Error{SC_ERR_ARG, "readCSRMatrix expects a .cfmtx path: " + path};
    auto a = std::make_unique<sc_csr>();
    a->A = sc::read_mtx(sc::companion_mtx_path(path), sc::MTX_SYMLIB);
    *csr = a.release();
  });
}

int sc_companion_mtx_path(const char *cfmtx_path, char *buf, size_t buflen) {
  SC_GUARD([&] {
    sc::need(cfmtx_path && buf, "null argument");
    std::string s = sc::companion_mtx_path(cfmtx_path);
    sc::need(buflen > s.size(), "path buffer too small");
    std::memcpy(buf, s.c_str(), s.size() + 1);
  });
}

int sc_cfmtx_info(const sc_cfmtx *cf, int32_t *m, int32_t *n, int32_t *km, int32_t *npat,
                  int32_t *kn, int32_t *npanels) {
  SC_GUARD([&] {
    sc::need(cf, "null argument");
    if (m) *m = cf->cf.m;
    if (n) *n = cf->cf.n;
    if (km) *km = cf->cf.km;
    if (npat) *npat = (int32_t)cf->cf.patterns.size();
    if (kn) *kn = cf->cf.kn;
    if (npanels) *npanels = cf->cf.npanels();
  });
}

int sc_cfmtx_pattern(const sc_cfmtx *cf, int32_t i, const char **bits, int32_t *id, int32_t *pop,
                     const int32_t **rpp, int64_t *nrpp, const int32_t **cb, int64_t *ncb,
                     const float **vals, int64_t *nvals) {
  SC_GUARD([&] {
    sc::need(cf && i >= 0 && i < (int32_t)cf->cf.patterns.size(), "pattern index out of range");
    const sc::Pattern &p = cf->cf.patterns[(size_t)i];
    if (bits) *bits = p.bits.c_str();
    if (id) *id = p.id;
    if (pop) *pop = p.pop;
    if (rpp) *rpp = p.rpp.data();
    if (nrpp) *nrpp = (int64_t)p.rpp.size();
    if (cb) *cb = p.cb.data();
    if (ncb) *ncb = (int64_t)p.cb.size();
    if (vals) *vals = p.val32.data();
    if (nvals) *nvals = (int64_t)p.val32.size();
  });
}

void sc_cfmtx_free(sc_cfmtx *cf) { delete cf; }

int sc_synth_uniform(int32_t m, int32_t n, double density, double sigma, uint64_t seed,
                     sc_csr **out) {
  SC_GUARD([&] {
    sc::need(out, "null argument");
    auto p = std::make_unique<sc_csr>();
    p->A = sc::synth_uniform(m, n, density, sigma, seed);
    *out = p.release();
  });
}

int sc_synth_blocks(int32_t m, int32_t n, double density, double sigma, uint64_t seed,
                    sc_csr **out) {
  SC_GUARD([&] {
    sc::need(out, "null argument");
    auto p = std::make_unique<sc_csr>();
    p->A = sc::synth_blocks(m, n, density, sigma, seed);
    *out = p.release();
  });
}

int sc_synth_dense(float *out, int64_t count, uint64_t seed) {
  SC_GUARD([&] {
    sc::need(out || count == 0, "null argument");
    sc::synth_dense(out, count, seed);
  });
}

int sc_synth_raw(uint64_t seed, uint64_t *out, int64_t count) {
  SC_GUARD([&] {
    sc::need(out || count == 0, "null argument");
    sc::Rng r(seed);
    for (int64_t k = 0; k < count; ++k) out[k] = r.next();
  });
}

}  // extern "C"

// Accessor for sc_plan.hip (same library): the format behind an opaque handle.
const sc::Cfmtx &sc_cfmtx_ref(const sc_cfmtx *cf) { return cf->cf; }
