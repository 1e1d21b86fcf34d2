// sc_format.cpp -- .mtx reader/writer, pattern enumeration, .cfmtx
// builder/writer/reader and the seeded synthetic inputs (host C++).
//
// Reference behaviour each function reproduces is cited on it.  The builder
// is not the reference's loop: it scatters each row panel's columns into
// occupancy masks and sorts the touched columns, which yields the same slots
// in the same order (columns ascending per pattern, values in ascending panel
// row order) in O(nnz + slots log slots).
#include "sc_format.hpp"

#include <algorithm>
#include <cerrno>
#include <charconv>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <map>
#include <sstream>

#include "sc_errors.hpp"

namespace sc {

// ---------------------------------------------------------------------------
// small text helpers
// ---------------------------------------------------------------------------

static void append_int(std::string &s, int64_t v) {
  char buf[24];
  auto r = std::to_chars(buf, buf + sizeof buf, v);
  s.append(buf, r.ptr);
}

// Python's repr(float) ('r' format of PyOS_double_to_string): shortest
// round-trip digits; positional when -4 < decpt <= 16, otherwise
// d[.ddd]e{+|-}XX with at least two exponent digits; ".0" appended to
// integral positional values.  numpy's str(np.float64) prints the same text,
// which is what format_generator.py:155-157 writes for real-valued .mtx.
std::string py_repr(double x) {
  if (std::isnan(x)) return "nan";
  if (std::isinf(x)) return x > 0 ? "inf" : "-inf";
  if (x == 0.0) return std::signbit(x) ? "-0.0" : "0.0";
  char buf[64];
  auto r = std::to_chars(buf, buf + sizeof buf, x, std::chars_format::scientific);
  const char *p = buf;
  bool neg = false;
  if (*p == '-') {
    neg = true;
    ++p;
  }
  std::string digits;
  while (p < r.ptr && *p != 'e') {
    if (*p != '.') digits.push_back(*p);
    ++p;
  }
  int exp10 = 0;
  std::from_chars(p + 1 + (p[1] == '+'), r.ptr, exp10);
  while (digits.size() > 1 && digits.back() == '0') digits.pop_back();
  const int nd = (int)digits.size();
  const int decpt = exp10 + 1;  // value = 0.d1d2... * 10^decpt
  std::string out;
  if (neg) out.push_back('-');
  if (decpt > -4 && decpt <= 16) {
    if (decpt <= 0) {
      out += "0.";
      out.append((size_t)(-decpt), '0');
      out += digits;
    } else if (decpt >= nd) {
      out += digits;
      out.append((size_t)(decpt - nd), '0');
      out += ".0";
    } else {
      out.append(digits, 0, (size_t)decpt);
      out.push_back('.');
      out.append(digits, (size_t)decpt, std::string::npos);
    }
  } else {
    out.push_back(digits[0]);
    if (nd > 1) {
      out.push_back('.');
      out.append(digits, 1, std::string::npos);
    }
    int e = decpt - 1;
    out.push_back('e');
    out.push_back(e < 0 ? '-' : '+');
    int ae = e < 0 ? -e : e;
    if (ae < 10) out.push_back('0');
    append_int(out, ae);
  }
  return out;
}

float reader_f32(double x) {
  float f = (float)x;
  if ((double)f == x || !std::isfinite(x)) return f;
  // strtof straight from the decimal text, as `iss >> float` does on the
  // written token (utils/Sparse_io.cpp:144-150); differs from (float)x only
  // when x sits next to a float rounding midpoint.
  std::string t = py_repr(x);
  return std::strtof(t.c_str(), nullptr);
}

// ---------------------------------------------------------------------------
// pattern enumeration
// ---------------------------------------------------------------------------

// generate_pattern_dictionary / build_patterns_map
// (code_gen/pattern_utiles/pattern_dictionary.py:29-46): id i-1 <-> the
// zero-filled binary text of 2^bits - i.  Equivalently the bit string of id is
// the binary text of (2^bits - 1 - id).
std::vector<std::string> enumerate_patterns(int km, int kn) {
  const int bits = km * kn;
  if (km <= 0 || kn <= 0 || bits > 20) throw Error{SC_ERR_ARG, "pattern width out of range (1..20 bits)"};
  const uint32_t top = (1u << bits) - 1;
  std::vector<std::string> out(top);
  for (uint32_t id = 0; id < top; ++id) {
    uint32_t x = top - id;
    std::string s((size_t)bits, '0');
    for (int c = 0; c < bits; ++c)
      if ((x >> (bits - 1 - c)) & 1) s[(size_t)c] = '1';
    out[id] = std::move(s);
  }
  return out;
}

// read_pattern_dictionary (pattern_dictionary.py:49-60) followed by the
// tuple-keyed dict of format_generator.py:200-205.  Python dict semantics are
// kept: a repeated id keeps its first position and takes the last bit string.
std::vector<std::pair<std::string, int32_t>> read_pattern_dictionary(const std::string &path) {
  std::ifstream in(path);
  if (!in) throw Error{SC_ERR_IO, "cannot open pattern dictionary " + path};
  std::string line;
  if (!std::getline(in, line)) throw Error{SC_ERR_FORMAT, "empty pattern dictionary " + path};
  {
    std::istringstream h(line);
    std::string a, b, c;
    if (!(h >> a >> b >> c)) throw Error{SC_ERR_FORMAT, "pattern dictionary header needs 'm n count'"};
  }
  std::vector<std::pair<std::string, int32_t>> order;
  std::map<int32_t, size_t> pos;
  while (std::getline(in, line)) {
    std::istringstream ls(line);
    std::string bits, key, extra;
    if (!(ls >> bits >> key) || (ls >> extra))
      throw Error{SC_ERR_FORMAT, "pattern dictionary line is not '<bits> <id>': " + line};
    char *end = nullptr;
    long id = std::strtol(key.c_str(), &end, 10);
    if (*end) throw Error{SC_ERR_FORMAT, "pattern id is not an integer: " + key};
    std::string norm(bits.size(), '0');
    for (size_t c = 0; c < bits.size(); ++c) norm[c] = bits[c] == '1' ? '1' : '0';
    auto it = pos.find((int32_t)id);
    if (it == pos.end()) {
      pos[(int32_t)id] = order.size();
      order.emplace_back(norm, (int32_t)id);
    } else {
      order[it->second].first = norm;
    }
  }
  // second dict, keyed by the bool tuple
  std::vector<std::pair<std::string, int32_t>> out;
  std::map<std::string, size_t> kpos;
  for (auto &e : order) {
    auto it = kpos.find(e.first);
    if (it == kpos.end()) {
      kpos[e.first] = out.size();
      out.push_back(e);
    } else {
      out[it->second].second = e.second;
    }
  }
  return out;
}

// ---------------------------------------------------------------------------
// .mtx
// ---------------------------------------------------------------------------

namespace {

std::string lower(std::string s) {
  for (auto &c : s) c = (char)std::tolower((unsigned char)c);
  return s;
}

struct Triplet {
  int32_t r, c;
  double v;
};

Csr triplets_to_csr(int32_t m, int32_t n, std::vector<Triplet> &t, bool sum_duplicates) {
  std::stable_sort(t.begin(), t.end(), [](const Triplet &a, const Triplet &b) {
    return a.r < b.r || (a.r == b.r && a.c < b.c);
  });
  Csr A;
  A.m = m;
  A.n = n;
  A.indptr.assign((size_t)m + 1, 0);
  for (size_t k = 0; k < t.size(); ++k) {
    if (sum_duplicates && !A.indices.empty() && k > 0 && t[k].r == t[k - 1].r && t[k].c == t[k - 1].c) {
      A.data.back() += t[k].v;
      continue;
    }
    A.indices.push_back(t[k].c);
    A.data.push_back(t[k].v);
    A.indptr[(size_t)t[k].r + 1]++;
  }
  for (int32_t i = 0; i < m; ++i) A.indptr[(size_t)i + 1] += A.indptr[(size_t)i];
  return A;
}

}  // namespace

// MTX_SCIPY reproduces scipy.io.mmread(path).tocsr() as called by
// format_generator.py:214-215: coordinate real/integer/pattern fields,
// general/symmetric/skew-symmetric expanded to full, duplicates summed,
// explicit zeros kept, columns sorted.
// MTX_SYMLIB reproduces readCSRMatrixFromMTX (utils/Sparse_io.cpp:48-82):
// sym_lib::read_header, read_triplets_real, compress_triplets_to_csc,
// make_full for symmetric, csc_to_csr (aggregation/utils/sparse_io.cpp:278-402,
// sparse_utilities.cpp:58-96, 229-268): duplicates kept.
Csr read_mtx(const std::string &path, MtxMode mode) {
  std::ifstream in(path);
  if (!in) throw Error{SC_ERR_IO, "cannot open " + path};
  std::string line;
  if (!std::getline(in, line)) throw Error{SC_ERR_FORMAT, "empty .mtx file " + path};
  std::istringstream hs(lower(line));
  std::string banner, mtx, crd, arith, sym;
  if (!(hs >> banner >> mtx >> crd >> arith >> sym))
    throw Error{SC_ERR_FORMAT, "first line does not contain 5 tokens"};
  if (banner != "%%matrixmarket") throw Error{SC_ERR_FORMAT, "first token is not %%MatrixMarket"};
  if (mtx != "matrix") throw Error{SC_ERR_FORMAT, "not a matrix"};
  if (crd != "coordinate") throw Error{SC_ERR_UNSUPPORTED, "only coordinate .mtx files are supported (got " + crd + ")"};
  ValueKind kind;
  if (arith == "real" || arith == "double")
    kind = VALUES_REAL;
  else if (arith == "integer")
    kind = VALUES_INTEGER;
  else if (arith == "pattern")
    kind = VALUES_PATTERN;
  else
    throw Error{SC_ERR_UNSUPPORTED, "unsupported .mtx field " + arith};
  int symmetry;  // 0 general, 1 symmetric, -1 skew
  if (sym == "general")
    symmetry = 0;
  else if (sym == "symmetric")
    symmetry = 1;
  else if (sym == "skew-symmetric" && mode == MTX_SCIPY)
    symmetry = -1;
  else
    throw Error{SC_ERR_UNSUPPORTED, "unsupported .mtx symmetry " + sym};
  // comments (and, for the scipy reader, blank lines)
  while (std::getline(in, line)) {
    if (!line.empty() && line[0] == '%') continue;
    if (mode == MTX_SCIPY && line.find_first_not_of(" \t\r") == std::string::npos) continue;
    break;
  }
  std::istringstream ds(line);
  long long m, n, nnz;
  if (!(ds >> m >> n >> nnz)) throw Error{SC_ERR_FORMAT, "the matrix dimension is missing"};
  if (m < 0 || n < 0 || nnz < 0 || m > INT32_MAX - 1 || n > INT32_MAX - 1 || nnz > INT32_MAX)
    throw Error{SC_ERR_FORMAT, "matrix dimensions out of range"};
  std::vector<Triplet> t;
  t.reserve((size_t)nnz * (symmetry ? 2 : 1));
  // Entries are whitespace-separated numbers; parse with strtod/strtoll on
  // the whole remaining text (fast, and equal to `>>` for well-formed files).
  std::string rest((std::istreambuf_iterator<char>(in)), std::istreambuf_iterator<char>());
  const char *p = rest.c_str();
  auto next_tok = [&](const char *&q) {
    while (*q == ' ' || *q == '\t' || *q == '\n' || *q == '\r') ++q;
    return q;
  };
  for (long long k = 0; k < nnz; ++k) {
    char *e;
    next_tok(p);
    long long r = std::strtoll(p, &e, 10);
    if (e == p) throw Error{SC_ERR_FORMAT, "truncated .mtx entry list"};
    p = e;
    next_tok(p);
    long long c = std::strtoll(p, &e, 10);
    if (e == p) throw Error{SC_ERR_FORMAT, "truncated .mtx entry list"};
    p = e;
    double v = 1.0;
    if (kind != VALUES_PATTERN) {
      next_tok(p);
      if (kind == VALUES_INTEGER && mode == MTX_SCIPY) {
        long long iv = std::strtoll(p, &e, 10);
        v = (double)iv;
      } else {
        v = std::strtod(p, &e);
      }
      if (e == p) throw Error{SC_ERR_FORMAT, "missing .mtx value"};
      p = e;
    }
    if (r < 1 || r > m || c < 1 || c > n) throw Error{SC_ERR_FORMAT, ".mtx entry index out of range"};
    int32_t ri = (int32_t)(r - 1), ci = (int32_t)(c - 1);
    t.push_back({ri, ci, v});
    if (symmetry != 0 && ri != ci) t.push_back({ci, ri, symmetry < 0 ? -v : v});
  }
  Csr A = triplets_to_csr((int32_t)m, (int32_t)n, t, mode == MTX_SCIPY);
  A.kind = (mode == MTX_SCIPY) ? kind : VALUES_REAL;
  return A;
}

void write_mtx(const Csr &A, const std::string &path) {
  std::string s;
  s.reserve((size_t)A.nnz() * 28 + 128);
  s += "%%MatrixMarket matrix coordinate ";
  s += A.kind == VALUES_INTEGER ? "integer" : A.kind == VALUES_PATTERN ? "pattern" : "real";
  s += " general\n";
  append_int(s, A.m);
  s.push_back(' ');
  append_int(s, A.n);
  s.push_back(' ');
  append_int(s, A.nnz());
  s.push_back('\n');
  for (int32_t i = 0; i < A.m; ++i)
    for (int32_t j = A.indptr[(size_t)i]; j < A.indptr[(size_t)i + 1]; ++j) {
      append_int(s, i + 1);
      s.push_back(' ');
      append_int(s, A.indices[(size_t)j] + 1);
      if (A.kind == VALUES_INTEGER) {
        s.push_back(' ');
        append_int(s, (int64_t)A.data[(size_t)j]);
      } else if (A.kind == VALUES_REAL) {
        s.push_back(' ');
        s += py_repr(A.data[(size_t)j]);
      }
      s.push_back('\n');
    }
  FILE *f = std::fopen(path.c_str(), "wb");
  if (!f) throw Error{SC_ERR_IO, "cannot write " + path};
  size_t w = std::fwrite(s.data(), 1, s.size(), f);
  std::fclose(f);
  if (w != s.size()) throw Error{SC_ERR_IO, "short write to " + path};
}

// ---------------------------------------------------------------------------
// .cfmtx builder
// ---------------------------------------------------------------------------

static void check_canonical(const Csr &A) {
  if ((int64_t)A.indptr.size() != (int64_t)A.m + 1 || A.indptr[0] != 0)
    throw Error{SC_ERR_ARG, "CSR row pointer has the wrong length or does not start at 0"};
  for (int32_t i = 0; i < A.m; ++i) {
    int32_t a = A.indptr[(size_t)i], b = A.indptr[(size_t)i + 1];
    if (b < a || b > (int32_t)A.indices.size()) throw Error{SC_ERR_ARG, "CSR row pointer is not monotone"};
    for (int32_t j = a; j < b; ++j) {
      int32_t c = A.indices[(size_t)j];
      if (c < 0 || c >= A.n) throw Error{SC_ERR_ARG, "CSR column index out of range"};
      if (j > a && c <= A.indices[(size_t)j - 1])
        throw Error{SC_ERR_ARG, "CSR columns must be sorted and unique within a row"};
    }
  }
  if (A.data.size() != A.indices.size()) throw Error{SC_ERR_ARG, "CSR data and indices differ in length"};
}

// csr_to_compressed_format_converter + transform_row_panel
// (code_gen/ss_format/format_generator.py:36-129).  Per row panel of km rows
// every column with a stored entry becomes one slot of the pattern given by
// the set of panel rows holding it; slots of a (panel, pattern) segment keep
// increasing column order, values ascending panel-row order.  Each segment is
// padded to a multiple of `pack` slots (pack = kn, or 32 // pop when kn == 0)
// with value 0 and the segment's largest column.  Slots whose pattern is not
// in the dictionary are dropped (format_generator.py:112-120).
Cfmtx build_cfmtx(const Csr &A, int km, int kn,
                  const std::vector<std::pair<std::string, int32_t>> *dictionary) {
  if (km < 1 || km > 20) throw Error{SC_ERR_ARG, "kernel_m must be in 1..20"};
  if (kn < 0) throw Error{SC_ERR_ARG, "kernel_n must be >= 0"};
  check_canonical(A);
  std::vector<std::pair<std::string, int32_t>> entries;
  if (dictionary) {
    entries = *dictionary;
  } else {
    auto bits = enumerate_patterns(km, 1);
    for (size_t id = 0; id < bits.size(); ++id) entries.emplace_back(bits[id], (int32_t)id);
  }
  const int32_t P = (int32_t)entries.size();
  if (P == 0) throw Error{SC_ERR_ARG, "empty pattern dictionary"};
  Cfmtx cf;
  cf.m = A.m;
  cf.n = A.n;
  cf.km = km;
  cf.kn = kn;
  cf.kind = A.kind;
  cf.has_exact = true;
  cf.patterns.resize((size_t)P);
  std::vector<uint8_t> seen((size_t)P, 0);
  std::vector<int32_t> mask_to_id((size_t)1 << km, -1);
  for (auto &e : entries) {
    if (e.second < 0 || e.second >= P || seen[(size_t)e.second])
      throw Error{SC_ERR_ARG, "pattern ids must be distinct and in 0..count-1"};
    seen[(size_t)e.second] = 1;
    Pattern &pt = cf.patterns[(size_t)e.second];
    pt.bits = e.first;
    pt.id = e.second;
    pt.pop = (int32_t)std::count(e.first.begin(), e.first.end(), '1');
    if (pt.pop == 0) throw Error{SC_ERR_ARG, "a pattern with no ones cannot be packed"};
    if ((int)e.first.size() == km) {
      uint32_t mask = 0;
      for (int r = 0; r < km; ++r)
        if (e.first[(size_t)r] == '1') mask |= 1u << r;
      mask_to_id[mask] = e.second;
    }
    pt.rpp.assign(1, 0);
  }
  cf.header_order.clear();
  for (auto &e : entries) cf.header_order.push_back(e.second);

  const int32_t npanels = cf.npanels();
  std::vector<int32_t> stamp((size_t)A.n, -1);
  std::vector<uint32_t> colmask((size_t)A.n, 0);
  std::vector<int32_t> touched;
  std::vector<int32_t> cursor((size_t)km);
  std::vector<std::vector<int32_t>> seg_cols((size_t)P);
  std::vector<std::vector<double>> seg_vals((size_t)P);
  for (int32_t p = 0; p < npanels; ++p) {
    const int32_t r0 = p * km;
    const int32_t nr = std::min(km, A.m - r0);
    touched.clear();
    for (int32_t r = 0; r < nr; ++r) {
      for (int32_t j = A.indptr[(size_t)(r0 + r)]; j < A.indptr[(size_t)(r0 + r) + 1]; ++j) {
        int32_t c = A.indices[(size_t)j];
        if (stamp[(size_t)c] != p) {
          stamp[(size_t)c] = p;
          colmask[(size_t)c] = 0;
          touched.push_back(c);
        }
        colmask[(size_t)c] |= 1u << r;
      }
      cursor[(size_t)r] = A.indptr[(size_t)(r0 + r)];
    }
    std::sort(touched.begin(), touched.end());
    for (auto &v : seg_cols) v.clear();
    for (auto &v : seg_vals) v.clear();
    for (int32_t c : touched) {
      uint32_t mask = colmask[(size_t)c];
      int32_t id = mask_to_id[mask];
      for (int32_t r = 0; r < nr; ++r) {
        if (!((mask >> r) & 1)) continue;
        if (id >= 0) seg_vals[(size_t)id].push_back(A.data[(size_t)cursor[(size_t)r]]);
        cursor[(size_t)r]++;
      }
      if (id >= 0) seg_cols[(size_t)id].push_back(c);
    }
    for (int32_t id = 0; id < P; ++id) {
      Pattern &pt = cf.patterns[(size_t)id];
      auto &sc = seg_cols[(size_t)id];
      auto &sv = seg_vals[(size_t)id];
      const int64_t pack = kn ? kn : 32 / pt.pop;
      if (pack == 0) throw Error{SC_ERR_ARG, "pattern wider than 32 rows cannot be packed with kernel_n 0"};
      const int64_t ns = (int64_t)sc.size();
      const int64_t padded = ns == 0 ? 0 : (ns + pack - 1) / pack * pack;
      for (double v : sv) {
        pt.val64.push_back(v);
        pt.pad.push_back(0);
      }
      for (int64_t q = ns * pt.pop; q < padded * pt.pop; ++q) {
        pt.val64.push_back(0.0);
        pt.pad.push_back(1);
      }
      for (int32_t c : sc) pt.cb.push_back(c);
      if (ns) {
        int32_t cmax = *std::max_element(sc.begin(), sc.end());
        for (int64_t q = ns; q < padded; ++q) pt.cb.push_back(cmax);
      }
      if ((int64_t)pt.cb.size() > INT32_MAX) throw Error{SC_ERR_ARG, "too many slots for int32 pointers"};
      pt.rpp.push_back((int32_t)pt.cb.size());
    }
  }
  for (auto &pt : cf.patterns) {
    pt.val32.resize(pt.val64.size());
    for (size_t q = 0; q < pt.val64.size(); ++q) pt.val32[q] = pt.pad[q] ? 0.0f : reader_f32(pt.val64[q]);
  }
  return cf;
}

// format_writer (format_generator.py:132-160): header, pattern lines with a
// trailing space in dictionary order, then RPP / CB / values per pattern id.
std::string cfmtx_text(const Cfmtx &cf) {
  std::string s;
  size_t est = 256;
  for (auto &pt : cf.patterns) est += pt.cb.size() * 8 + pt.val32.size() * 24 + pt.rpp.size() * 8;
  s.reserve(est);
  append_int(s, cf.m);
  s.push_back(' ');
  append_int(s, cf.n);
  s.push_back(' ');
  append_int(s, cf.km);
  s.push_back(' ');
  append_int(s, (int64_t)cf.patterns.size());
  s.push_back(' ');
  append_int(s, cf.kn);
  s.push_back('\n');
  for (int32_t idx : cf.header_order) {
    const Pattern &pt = cf.patterns[(size_t)idx];
    s += pt.bits;
    s.push_back(' ');
    append_int(s, pt.id);
    s += " \n";
  }
  for (const Pattern &pt : cf.patterns) {
    for (size_t j = 0; j < pt.rpp.size(); ++j) {
      if (j) s.push_back(' ');
      append_int(s, pt.rpp[j]);
    }
    s.push_back('\n');
    for (size_t j = 0; j < pt.cb.size(); ++j) {
      if (j) s.push_back(' ');
      append_int(s, pt.cb[j]);
    }
    s.push_back('\n');
    for (size_t j = 0; j < pt.val32.size(); ++j) {
      if (j) s.push_back(' ');
      if (cf.has_exact && pt.pad[j]) {
        s.push_back('0');
      } else if (cf.has_exact) {
        // integer and pattern fields print as floats too: the reference
        // stacks its float64 padding rows onto the CSR first
        // (format_generator.py:80-81), which upcasts the values
        s += py_repr(pt.val64[j]);
      } else {
        s += py_repr((double)pt.val32[j]);
      }
    }
    s.push_back('\n');
  }
  return s;
}

void write_cfmtx(const Cfmtx &cf, const std::string &path) {
  std::string s = cfmtx_text(cf);
  FILE *f = std::fopen(path.c_str(), "wb");
  if (!f) throw Error{SC_ERR_IO, "cannot write " + path};
  size_t w = std::fwrite(s.data(), 1, s.size(), f);
  std::fclose(f);
  if (w != s.size()) throw Error{SC_ERR_IO, "short write to " + path};
}

// ---------------------------------------------------------------------------
// .cfmtx reader
// ---------------------------------------------------------------------------

namespace {

// `iss >> int` / `iss >> float` on one line: values are taken while the
// stream extraction would succeed; the first token it would reject (or an
// out-of-range one) ends the line, as the reference's while loops do.
const char *skip_ws(const char *p) {
  while (*p == ' ' || *p == '\t' || *p == '\r' || *p == '\v' || *p == '\f') ++p;
  return p;
}

bool next_int(const char *&p, int32_t &out) {
  p = skip_ws(p);
  const char *q = p;
  if (*q == '+' || *q == '-') ++q;
  if (!std::isdigit((unsigned char)*q)) return false;
  while (std::isdigit((unsigned char)*q)) ++q;
  std::string tok(p, q);
  errno = 0;
  long long v = std::strtoll(tok.c_str(), nullptr, 10);
  if (errno == ERANGE || v > INT32_MAX || v < INT32_MIN) return false;
  out = (int32_t)v;
  p = q;
  return true;
}

bool next_float(const char *&p, float &out) {
  p = skip_ws(p);
  const char *q = p;
  if (*q == '+' || *q == '-') ++q;
  bool digits = false;
  while (std::isdigit((unsigned char)*q)) {
    ++q;
    digits = true;
  }
  if (*q == '.') {
    ++q;
    while (std::isdigit((unsigned char)*q)) {
      ++q;
      digits = true;
    }
  }
  if (!digits) return false;
  if (*q == 'e' || *q == 'E') {
    const char *e = q + 1;
    if (*e == '+' || *e == '-') ++e;
    if (std::isdigit((unsigned char)*e)) {
      while (std::isdigit((unsigned char)*e)) ++e;
      q = e;
    } else {
      return false;  // num_get consumes "1e" and then fails the conversion
    }
  }
  std::string tok(p, q);
  float v = std::strtof(tok.c_str(), nullptr);
  if (std::isinf(v)) return false;
  out = v;
  p = q;
  return true;
}

}  // namespace

// readCFMTXFile (utils/Sparse_io.cpp:84-182): header "rows cols km P kn",
// P pattern lines (pop = number of '1' characters of the i-th line, paired
// with the i-th data block), then per pattern an RPP line (NPP = RPP * pop),
// a CB line and the values read as fp32.  RPP lines longer than
// ceil(M/km)+1 entries are rejected (the reference writes past its array).
Cfmtx read_cfmtx(const std::string &path) {
  std::ifstream in(path);
  if (!in.is_open()) throw Error{SC_ERR_IO, "Unable to open file " + path};
  std::string line;
  int32_t hdr[5] = {0, 0, 0, 0, 0};
  if (std::getline(in, line)) {
    const char *p = line.c_str();
    for (int k = 0; k < 5; ++k)
      if (!next_int(p, hdr[k])) throw Error{SC_ERR_FORMAT, "bad .cfmtx header line: " + line};
  } else {
    throw Error{SC_ERR_FORMAT, "empty .cfmtx file " + path};
  }
  Cfmtx cf;
  cf.m = hdr[0];
  cf.n = hdr[1];
  cf.km = hdr[2];
  cf.kn = hdr[4];
  cf.has_exact = false;
  const int32_t P = hdr[3];
  if (cf.m < 0 || cf.n < 0 || cf.km <= 0 || P <= 0 || P > (1 << 20))
    throw Error{SC_ERR_FORMAT, "bad .cfmtx header values"};
  const int64_t nrpp = cf.npanels() + 1;
  cf.patterns.resize((size_t)P);
  for (int32_t i = 0; i < P; ++i) {
    Pattern &pt = cf.patterns[(size_t)i];
    if (!std::getline(in, line)) throw Error{SC_ERR_FORMAT, "missing pattern line"};
    std::istringstream ls(line);
    std::string bits;
    int32_t id = 0;
    ls >> bits >> id;
    pt.bits = bits;
    pt.id = id;
    pt.pop = (int32_t)std::count(bits.begin(), bits.end(), '1');
    cf.header_order.push_back(i);
  }
  for (int32_t i = 0; i < P; ++i) {
    Pattern &pt = cf.patterns[(size_t)i];
    pt.rpp.assign((size_t)nrpp, 0);
    if (std::getline(in, line)) {
      const char *p = line.c_str();
      int32_t v;
      int64_t k = 0;
      while (next_int(p, v)) {
        if (k >= nrpp) throw Error{SC_ERR_FORMAT, "row-panel pointer line longer than ceil(rows/km)+1"};
        pt.rpp[(size_t)k++] = v;
      }
    }
    if (std::getline(in, line)) {
      const char *p = line.c_str();
      int32_t v;
      while (next_int(p, v)) pt.cb.push_back(v);
    }
    if (std::getline(in, line)) {
      const char *p = line.c_str();
      float v;
      while (next_float(p, v)) pt.val32.push_back(v);
    }
  }
  return cf;
}

// companionMtxPathFromCFMTX (utils/Sparse_io.cpp:28-46):
// "<stem>-<a>-<b>.cfmtx" -> "<stem>.mtx".
std::string companion_mtx_path(const std::string &cfmtx_path) {
  const size_t suffix = 6;  // ".cfmtx"
  if (cfmtx_path.size() <= suffix) return cfmtx_path;
  std::string stem = cfmtx_path.substr(0, cfmtx_path.size() - suffix);
  const size_t last = stem.rfind('-');
  if (last == std::string::npos || last == 0) return stem + ".mtx";
  const size_t second = stem.rfind('-', last - 1);
  if (second == std::string::npos) return stem + ".mtx";
  stem.resize(second);
  return stem + ".mtx";
}

// ---------------------------------------------------------------------------
// synthetic inputs
// ---------------------------------------------------------------------------

static inline uint64_t rotl(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }

// xoshiro256** (Blackman & Vigna) seeded through splitmix64 (Vigna).
Rng::Rng(uint64_t seed) {
  uint64_t x = seed;
  for (auto &w : s) {
    uint64_t z = (x += 0x9e3779b97f4a7c15ULL);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
    w = z ^ (z >> 31);
  }
}

uint64_t Rng::next() {
  const uint64_t result = rotl(s[1] * 5, 7) * 9;
  const uint64_t t = s[1] << 17;
  s[2] ^= s[0];
  s[3] ^= s[1];
  s[1] ^= s[2];
  s[0] ^= s[3];
  s[2] ^= t;
  s[3] = rotl(s[3], 45);
  return result;
}

double Rng::uniform() { return (double)(next() >> 11) * 0x1.0p-53; }

double Rng::normal() {
  const double u1 = 1.0 - uniform();  // (0, 1]
  const double u2 = uniform();
  return std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2);
}

float Rng::uniform_pm1_f32() {
  const uint64_t u = next() >> 40;  // 24 bits
  return (float)((double)u * 0x1.0p-23 - 1.0);
}

static float nonzero_value(Rng &rv, double sigma) {
  for (;;) {
    float v = (float)(sigma * rv.normal());
    if (v != 0.0f) return v;
  }
}

// Exactly round(density*m*n) positions, uniform without replacement
// (selection sampling, Knuth TAOCP vol. 2, Algorithm S), values N(0, sigma^2)
// rounded to fp32 and never 0.
Csr synth_uniform(int32_t m, int32_t n, double density, double sigma, uint64_t seed) {
  if (m <= 0 || n <= 0 || density < 0 || density > 1) throw Error{SC_ERR_ARG, "bad synthetic matrix arguments"};
  const int64_t cells = (int64_t)m * n;
  int64_t need = (int64_t)std::llround(density * (double)cells);
  if (need > INT32_MAX) throw Error{SC_ERR_ARG, "too many nonzeros"};
  Rng rp(seed), rv(~seed);
  Csr A;
  A.m = m;
  A.n = n;
  A.indptr.assign((size_t)m + 1, 0);
  A.indices.reserve((size_t)need);
  A.data.reserve((size_t)need);
  for (int64_t t = 0; t < cells && need > 0; ++t) {
    if ((double)(cells - t) * rp.uniform() < (double)need) {
      A.indices.push_back((int32_t)(t % n));
      A.indptr[(size_t)(t / n) + 1]++;
      --need;
    }
  }
  for (int32_t i = 0; i < m; ++i) A.indptr[(size_t)i + 1] += A.indptr[(size_t)i];
  for (size_t k = 0; k < A.indices.size(); ++k) A.data.push_back((double)nonzero_value(rv, sigma));
  return A;
}

// Non-overlapping aligned 1x8 row vectors (column start = 0 mod 8) and 4x4
// blocks (row and column start = 0 mod 4), each placement a fair coin flip
// between the two, until nnz reaches round(density*m*n) (overshoot <= 15).
Csr synth_blocks(int32_t m, int32_t n, double density, double sigma, uint64_t seed) {
  if (m <= 0 || n <= 0 || m % 4 || n % 8 || density < 0 || density > 0.5)
    throw Error{SC_ERR_ARG, "structured synthetic matrix needs rows % 4 == 0, cols % 8 == 0, density <= 0.5"};
  const int64_t target = (int64_t)std::llround(density * (double)m * (double)n);
  std::vector<uint8_t> occ((size_t)m * n, 0);
  Rng rp(seed), rv(~seed);
  int64_t nnz = 0, fails = 0;
  while (nnz < target) {
    bool block = (rp.next() >> 63) != 0;
    if (block && nnz + 16 > target + 15) block = false;
    int32_t r0, c0, h, w;
    if (block) {
      r0 = 4 * (int32_t)(rp.uniform() * (m / 4));
      c0 = 4 * (int32_t)(rp.uniform() * (n / 4));
      h = 4;
      w = 4;
    } else {
      r0 = (int32_t)(rp.uniform() * m);
      c0 = 8 * (int32_t)(rp.uniform() * (n / 8));
      h = 1;
      w = 8;
    }
    bool free_ = true;
    for (int32_t r = r0; r < r0 + h && free_; ++r)
      for (int32_t c = c0; c < c0 + w; ++c)
        if (occ[(size_t)r * n + c]) {
          free_ = false;
          break;
        }
    if (!free_) {
      if (++fails > 100000000) throw Error{SC_ERR_ARG, "cannot place blocks at this density"};
      continue;
    }
    for (int32_t r = r0; r < r0 + h; ++r)
      for (int32_t c = c0; c < c0 + w; ++c) occ[(size_t)r * n + c] = 1;
    nnz += (int64_t)h * w;
  }
  Csr A;
  A.m = m;
  A.n = n;
  A.indptr.assign((size_t)m + 1, 0);
  A.indices.reserve((size_t)nnz);
  for (int32_t r = 0; r < m; ++r) {
    const uint8_t *row = &occ[(size_t)r * n];
    for (int32_t c = 0; c < n; ++c)
      if (row[c]) A.indices.push_back(c);
    A.indptr[(size_t)r + 1] = (int32_t)A.indices.size();
  }
  A.data.reserve(A.indices.size());
  for (size_t k = 0; k < A.indices.size(); ++k) A.data.push_back((double)nonzero_value(rv, sigma));
  return A;
}

void synth_dense(float *out, int64_t count, uint64_t seed) {
  Rng r(seed);
  for (int64_t k = 0; k < count; ++k) out[k] = r.uniform_pm1_f32();
}

}  // namespace sc
