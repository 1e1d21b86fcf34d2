// sc_format.hpp -- host-side types of the enumerate-and-sparse-coarsen format.
//
// These replace the reference's host structures:
//   Csr      <- sym_lib::CSR                (aggregation/include/aggregation/def.h:181-240)
//               and the scipy CSR the Python builder works on
//               (code_gen/ss_format/format_generator.py:214-215)
//   Cfmtx    <- MixedFormat<float> of per-pattern CompressedFormat<float>
//               (include/compressed_format/CompressedFormat.h:88-279), plus the
//               exact values the Python builder keeps for writing
//               (format_generator.py:21-33)
#pragma once

#include <cstdint>
#include <string>
#include <vector>

namespace sc {

// Kind of the values a .mtx field holds; it decides how the .cfmtx writer
// prints them (numpy float64 -> "1.0", numpy int64 -> "1").
enum ValueKind : int32_t { VALUES_REAL = 0, VALUES_INTEGER = 1, VALUES_PATTERN = 2 };

struct Csr {
  int32_t m = 0, n = 0;
  std::vector<int32_t> indptr;   // m + 1
  std::vector<int32_t> indices;  // nnz, sorted and unique within a row
  std::vector<double> data;      // nnz
  ValueKind kind = VALUES_REAL;
  int64_t nnz() const { return indptr.empty() ? 0 : indptr.back(); }
};

// One pattern of a .cfmtx: header line `<bits> <id> ` and its three data lines.
struct Pattern {
  std::string bits;             // character r == '1' <=> panel row r is present
  int32_t id = 0;               // the id printed on the header line
  int32_t pop = 0;              // number of '1' characters
  std::vector<int32_t> rpp;     // row-panel pointer into slots (cumulative, padded)
  std::vector<int32_t> cb;      // column of every slot (padding repeats the max)
  std::vector<double> val64;    // exact values as built (only when built here)
  std::vector<uint8_t> pad;     // 1 = padding entry, printed as "0"
  std::vector<float> val32;     // the values as the reader holds them (fp32)
};

struct Cfmtx {
  int32_t m = 0, n = 0;         // original (unpadded) matrix shape
  int32_t km = 0;               // row coarsen factor (kernel_m)
  int32_t kn = 0;               // column pack as written in the header (0 allowed)
  ValueKind kind = VALUES_REAL;
  bool has_exact = false;       // val64/pad are valid (built, not read)
  // Data-block order: patterns[i] is the i-th RPP/CB/value block.  Built
  // files put block `id` at position id; the reader pairs the i-th header
  // line with the i-th data block (utils/Sparse_io.cpp:136-182).
  std::vector<Pattern> patterns;
  // Order of the header's pattern lines, as indices into `patterns`
  // (dictionary insertion order, format_generator.py:149-152).
  std::vector<int32_t> header_order;
  int32_t npanels() const { return km > 0 ? (m + km - 1) / km : 0; }
};

// Errors are reported by throwing sc::Error; the C ABI turns them into codes.
struct Error {
  int code;
  std::string msg;
};

// ---- pattern enumeration ----------------------------------------------------
// id -> bit string, for ids 0 .. 2^bits-2 (closed form id = 2^bits-1-int(bits,2)).
std::vector<std::string> enumerate_patterns(int km, int kn);
// The dictionary file of --pattern_dictionary: header "m n count", then lines
// "<bits> <id>"; returned in file order as (bits, id) pairs.
std::vector<std::pair<std::string, int32_t>> read_pattern_dictionary(const std::string &path);

// ---- .mtx -------------------------------------------------------------------
enum MtxMode : int32_t {
  MTX_SCIPY = 0,   // scipy.io.mmread(...).tocsr(): duplicates summed
  MTX_SYMLIB = 1,  // sym_lib read_header/read_triplets_real: duplicates kept
};
Csr read_mtx(const std::string &path, MtxMode mode);
void write_mtx(const Csr &A, const std::string &path);

// ---- .cfmtx -----------------------------------------------------------------
Cfmtx build_cfmtx(const Csr &A, int km, int kn,
                  const std::vector<std::pair<std::string, int32_t>> *dictionary);
std::string cfmtx_text(const Cfmtx &cf);
void write_cfmtx(const Cfmtx &cf, const std::string &path);
Cfmtx read_cfmtx(const std::string &path);
std::string companion_mtx_path(const std::string &cfmtx_path);

// Python repr() of a double (the text numpy's str(np.float64) prints).
std::string py_repr(double x);
// The fp32 value the reference's reader obtains from the text of x.
float reader_f32(double x);

// ---- synthetic inputs (seeded, platform independent) ------------------------
struct Rng {
  uint64_t s[4];
  explicit Rng(uint64_t seed);
  uint64_t next();
  double uniform();        // [0, 1) with 53 bits
  double normal();         // Box-Muller in double
  float uniform_pm1_f32(); // (float)(2u - 1), u a 24-bit uniform
};
Csr synth_uniform(int32_t m, int32_t n, double density, double sigma, uint64_t seed);
Csr synth_blocks(int32_t m, int32_t n, double density, double sigma, uint64_t seed);
void synth_dense(float *out, int64_t count, uint64_t seed);

}  // namespace sc
