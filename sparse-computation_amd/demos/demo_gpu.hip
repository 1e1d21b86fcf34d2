// demo_gpu.hip -- the SpMM / small-B SpMM / SpMV demo drivers on gfx950.
//
// Replaces example_cuda/spmm_demo_gpu.cu, spmm_small_b_col_demo_gpu.cu and
// spmv_demo_gpu.cu (one source, built with SC_DEMO_KIND 0 / 1 / 2): same
// command line (src/InputParser.cpp:22-163), same load path
// (loadCfmtxMatrices -> .cfmtx + companion .mtx), same trial loop
// (benchmark/src/SWBench.cpp:26-41: 7 trials for SpMM, 20 for SpMV, each
// timed with device events around the kernel only) and the same CSV layout
// (benchmark/src/Stats.cpp:35-90, src/test_utils.cpp:12-32,
// example_cuda/spmm_demo_gpu.cu:159-197).
//
// The kernel is the generated unit linked into the binary (sc_gen_unit_record /
// sc_gen_unit_launch, emitted by code_gen/main_spmm.py,
// main_spmm_small_b_col.py or main_spmv.py), launched through
// sc_spmm_generated, which rejects a .cfmtx the unit was not generated for.
//
// Differences, by design: B is filled from a seeded generator instead of
// unseeded rand(); the correctness reference is the fp64 product on the host
// (the reference compares with cuSPARSE), and Correct is 1 when the max error
// normalised by (|A| |B|)_ij is <= 1e-5 while Error keeps the reference's
// inf-norm of the difference.  --baseline adds the vendor-library rows of
// the reference in its order, on this platform's libraries (libsc_vendor:
// hipBLAS Sgemm for "CuBlas", hipBLAS fp16 GemmEx for "CuBlas Half Tensor",
// hipBLAS fp32 GemmEx for "CuBlas GemmX", rocSPARSE for "CuSparse"; gfx950
// has no TF32, so the "GemmX Tensor Float" row is not printed), then the
// single-thread CPU spmm_csr_float row.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <sstream>
#include <string>
#include <vector>

#include "sc_api.h"
#include "sc_synth.h"
#include "sc_vendor.h"

#ifndef SC_DEMO_KIND
#define SC_DEMO_KIND 0
#endif

extern "C" const sc_gen_record *sc_gen_unit_record;
extern "C" int sc_gen_unit_launch(const void *view, const float *B, float *C, int N, int accumulate,
                                  int waves, void *stream);

namespace {

struct Config {
  std::string matrixPath, dictionaryPath, op, storage;
  int header = 0, nThread = 1, coarsening = 5, packing = 1, tuning = 0, lim = 0;
  int number_of_warps = 8, b_unroll_factor = 4, mTile = 64, nTile = 64, bCols = 256;
  int hint = 0, prefetch = 0;
  bool baseline = false, analyze = false, prefer_fsc = false;
};

void usage() {
  std::printf(
      "Usage: demo [options]\n"
      "  -m, --matrix PATH            .cfmtx file (companion .mtx next to it)\n"
      "      --dict PATH              dictionary file\n"
      "  -n, --numerical_operation    SPMV | SPTRS | SPMM\n"
      "  -s, --storage_format         CSR | CSC\n"
      "  -t, --threads N              (default 1)\n"
      "  -c, --coarsening N  -p, --packing N  -u, --tuning N  --iteration_limit N\n"
      "      --prefer_fsc[=bool] --number_of_warps N (8) --b_unroll_factor N (4)\n"
      "      --m_tile_size N (64) --n_tile_size N (64) --b_matrix_columns N (256)\n"
      "      --hint N --prefetch_distance N --baseline[=bool] --analyze_codelets[=bool]\n"
      "  -d, --header                 print the CSV header\n"
      "  -h, --help\n");
}

bool parse_bool(const std::string &v) { return v.empty() || v == "true" || v == "1" || v == "yes"; }

// The cxxopts syntax the run scripts use: --opt=value, --opt value, -o value,
// bare boolean flags.  Mandatory options missing -> message and exit(0), as
// the reference does.
Config parse(int argc, char **argv) {
  static const std::map<std::string, std::string> shorts = {
      {"m", "matrix"}, {"n", "numerical_operation"}, {"s", "storage_format"}, {"t", "threads"},
      {"c", "coarsening"}, {"p", "packing"}, {"u", "tuning"}, {"d", "header"}, {"h", "help"}};
  static const char *flags[] = {"header", "help", "baseline", "analyze_codelets", "prefer_fsc"};
  std::map<std::string, std::string> kv;
  for (int i = 1; i < argc; ++i) {
    std::string a = argv[i], key, val;
    bool has_val = false;
    if (a.rfind("--", 0) == 0) {
      key = a.substr(2);
      size_t eq = key.find('=');
      if (eq != std::string::npos) {
        val = key.substr(eq + 1);
        key = key.substr(0, eq);
        has_val = true;
      }
    } else if (a.size() >= 2 && a[0] == '-') {
      auto it = shorts.find(a.substr(1, 1));
      if (it == shorts.end()) {
        std::printf("Unknown option %s\n", a.c_str());
        std::exit(1);
      }
      key = it->second;
      if (a.size() > 2) {
        val = a.substr(2);
        has_val = true;
      }
    } else {
      std::printf("Unexpected argument %s\n", a.c_str());
      std::exit(1);
    }
    const bool is_flag = std::find(std::begin(flags), std::end(flags), key) != std::end(flags);
    if (!has_val && !is_flag) {
      if (i + 1 >= argc) {
        std::printf("Option %s requires a value\n", key.c_str());
        std::exit(1);
      }
      val = argv[++i];
    }
    kv[key] = val;
  }
  if (kv.count("help")) {
    usage();
    std::exit(0);
  }
  Config c;
  auto geti = [&](const char *k, int &dst) {
    if (kv.count(k)) dst = std::atoi(kv[k].c_str());
  };
  if (!kv.count("matrix")) {
    std::printf("'matrix' is manditory argument. Use --help\n");
    std::exit(0);
  }
  if (!kv.count("numerical_operation")) {
    std::printf("'numerical_operation' is manditory argument. Use --help\n");
    std::exit(0);
  }
  if (!kv.count("storage_format")) {
    std::printf("'storage_format' is manditory argument. Use --help\n");
    std::exit(0);
  }
  c.matrixPath = kv["matrix"];
  if (kv.count("dict")) c.dictionaryPath = kv["dict"];
  c.op = kv["numerical_operation"];
  c.storage = kv["storage_format"];
  if (c.op != "SPMV" && c.op != "SPTRS" && c.op != "SPMM") {
    std::printf("'numerical_operation' must be passed in as one of: ['SPMV', 'SPTRS', 'SPMM']\n");
    std::exit(0);
  }
  if (c.storage != "CSR" && c.storage != "CSC") {
    std::printf("'storage_format' must be passed in as one of: ['CSC', 'CSR']\n");
    std::exit(0);
  }
  geti("threads", c.nThread);
  geti("coarsening", c.coarsening);
  geti("packing", c.packing);
  geti("tuning", c.tuning);
  geti("iteration_limit", c.lim);
  geti("number_of_warps", c.number_of_warps);
  geti("b_unroll_factor", c.b_unroll_factor);
  geti("m_tile_size", c.mTile);
  geti("n_tile_size", c.nTile);
  geti("b_matrix_columns", c.bCols);
  geti("hint", c.hint);
  geti("prefetch_distance", c.prefetch);
  if (kv.count("baseline")) c.baseline = parse_bool(kv["baseline"]);
  if (kv.count("analyze_codelets")) c.analyze = parse_bool(kv["analyze_codelets"]);
  if (kv.count("prefer_fsc")) c.prefer_fsc = parse_bool(kv["prefer_fsc"]);
  c.header = kv.count("header") ? 1 : 0;
  return c;
}

#define HIP_OK(x)                                                                   \
  do {                                                                              \
    hipError_t e_ = (x);                                                            \
    if (e_ != hipSuccess) {                                                         \
      std::fprintf(stderr, "HIP error %s at %s:%d\n", hipGetErrorString(e_), __FILE__, __LINE__); \
      std::exit(2);                                                                 \
    }                                                                               \
  } while (0)

#define SC_OK_OR_DIE(x)                                                              \
  do {                                                                               \
    int rc_ = (x);                                                                   \
    if (rc_ != SC_OK) {                                                              \
      std::fprintf(stderr, "libsc error %d: %s\n", rc_, sc_last_error());           \
      std::exit(1);                                                                  \
    }                                                                                \
  } while (0)

std::string fixed9(double v) {
  char b[64];
  std::snprintf(b, sizeof b, "%.9f", v);
  return b;
}

// std::to_string formatting of a double / int, as the reference's CSV uses
std::string tostr(double v) { return std::to_string(v); }

struct Trial {
  double seconds;
  bool correct;
  double error;
};

// Stats::printCSVHeader / printCSV (benchmark/src/Stats.cpp:35-90) for one
// implementation: no analysis timer, no PAPI events, one timed region per trial.
std::string stats_header(int trials) {
  std::ostringstream os;
  os << "Operation Name,Implementation Name,Number of Trials,Matrix Name,Number of Threads,"
        "Number of Subregions,";
  for (int i = 0; i < trials; ++i)
    os << "Trial" << i << " Subregion0 Executor," << "Correct" << i << ",Error" << i << ",";
  return os.str();
}

std::string stats_row(const std::string &op, const std::string &name, const std::string &matrix,
                      int threads, const std::vector<Trial> &t) {
  std::ostringstream os;
  os << op << "," << name << "," << t.size() << "," << matrix << "," << threads << ",0,";
  for (auto &x : t) os << fixed9(x.seconds) << "," << (x.correct ? 1 : 0) << "," << tostr(x.error) << ",";
  return os.str();
}

}  // namespace

int main(int argc, char **argv) {
  Config cfg = parse(argc, argv);
  sc_csr *A = nullptr;
  sc_cfmtx *cf = nullptr;
  if (sc_load_cfmtx_matrices(cfg.matrixPath.c_str(), &A, &cf) != SC_OK) {
    std::fprintf(stderr, "%s\n", sc_last_error());
    return 1;
  }
  int32_t M, K, km, npat, kn, npanels, kind;
  int64_t nnz;
  SC_OK_OR_DIE(sc_csr_info(A, &M, &K, &nnz, &kind));
  SC_OK_OR_DIE(sc_cfmtx_info(cf, nullptr, nullptr, &km, &npat, &kn, &npanels));
  const int kernel_n = kn == 0 ? 1 : kn;  // the reader turns a header kn of 0 into 1
#if SC_DEMO_KIND == 2
  const int N = 1;
  const int trials = 20;
  const char *op_name = "SpMV Compressed Format";  // spmv_demo_gpu.cu:124
  const char *exp_name = "SpMV_Demo";
#elif SC_DEMO_KIND == 1
  const int N = cfg.bCols;
  const int trials = 7;
  const char *op_name = "SpMM Format Pack Block Cache less";  // spmm_small_b_col_demo_gpu.cu
  const char *exp_name = "SpMM_Demo";
#else
  const int N = cfg.bCols;
  const int trials = 7;
  const char *op_name = "SpMM Format Pack Block Cache less";
  const char *exp_name = "SpMM_Demo";
#endif
  if (N < 1) {
    std::fprintf(stderr, "b_matrix_columns must be >= 1\n");
    return 1;
  }
  const int32_t *ip, *ix;
  const double *ax;
  SC_OK_OR_DIE(sc_csr_arrays(A, &ip, &ix, &ax));
  std::vector<float> B((size_t)K * N);
  SC_OK_OR_DIE(sc_synth_dense(B.data(), (int64_t)B.size(), 0x5EED0000ull + (uint64_t)N));

  // host reference: fp64 product of the fp32 operands and its |A||B| bound
  std::vector<double> ref((size_t)M * N, 0.0), bound((size_t)M * N, 0.0);
  for (int i = 0; i < M; ++i)
    for (int j = ip[i]; j < ip[i + 1]; ++j) {
      const double a = (double)(float)ax[j];
      const float *b = &B[(size_t)ix[j] * N];
      for (int k = 0; k < N; ++k) {
        ref[(size_t)i * N + k] += a * b[k];
        bound[(size_t)i * N + k] += std::fabs(a) * std::fabs((double)b[k]);
      }
    }
  auto check = [&](const std::vector<float> &C, bool &ok) {
    double inf = 0.0, rel = 0.0;
    for (size_t t = 0; t < C.size(); ++t) {
      const double d = std::fabs((double)C[t] - ref[t]);
      inf = std::max(inf, d);
      if (bound[t] > 0) rel = std::max(rel, d / bound[t]);
      else if (d > 0) rel = INFINITY;
    }
    ok = rel <= 1e-5;
    return inf;
  };

  sc_plan *plan = nullptr;
  // both layouts: the generated unit runs its km-row bodies or, for launches
  // whose one-row gathers stay small, its one-row body (sc_spmm's rule)
  SC_OK_OR_DIE(sc_plan_create(cf, 0, &plan));
  float *dB = nullptr, *dC = nullptr;
  HIP_OK(hipMalloc(&dB, B.size() * sizeof(float)));
  HIP_OK(hipMalloc(&dC, (size_t)M * N * sizeof(float)));
  HIP_OK(hipMemcpy(dB, B.data(), B.size() * sizeof(float), hipMemcpyHostToDevice));
  hipEvent_t e0, e1;
  HIP_OK(hipEventCreate(&e0));
  HIP_OK(hipEventCreate(&e1));
  std::vector<Trial> gpu;
  std::vector<float> C((size_t)M * N);
  // first call outside the timed trials (plan workspace, code object load)
  SC_OK_OR_DIE(sc_spmm_generated(plan, sc_gen_unit_record, sc_gen_unit_launch, dB, dC, N, 0, 0, nullptr));
  HIP_OK(hipDeviceSynchronize());
  for (int tr = 0; tr < trials; ++tr) {
    HIP_OK(hipEventRecord(e0, nullptr));
    SC_OK_OR_DIE(sc_spmm_generated(plan, sc_gen_unit_record, sc_gen_unit_launch, dB, dC, N, 0, 0, nullptr));
    HIP_OK(hipEventRecord(e1, nullptr));
    HIP_OK(hipEventSynchronize(e1));
    float ms = 0;
    HIP_OK(hipEventElapsedTime(&ms, e0, e1));
    HIP_OK(hipMemcpy(C.data(), dC, C.size() * sizeof(float), hipMemcpyDeviceToHost));
    Trial t{ms * 1e-3, false, 0.0};
    t.error = check(C, t.correct);
    gpu.push_back(t);
  }

  // One vendor-library row: set-up outside the timer, the library call alone
  // between the events (the reference's execute() brackets), result checked
  // like the pattern kernel's.
  auto vendor_trials = [&](int vkind, int alg) {
    std::vector<Trial> out;
    sc_vendor *h = nullptr;
    if (sc_vendor_create(A, vkind, N, alg, &h) != SC_OK ||
        sc_vendor_bind(h, dB, dC, nullptr) != SC_OK || sc_vendor_run(h, nullptr) != SC_OK) {
      std::fprintf(stderr, "vendor baseline %d: %s\n", vkind, sc_vendor_last_error());
      if (h) sc_vendor_destroy(h);
      return out;
    }
    HIP_OK(hipDeviceSynchronize());
    std::vector<float> Cv((size_t)M * N);
    for (int tr = 0; tr < trials; ++tr) {
      HIP_OK(hipEventRecord(e0, nullptr));
      if (sc_vendor_run(h, nullptr) != SC_OK) {
        std::fprintf(stderr, "vendor baseline %d: %s\n", vkind, sc_vendor_last_error());
        break;
      }
      HIP_OK(hipEventRecord(e1, nullptr));
      HIP_OK(hipEventSynchronize(e1));
      float ms = 0;
      HIP_OK(hipEventElapsedTime(&ms, e0, e1));
      if (sc_vendor_fetch(h, nullptr) != SC_OK) break;
      HIP_OK(hipMemcpy(Cv.data(), dC, Cv.size() * sizeof(float), hipMemcpyDeviceToHost));
      Trial t{ms * 1e-3, false, 0.0};
      t.error = check(Cv, t.correct);
      out.push_back(t);
    }
    sc_vendor_destroy(h);
    return out;
  };

  const std::string tp_header = "MatrixName,Density,nRows,nCols,NNZ,Mode,Algorithm,bCols";
  const std::string tp_row = cfg.matrixPath + "," + tostr(0.0) + "," + tostr((double)M) + "," +
                             tostr((double)K) + "," + tostr((double)nnz) + ",Random,," + std::to_string(0);
  const std::string sp_header = "nThreads,Iter Per Partition,MTile,NTile,";
  const std::string sp_row = "1,1,1,1,";
  std::ostringstream suffix;
  suffix << "," << kernel_n << "," << km << "," << N << "," << cfg.b_unroll_factor << ","
         << cfg.number_of_warps;
  if (cfg.header)
    std::printf("%s%s%s,kernel_n,kernel_m,b_cols,b_unroll_factor,number_of_warps\n",
                stats_header(trials).c_str(), sp_header.c_str(), tp_header.c_str());
  if (cfg.baseline) {
    auto row = [&](const char *name, const std::vector<Trial> &t) {
      if (t.size() == (size_t)trials)
        std::printf("%s%s%s%s\n", stats_row(name, exp_name, cfg.matrixPath, cfg.nThread, t).c_str(),
                    sp_row.c_str(), tp_row.c_str(), suffix.str().c_str());
    };
#if SC_DEMO_KIND == 2
    // example_cuda/spmv_demo_gpu.cu:150-157: cuSPARSE, then cuBLAS
    row("SpMV rocSparse GPU", vendor_trials(SC_VENDOR_ROCSPARSE_SPMV, 0));
    row("SpMV hipBlas GPU", vendor_trials(SC_VENDOR_HIPBLAS_SGEMM, 0));
#else
    // example_cuda/spmm_demo_gpu.cu:172-191: cuBLAS, Half, GemmX, (TF32), cuSPARSE
    row("SpMM hipBlas", vendor_trials(SC_VENDOR_HIPBLAS_SGEMM, 0));
    row("SpMM hipBlas Half Tensor", vendor_trials(SC_VENDOR_HIPBLAS_HALF, 0));
    row("SpMM hipBlas GemmX", vendor_trials(SC_VENDOR_HIPBLAS_GEMMEX, 0));
    row("SpMM rocSparse", vendor_trials(SC_VENDOR_ROCSPARSE_SPMM, 0));
#endif
    // The reference's CPU routines, one thread: spmm_csr_float
    // (example_cuda/spmm_demo_gpu_utils.h:25-36, fp32 sums) for SpMM,
    // spmv_csr_float (example_cuda/spmv_demo_gpu_utils.h:86-98, fp64 row
    // sums) for SpMV.
    std::vector<Trial> cpu;
    std::vector<float> Cc((size_t)M * N);
    for (int tr = 0; tr < trials; ++tr) {
      std::fill(Cc.begin(), Cc.end(), 0.0f);
      auto t0 = std::chrono::steady_clock::now();
#if SC_DEMO_KIND == 2
      for (int i = 0; i < M; ++i) {
        double sum = 0.0;
        for (int j = ip[i]; j < ip[i + 1]; ++j) sum += (double)(float)ax[j] * B[ix[j]];
        Cc[i] += (float)sum;
      }
#else
      for (int i = 0; i < M; ++i)
        for (int j = ip[i]; j < ip[i + 1]; ++j) {
          const float v = (float)ax[j];
          const float *b = &B[(size_t)ix[j] * N];
          float *c = &Cc[(size_t)i * N];
          for (int k = 0; k < N; ++k) c[k] += v * b[k];
        }
#endif
      auto t1 = std::chrono::steady_clock::now();
      Trial t{std::chrono::duration<double>(t1 - t0).count(), false, 0.0};
      t.error = check(Cc, t.correct);
      cpu.push_back(t);
    }
#if SC_DEMO_KIND == 2
    row("SpMV Serial Float", cpu);
#else
    row("SpMM Serial Float", cpu);
#endif
  }
  std::printf("%s%s%s%s\n", stats_row(op_name, exp_name, cfg.matrixPath, cfg.nThread, gpu).c_str(),
              sp_row.c_str(), tp_row.c_str(), suffix.str().c_str());
  HIP_OK(hipFree(dB));
  HIP_OK(hipFree(dC));
  sc_plan_destroy(plan);
  sc_cfmtx_free(cf);
  sc_csr_free(A);
  return 0;
}
