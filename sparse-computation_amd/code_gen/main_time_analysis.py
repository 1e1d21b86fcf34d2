"""Time-analysis generator: per-kernel resources and timing of the two
code-generation styles of the pattern kernels.

Counterpart of code_gen/main_time_analysis.py of the reference, same argv:

    python3 main_time_analysis.py <out.hip> <m> <n> <compact> [--report] [--dictionary FILE]

compact = 1: pop-count bodies, one per number of rows in a pattern, the rows
  read from the segment's mask at run time (the reference's "nnz based"
  codelets, code_gen/spmm/spmm_time_analysis.py:73-205);
compact = 0: one straight-line body per pattern (the "pattern based"
  codelets, spmm_time_analysis.py:208-335), the style the library ships.

The file holds the kernel unit (m-row panels, n-slot packs) and a standalone
main() (left out when SC_NO_MAIN is defined) that times the unit on a seeded
uniform matrix and checks it against the fp64 product, the counterpart of the
reference's RunSpMMKernel host driver (spmm_time_analysis.py:337-491):

    hipcc --offload-arch=gfx950 -O3 -I<pkg>/csrc -I<repo>/include <out.hip> \\
          -L<pkg>/lib -lsc -o ta && ./ta [M K N density trials]

--report compiles the unit for gfx950 to assembly and prints, for every
kernel, its code size, VGPRs, SGPRs, scratch and occupancy (the resource
study the reference does with `--ptxas-options=-v`).
"""
import argparse
import os
import re
import subprocess
import sys
import tempfile

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
import _paths  # noqa: E402,F401
import pattern_utiles.pattern_dictionary as pdict  # noqa: E402
from hip.emit import dictionary_patterns, emit_unit, sanitize  # noqa: E402

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
PKG = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(PKG, "csrc")
INCLUDE = os.path.join(os.path.dirname(PKG), "include")
HIPFLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature", "-Xclang",
            "-packed-fp32-ops", "-Wno-unused-command-line-argument"]

MAIN_TEMPLATE = r"""
#ifndef SC_NO_MAIN
// ---------------------------------------------------------------------------
// Standalone timing driver: seeded uniform A (M x K, density), B (K x N),
// plan, `trials` launches of this unit timed with HIP events, and the max
// error normalised by (|A| |B|)_ij against the fp64 product.
// ---------------------------------------------------------------------------
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "sc_synth.h"

#define TA_CHECK(x)                                                                      \
  do {                                                                                   \
    int rc_ = (int)(x);                                                                  \
    if (rc_ != 0) {                                                                      \
      std::fprintf(stderr, "%s failed (%d): %s\n", #x, rc_, sc_last_error());            \
      return 1;                                                                          \
    }                                                                                    \
  } while (0)

int main(int argc, char **argv) {
  const int M = argc > 1 ? std::atoi(argv[1]) : 4096;
  const int K = argc > 2 ? std::atoi(argv[2]) : 4096;
  const int N = argc > 3 ? std::atoi(argv[3]) : 128;
  const double density = argc > 4 ? std::atof(argv[4]) : 0.1;
  const int trials = argc > 5 ? std::atoi(argv[5]) : 20;
  sc_csr *A = nullptr;
  sc_cfmtx *cf = nullptr;
  sc_plan *plan = nullptr;
  TA_CHECK(sc_synth_uniform(M, K, density, 0.05, 0x5EED7A00ull, &A));
  TA_CHECK(sc_cfmtx_build(A, __KM__, __KN__, nullptr, &cf));
  TA_CHECK(sc_plan_create(cf, 0, &plan));
  int64_t nnz = 0;
  TA_CHECK(sc_csr_info(A, nullptr, nullptr, &nnz, nullptr));
  std::vector<float> B((size_t)K * N), C((size_t)M * N);
  TA_CHECK(sc_synth_dense(B.data(), (int64_t)B.size(), 0x5EED7A01ull));
  float *dB = nullptr, *dC = nullptr;
  TA_CHECK(hipMalloc(&dB, B.size() * sizeof(float)));
  TA_CHECK(hipMalloc(&dC, C.size() * sizeof(float)));
  TA_CHECK(hipMemcpy(dB, B.data(), B.size() * sizeof(float), hipMemcpyHostToDevice));
  auto run = [&]() {
    return sc_spmm_generated(plan, &sc_gen___NAME___record, (sc_gen_launch_fn)sc_gen___NAME___launch,
                             dB, dC, N, 0, 0, nullptr);
  };
  TA_CHECK(run());
  TA_CHECK(hipDeviceSynchronize());
  hipEvent_t e0, e1;
  TA_CHECK(hipEventCreate(&e0));
  TA_CHECK(hipEventCreate(&e1));
  std::vector<float> us;
  for (int t = 0; t < trials; ++t) {
    TA_CHECK(hipEventRecord(e0, nullptr));
    TA_CHECK(run());
    TA_CHECK(hipEventRecord(e1, nullptr));
    TA_CHECK(hipEventSynchronize(e1));
    float ms = 0;
    TA_CHECK(hipEventElapsedTime(&ms, e0, e1));
    us.push_back(ms * 1000.0f);
  }
  TA_CHECK(hipMemcpy(C.data(), dC, C.size() * sizeof(float), hipMemcpyDeviceToHost));
  const int32_t *ip, *ix;
  const double *ax;
  TA_CHECK(sc_csr_arrays(A, &ip, &ix, &ax));
  double err = 0.0;
  for (int i = 0; i < M; ++i) {
    std::vector<double> ref(N, 0.0), bnd(N, 0.0);
    for (int j = ip[i]; j < ip[i + 1]; ++j) {
      const double a = (double)(float)ax[j];
      for (int k = 0; k < N; ++k) {
        ref[k] += a * B[(size_t)ix[j] * N + k];
        bnd[k] += std::fabs(a) * std::fabs((double)B[(size_t)ix[j] * N + k]);
      }
    }
    for (int k = 0; k < N; ++k) {
      const double d = std::fabs((double)C[(size_t)i * N + k] - ref[k]);
      if (bnd[k] > 0) err = std::max(err, d / bnd[k]);
      else if (d > 0) err = INFINITY;
    }
  }
  std::sort(us.begin(), us.end());
  std::printf("style,km,kn,M,K,N,nnz,us_min,us_median,max_rel_err\n");
  std::printf("__STYLE__,%d,%d,%d,%d,%d,%lld,%.3f,%.3f,%.3e\n", __KM__, __KN__, M, K, N, (long long)nnz,
              us.front(), us[us.size() / 2], err);
  (void)hipFree(dB);
  (void)hipFree(dC);
  sc_plan_destroy(plan);
  sc_cfmtx_free(cf);
  sc_csr_free(A);
  return err <= 1e-5 ? 0 : 2;
}
#endif
"""


def write_text_to_file(text, file_path):
    with open(file_path, "w") as f:
        f.write(text)
    print(f"Text successfully written to {file_path}")


def unit_name(m, n, compact):
    return sanitize(f"ta_{'popcount' if compact else 'pattern'}_km{m}_kn{n}")


def generate(m, n, compact, ptd):
    name = unit_name(m, n, compact)
    style = "popcount" if compact else "pattern"
    text = emit_unit(name, m, dictionary_patterns(ptd), kn=n, waves=0, variant=0,
                     origin=f"main_time_analysis.py m={m} n={n} compact={int(compact)}", style=style)
    main = (MAIN_TEMPLATE.replace("__NAME__", name).replace("__KM__", str(m))
            .replace("__KN__", str(n)).replace("__STYLE__", style))
    return text + main


def resource_report(path):
    """Per-kernel resources of the unit in `path` (gfx950 assembly of this
    build: code bytes, VGPRs, SGPRs, scratch bytes per lane, occupancy)."""
    with tempfile.TemporaryDirectory() as d:
        asm = os.path.join(d, "unit.s")
        cmd = [HIPCC, *HIPFLAGS, f"-I{CSRC}", f"-I{INCLUDE}", "-DSC_NO_MAIN", "--cuda-device-only", "-S",
               path, "-o", asm]
        subprocess.run(cmd, check=True, capture_output=True)
        rows = []
        func = None
        cur = {}
        with open(asm) as f:
            for line in f:
                mlabel = re.match(r"^(_Z\S+):", line)
                if mlabel:
                    func = mlabel.group(1)
                    continue
                mkey = re.match(r"^; (codeLenInByte|TotalNumSgprs|NumVgprs|ScratchSize|Occupancy)"
                                r"(?: =|:) (\d+)", line)
                if mkey and func:
                    cur[mkey.group(1)] = int(mkey.group(2))
                    if mkey.group(1) == "Occupancy":
                        rows.append((func, dict(cur)))
                        cur = {}
    return rows


def short_kernel(mangled):
    m = re.match(r"_ZN2sc\d+(\w+?)ILi(\d+)ELi(\d+)E(?:Lb(\d)E)?", mangled)
    if not m:
        m1 = re.match(r"_ZN2sc\d+(\w+?)I", mangled)
        return m1.group(1) if m1 else mangled[:60]
    name, km, v, flag = m.groups()
    if flag and name == "gather_kernel":
        tag = " f16" if flag == "1" else " f32"  # binary16 values / B / C
    elif flag:
        tag = " stage" if flag == "1" else " nostage"
    else:
        tag = ""
    return f"{name}(km={km} V={v}{tag})"


def main(argv=None):
    parser = argparse.ArgumentParser(description="Time-analysis generator for the gfx950 pattern kernels.")
    parser.add_argument("path", type=str, default="spmm_time_analysis.hip")
    parser.add_argument("m", type=int, default=4)
    parser.add_argument("n", type=int, default=4)
    parser.add_argument("compact", type=int, default=1)
    parser.add_argument("--report", action="store_true",
                        help="compile for gfx950 and print the per-kernel resources")
    parser.add_argument("--dictionary", type=str, default="",
                        help="pattern dictionary file (default: every pattern of m rows)")
    args = parser.parse_args(argv)
    ptd = (pdict.read_pattern_dictionary(args.dictionary) if args.dictionary
           else pdict.generate_pattern_dictionary(args.m, 1))
    text = generate(args.m, args.n, bool(args.compact), ptd)
    write_text_to_file(text, args.path)
    if args.report:
        rows = resource_report(args.path)
        print("kernel,code_bytes,vgprs,sgprs,scratch_bytes_per_lane,occupancy_waves_per_simd")
        for func, r in rows:
            print(f"{short_kernel(func)},{r.get('codeLenInByte')},{r.get('NumVgprs')},{r.get('TotalNumSgprs')},"
                  f"{r.get('ScratchSize')},{r.get('Occupancy')}")
    return text


if __name__ == "__main__":
    main()
