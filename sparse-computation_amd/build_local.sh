#!/bin/bash
# Generate the three kernel units and build libsc and the three demo
# binaries into build/ (drop-in for the reference's build_local.sh; same
# arguments, no venv/pip step).
# Example: ./build_local.sh 4 32
set -euo pipefail
here="$(cd "$(dirname "$0")" && pwd)"

kernel_m=${1:-4}
b_col=${2:-32}
kernel_n=2
b_unroll_factor=1
if [ "$b_col" -gt 32 ]; then
  warp_num=2
else
  warp_num=1
fi

mkdir -p "$here/build"
python3 "$here/code_gen/main_spmm_small_b_col.py" "$here/build/spmm_small_b_col_demo_gpu_kernels.hip" "$kernel_m" 1 "$b_col" --pattern_dictionary false
python3 "$here/code_gen/main_spmm.py" "$here/build/spmm_demo_gpu_kernels.hip" format "$kernel_m" "$kernel_n" "$b_unroll_factor" "$warp_num" i-j --pattern_dictionary false
python3 "$here/code_gen/main_spmv.py" "$here/build/spmv_demo_gpu_kernels.hip" "$kernel_m" 1 --pattern_dictionary false

"$here/build_demo.sh" 1 "$here/build/spmm_small_b_col_demo_gpu_kernels.hip" "$here/build/spmm_small_b_col_demo_gpu"
"$here/build_demo.sh" 0 "$here/build/spmm_demo_gpu_kernels.hip" "$here/build/spmm_demo_gpu"
"$here/build_demo.sh" 2 "$here/build/spmv_demo_gpu_kernels.hip" "$here/build/spmv_demo_gpu"
