#!/bin/bash
# Small-B SpMM demo on gfx950 (drop-in for the reference's
# run_local_spmm_small_b_col.sh; same arguments, no venv/pip step).
# Example: ./run_local_spmm_small_b_col.sh data/ash85.mtx 4
# SC_DEMO_BUILD_ONLY=1 stops after building the demo binary.
set -euo pipefail
here="$(cd "$(dirname "$0")" && pwd)"

matrix_path=$1
b_col=$2

kernel_m=4
kernel_n=1

matrix_dir=$(dirname "$matrix_path")
matrix_name=$(basename "$matrix_path" .mtx)
compressed_matrix_path="${matrix_dir}/${matrix_name}-${kernel_m}-${kernel_n}.cfmtx"

python3 "$here/code_gen/ss_format/format_generator.py" "$matrix_path" "$kernel_m" "$kernel_n" --pattern_dictionary false

mkdir -p "$here/build"
python3 "$here/code_gen/main_spmm_small_b_col.py" "$here/build/spmm_small_b_col_demo_gpu_kernels.hip" "$kernel_m" 1 "$b_col" --pattern_dictionary false

"$here/build_demo.sh" 1 "$here/build/spmm_small_b_col_demo_gpu_kernels.hip" "$here/build/spmm_small_b_col_demo_gpu"
[ "${SC_DEMO_BUILD_ONLY:-0}" = "1" ] && exit 0

"$here/build/spmm_small_b_col_demo_gpu" \
  -m "$compressed_matrix_path" \
  --header --baseline=true \
  -n SPMM -s CSR -t "$b_col" \
  --b_matrix_columns="$b_col" \
  --number_of_warps=1
