#!/bin/bash
# build_demo.sh <kind 0|1|2> <generated unit .hip> <output binary>
# Builds libsc if needed, then one demo driver (0 large-B SpMM, 1 small-B
# SpMM, 2 SpMV) linked with the generated kernel unit, for gfx950.
set -euo pipefail
here="$(cd "$(dirname "$0")" && pwd)"
kind=$1
unit=$2
out=$3
make -s -C "$here/csrc" ../lib/libsc.so ../lib/libsc_vendor.so
HIPCC=${HIPCC:-/opt/rocm/bin/hipcc}
"$HIPCC" --offload-arch=gfx950 -O3 -std=c++17 -Xclang -target-feature -Xclang -packed-fp32-ops \
  -Wno-unused-command-line-argument -I"$here/csrc" -I"$here/../include" -DSC_DEMO_KIND="$kind" \
  "$here/demos/demo_gpu.hip" "$unit" -L"$here/lib" -lsc -lsc_vendor -Wl,-rpath,"$here/lib" -o "$out" 2>&1 \
  | grep -v "packed-fp32-ops' is not a recognized feature" || true
test -x "$out"
