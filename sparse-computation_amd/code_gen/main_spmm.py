"""Generate the large-B (N a multiple of 64, or any N) pattern SpMM kernels.

Drop-in for code_gen/main_spmm.py of the reference, same argv:

    python3 main_spmm.py <out.hip> format <m> <n> <bcol_unroll_factor> <warp_num>
                         <loop_order> [--pattern_dictionary false|FILE]
                         [--second_grid_dim 1]

Writes one gfx950 HIP translation unit: a straight-line body per pattern of
the dictionary (m-row panels, n-slot packs unrolled), the mask switch and
`extern "C"` sc_gen_spmm_km<m>_kn<n>_launch / _record.  Compile it with
`hipcc --offload-arch=gfx950 -I<pkg>/csrc -I<repo>/include` and call it through
sc_spmm_generated().  bcol_unroll_factor, warp_num, loop_order and
second_grid_dim are CUDA launch-shape knobs of the reference; the wave64
kernel picks its lane mapping from N and its waves per panel at launch, so
they are recorded in the file header only.  matrix_type `dense` (the
reference's dense-A variant) is not generated.
"""
import argparse
import os
import sys

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
import _paths  # noqa: E402,F401
import pattern_utiles.pattern_dictionary as pdict  # noqa: E402
from hip.emit import dictionary_patterns, emit_unit  # noqa: E402


def write_text_to_file(text, file_path):
    with open(file_path, "w") as f:
        f.write(text)
    print(f"Text successfully written to {file_path}")


def main_format(m, n, bcol_unroll_factor, warp_num, path, second_grid_dim, ptd, loop_order="i-j"):
    origin = (f"main_spmm.py format m={m} n={n} bcol_unroll_factor={bcol_unroll_factor} "
              f"warp_num={warp_num} loop_order={loop_order} second_grid_dim={second_grid_dim}")
    text = emit_unit(f"spmm_km{m}_kn{n}", m, dictionary_patterns(ptd), kn=n, waves=0, variant=0,
                     origin=origin, alias=True)
    write_text_to_file(text, path)
    return text


def main(argv=None):
    parser = argparse.ArgumentParser(description="Generate gfx950 pattern SpMM kernels.")
    parser.add_argument("path", type=str, default="spmm_demo_gpu_kernels.hip")
    parser.add_argument("matrix_type", type=str, default="format")
    parser.add_argument("m", type=int, default=4)
    parser.add_argument("n", type=int, default=4)
    parser.add_argument("bcol_unroll_factor", type=int, default=32)
    parser.add_argument("warp_num", type=int, default=1)
    parser.add_argument("loop_order", type=str, default="i-j")
    parser.add_argument("--pattern_dictionary", type=str, default="false")
    parser.add_argument("--second_grid_dim", type=int, default=1)
    args = parser.parse_args(argv)
    if args.pattern_dictionary != "false":
        ptd = pdict.read_pattern_dictionary(args.pattern_dictionary)
    else:
        ptd = pdict.generate_pattern_dictionary(args.m, 1)
    if args.matrix_type == "dense":
        raise SystemExit("main_spmm.py: the dense-A variant is not generated for gfx950 "
                         "(its loader never sets MixedFormat::Dense)")
    return main_format(args.m, args.n, args.bcol_unroll_factor, args.warp_num, args.path,
                       args.second_grid_dim, ptd, args.loop_order)


if __name__ == "__main__":
    main()
