"""Generate the small-B (N in {1, 2, 4}) pattern SpMM kernels.

Drop-in for code_gen/main_spmm_small_b_col.py of the reference, same argv:

    python3 main_spmm_small_b_col.py <out.hip> <m> <number_of_warps> <b_col>
                                     [--pattern_dictionary false|FILE]

b_col is baked into the launcher (sc_gen_spmm_small_km<m>_b<b_col>_launch
rejects any other N).  Each lane of a wave64 owns one slot of a pattern
segment, reads its B row as one dword/dwordx2/dwordx4 load and keeps pop x
b_col partial sums; the slot lanes are reduced with wave64 cross-lane
shuffles at the end of the panel (the reference reduces warp32 lanes with
__shfl_down_sync at stride pop).  number_of_warps is recorded only.
"""
import argparse
import os
import sys

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
import _paths  # noqa: E402,F401
import pattern_utiles.pattern_dictionary as pdict  # noqa: E402
from hip.emit import dictionary_patterns, emit_unit  # noqa: E402


def main(argv=None):
    parser = argparse.ArgumentParser(description="Generate gfx950 small-B pattern SpMM kernels.")
    parser.add_argument("path", type=str, default="spmm_small_b_col_demo_gpu_kernels.hip")
    parser.add_argument("m", type=int, default=4)
    parser.add_argument("number_of_warps", type=int, default=1)
    parser.add_argument("b_col", type=int, default=1)
    parser.add_argument("--pattern_dictionary", type=str, default="false")
    args = parser.parse_args(argv)
    if args.b_col < 1:
        raise SystemExit("b_col must be >= 1")
    if args.pattern_dictionary != "false":
        ptd = pdict.read_pattern_dictionary(args.pattern_dictionary)
    else:
        ptd = pdict.generate_pattern_dictionary(args.m, 1)
    origin = (f"main_spmm_small_b_col.py m={args.m} number_of_warps={args.number_of_warps} "
              f"b_col={args.b_col}")
    text = emit_unit(f"spmm_small_km{args.m}_b{args.b_col}", args.m, dictionary_patterns(ptd),
                     kn=1, waves=0, variant=args.b_col, origin=origin, alias=True)
    with open(args.path, "w") as f:
        f.write(text)
    print(f"Text successfully written to {args.path}")
    return text


if __name__ == "__main__":
    main()
