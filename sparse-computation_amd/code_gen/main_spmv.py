"""Generate the pattern SpMV kernels (y = A x).

Drop-in for code_gen/main_spmv.py of the reference, same argv:

    python3 main_spmv.py <out.hip> <m> <number_of_warps> [--pattern_dictionary false|FILE]

The launcher sc_gen_spmv_km<m>_launch accepts N = 1 only.  Lanes own slots,
accumulate pop partial sums each and are reduced across the wave64 at the end
of the panel.  The number of bodies follows the dictionary (the reference's
SpMV launch hard-codes 2^m - 1 blocks per panel even in dictionary mode).
"""
import argparse
import os
import sys

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
import _paths  # noqa: E402,F401
import pattern_utiles.pattern_dictionary as pdict  # noqa: E402
from hip.emit import dictionary_patterns, emit_unit  # noqa: E402


def main(argv=None):
    parser = argparse.ArgumentParser()
    parser.add_argument("path", type=str, default="spmv_demo_gpu_kernels.hip")
    parser.add_argument("m", type=int, default=4)
    parser.add_argument("number_of_warps", type=int, default=1)
    parser.add_argument("--pattern_dictionary", type=str, default="false")
    args = parser.parse_args(argv)
    if args.pattern_dictionary != "false":
        ptd = pdict.read_pattern_dictionary(args.pattern_dictionary)
    else:
        ptd = pdict.generate_pattern_dictionary(args.m, 1)
    origin = f"main_spmv.py m={args.m} number_of_warps={args.number_of_warps}"
    text = emit_unit(f"spmv_km{args.m}", args.m, dictionary_patterns(ptd), kn=1, waves=0,
                     variant=1, origin=origin, alias=True)
    with open(args.path, "w") as f:
        f.write(text)
    print(f"Text successfully written to {args.path}")
    return text


if __name__ == "__main__":
    main()
