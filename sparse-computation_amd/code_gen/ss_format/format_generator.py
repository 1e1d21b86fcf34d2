"""Build the .cfmtx compressed format of a Matrix Market file.

Drop-in for code_gen/ss_format/format_generator.py of the reference: same
command line, same output files (byte-identical), same companion naming:

    python3 format_generator.py <matrix.mtx> <kernel_m> <kernel_n>
            [--pattern_dictionary false|FILE] [--save_collection false|true]

writes <matrix>-<kernel_m>-<kernel_n>.cfmtx (and <matrix>.cfmtx with
--save_collection true).  The work is done by libsc (sc_mtx_read in scipy
mode, sc_cfmtx_build, sc_cfmtx_write); this file only parses arguments and
prints the per-pattern slot counts.
"""
import argparse
import os
import sys
import time

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
import _paths  # noqa: E402,F401
import sc_amd  # noqa: E402


def generate(path, kernel_m, kernel_n, pattern_dictionary="false", save_collection=False,
             verbose=True):
    """Returns the list of written paths (empty if `path` is not a .mtx)."""
    if path == "":
        raise ValueError("Please provide the path to the matrix file")
    if not path.endswith(".mtx"):
        return []
    dictionary = None if pattern_dictionary == "false" else pattern_dictionary
    t0 = time.time()
    A = sc_amd.Csr.from_mtx(path, sc_amd.MTX_SCIPY)
    cf = sc_amd.Cfmtx.build(A, kernel_m, kernel_n, dictionary)
    out = [path[:-4] + f"-{kernel_m}-{kernel_n}.cfmtx"]
    cf.write(out[0])
    if save_collection:
        out.append(path[:-4] + ".cfmtx")
        cf.write(out[1])
    if verbose:
        m, n = A.shape
        print(f"matrix {path}: {m} x {n}, nnz {A.nnz}, km {kernel_m}, kn {kernel_n}")
        for p in cf.patterns():
            print(f"pattern {p['id']:3d} {p['bits']}: {len(p['cb'])} slots")
        print(f"wrote {', '.join(out)} in {time.time() - t0:.3f} s")
    return out


def main(argv=None):
    parser = argparse.ArgumentParser(description="Build the .cfmtx format of a .mtx matrix.")
    parser.add_argument("path", type=str, default="")
    parser.add_argument("kernel_m", type=int, default=4)
    parser.add_argument("kernel_n", type=int, default=4)
    parser.add_argument("--pattern_dictionary", type=str, default="false")
    parser.add_argument("--save_collection", type=str, default="false")
    args = parser.parse_args(argv)
    generate(args.path, args.kernel_m, args.kernel_n, args.pattern_dictionary,
             args.save_collection == "true")


if __name__ == "__main__":
    main()
