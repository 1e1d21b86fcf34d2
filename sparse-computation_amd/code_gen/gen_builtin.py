"""Generate the pattern kernels libsc ships with.

For every row coarsen factor km in 1..KM_MAX this writes
``csrc/gen/sc_gen_builtin_km<km>.hip`` with the full enumeration of the
2**km - 1 patterns (generate_pattern_dictionary(km, 1)), pack 1 (valid for
any .cfmtx kernel_n, since every segment length is a multiple of 1) and the
waves per panel chosen at launch.  Run by the build before compiling libsc.

    python3 gen_builtin.py [out_dir]
"""
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)

from hip.emit import dictionary_patterns, emit_unit  # noqa: E402
from pattern_utiles.pattern_dictionary import generate_pattern_dictionary  # noqa: E402

KM_MAX = 6


def main(out_dir=None):
    out_dir = out_dir or os.path.join(HERE, "..", "csrc", "gen")
    os.makedirs(out_dir, exist_ok=True)
    written = []
    for km in range(1, KM_MAX + 1):
        ptd = generate_pattern_dictionary(km, 1)
        text = emit_unit(f"builtin_km{km}", km, dictionary_patterns(ptd), kn=1, waves=0,
                         variant=0, origin=f"code_gen/gen_builtin.py: km={km}, all patterns")
        path = os.path.join(out_dir, f"sc_gen_builtin_km{km}.hip")
        old = open(path).read() if os.path.exists(path) else None
        if old != text:  # keep timestamps (and make) quiet when nothing changed
            with open(path, "w") as f:
                f.write(text)
        written.append(path)
    return written


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else None)
