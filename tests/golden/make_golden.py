"""Write golden .cfmtx vectors for the builder behaviours that no fixture of
the reference pins: non-integral value text, --pattern_dictionary mode
(lossy), kernel_n 0 (32 // pop packing), integer and pattern .mtx fields,
symmetric and duplicate-entry .mtx inputs, and rows not a multiple of km.

Inputs are small seeded .mtx files written here (numpy only).  The expected
outputs come from running the reference's own CLI,
code_gen/ss_format/format_generator.py, as a subprocess in this container
(the reference tree is not available on the GPU box; only the resulting
files are committed).  Re-run with:

    python3 tests/golden/make_golden.py /root/reference
"""
import json
import os
import shutil
import subprocess
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def write_mtx(path, m, n, entries, field="real", symmetry="general"):
    with open(path, "w") as f:
        f.write(f"%%MatrixMarket matrix coordinate {field} {symmetry}\n")
        f.write("% seeded golden input\n")
        f.write(f"{m} {n} {len(entries)}\n")
        for (r, c, v) in entries:
            if field == "pattern":
                f.write(f"{r + 1} {c + 1}\n")
            elif field == "integer":
                f.write(f"{r + 1} {c + 1} {int(v)}\n")
            else:
                f.write(f"{r + 1} {c + 1} {v}\n")


def random_entries(rng, m, n, density, scale):
    mask = rng.random((m, n)) < density
    rows, cols = np.nonzero(mask)
    vals = rng.standard_normal(len(rows)) * scale
    # mix magnitudes so that positional and exponent text both appear
    vals[::7] *= 1e-4
    vals[::11] *= 1e6
    vals[::13] = np.round(vals[::13] * 100)  # integral floats print as "x.0"
    vals = vals.astype(np.float32).astype(np.float64)
    vals[vals == 0] = 0.5
    return [(int(r), int(c), repr(float(v))) for r, c, v in zip(rows, cols, vals)]


def cases(rng):
    out = []
    out.append(("real_17x23", 17, 23, random_entries(rng, 17, 23, 0.35, 0.05), "real", "general",
                [(4, 1), (4, 3), (3, 0), (6, 2), (1, 5), (2, 0), (5, 8)]))
    out.append(("real_64x40", 64, 40, random_entries(rng, 64, 40, 0.2, 1.0), "real", "general",
                [(4, 1), (4, 2), (5, 0), (6, 0)]))
    ints = [(r, c, str(int(v))) for r, c, v in
            [(e[0], e[1], rng.integers(-9, 10) or 3) for e in random_entries(rng, 13, 9, 0.4, 1.0)]]
    out.append(("integer_13x9", 13, 9, ints, "integer", "general", [(4, 1), (3, 2)]))
    pat = [(e[0], e[1], "") for e in random_entries(rng, 11, 14, 0.3, 1.0)]
    out.append(("pattern_11x14", 11, 14, pat, "pattern", "general", [(4, 1), (2, 0)]))
    low = [(e[0], e[1], e[2]) for e in random_entries(rng, 12, 12, 0.3, 1.0) if e[0] >= e[1]]
    out.append(("symmetric_12", 12, 12, low, "real", "symmetric", [(4, 1), (3, 2)]))
    dup = random_entries(rng, 9, 10, 0.3, 1.0)
    dup = dup + [(r, c, "0.25") for (r, c, _) in dup[:5]]  # repeated coordinates are summed
    out.append(("duplicates_9x10", 9, 10, dup, "real", "general", [(4, 1), (2, 2)]))
    return out


DICTS = {
    # header "m n count" then "<bits> <id>" lines (read_pattern_dictionary)
    "dict4_sub": "4 1 6\n1111 0\n1000 1\n0100 2\n0010 3\n0001 4\n1100 5\n",
    "dict3_all_reversed": "3 1 7\n001 0\n010 1\n011 2\n100 3\n101 4\n110 5\n111 6\n",
}


def main(ref_root):
    gen = os.path.join(ref_root, "code_gen", "ss_format", "format_generator.py")
    if not os.path.exists(gen):
        raise SystemExit(f"reference format_generator.py not found under {ref_root}")
    rng = np.random.default_rng(0x5EED)
    manifest = []
    out_dir = os.path.join(HERE, "cfmtx")
    shutil.rmtree(out_dir, ignore_errors=True)
    os.makedirs(out_dir)
    with tempfile.TemporaryDirectory() as tmp:
        for name, m, n, entries, field, sym, factors in cases(rng):
            mtx = os.path.join(tmp, name + ".mtx")
            write_mtx(mtx, m, n, entries, field, sym)
            shutil.copy(mtx, os.path.join(out_dir, name + ".mtx"))
            runs = [(km, kn, None) for km, kn in factors]
            if field == "real" and sym == "general":
                runs += [(4, 1, "dict4_sub"), (3, 2, "dict3_all_reversed"), (4, 0, "dict4_sub")]
            for km, kn, dname in runs:
                args = [sys.executable, gen, mtx, str(km), str(kn)]
                tag = f"{name}-{km}-{kn}"
                if dname:
                    dpath = os.path.join(tmp, dname + ".txt")
                    with open(dpath, "w") as f:
                        f.write(DICTS[dname])
                    shutil.copy(dpath, os.path.join(out_dir, dname + ".txt"))
                    args += ["--pattern_dictionary", dpath]
                    tag += f"-{dname}"
                r = subprocess.run(args, cwd=tmp, capture_output=True, text=True)
                produced = os.path.join(tmp, f"{name}-{km}-{kn}.cfmtx")
                if r.returncode != 0 or not os.path.exists(produced):
                    manifest.append({"tag": tag, "mtx": name + ".mtx", "km": km, "kn": kn,
                                     "dictionary": dname, "error": r.stderr.strip().splitlines()[-1]})
                    continue
                shutil.move(produced, os.path.join(out_dir, tag + ".cfmtx"))
                manifest.append({"tag": tag, "mtx": name + ".mtx", "km": km, "kn": kn,
                                 "dictionary": dname, "cfmtx": tag + ".cfmtx"})
    with open(os.path.join(HERE, "manifest.json"), "w") as f:
        json.dump(manifest, f, indent=1)
    print(f"wrote {len(manifest)} golden cases to {out_dir}")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
