"""Reference citations in the repository point at real lines.

Every `file:a-b` citation of a reference file in the repository's sources and
documents must lie inside that file, and a citation next to the name of a
function or class the cited file defines must cite lines that hold that name.
The reference tree is mounted only in the build container; elsewhere the
test is skipped.
"""
import glob
import os
import re

import pytest

REF = "/root/reference"
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

pytestmark = pytest.mark.skipif(not os.path.isdir(REF), reason="reference tree not mounted")

PATTERNS = ["include/*.h", "DESIGN.md", "INTEGRATION.md", "README.md", "oracle/*.c", "oracle/*.cpp",
            "oracle/*.py", "sparse-computation_amd/**/*.py", "sparse-computation_amd/**/*.hip",
            "sparse-computation_amd/**/*.hpp", "sparse-computation_amd/**/*.cpp",
            "sparse-computation_amd/**/*.sh", "tests/*.py", "bench.py", "__graft_entry__.py"]
CITE = re.compile(r"([A-Za-z0-9_./-]+\.(?:py|cpp|h|cu|cuh|sh|txt|hpp|c)):(\d+)(?:-(\d+))?")


def _sources():
    out = set()
    for pat in PATTERNS:
        for f in glob.glob(os.path.join(ROOT, pat), recursive=True):
            if "/gen/" not in f and "/gen_units/" not in f:
                out.add(f)
    return sorted(out)


_lines = {}


def _ref_lines(path):
    cands = [os.path.join(REF, path)] + glob.glob(os.path.join(REF, "**", os.path.basename(path)),
                                                    recursive=True)
    real = next((c for c in cands if os.path.isfile(c) and c.endswith(path)), None)
    if real is None:
        return None, None
    if real not in _lines:
        with open(real, errors="replace") as f:
            _lines[real] = f.read().splitlines()
    return real, _lines[real]


_defs = {}


def _defined_names(real, lines):
    if real not in _defs:
        txt = "\n".join(lines)
        names = set(re.findall(r"^\s*(?:def|class|struct)\s+(\w+)", txt, re.M))
        if not real.endswith(".py"):
            names |= set(re.findall(r"^[A-Za-z_][\w:<>,\s*&]*?\b([A-Za-z_]\w*)\s*\([^;]*$", txt, re.M))
        _defs[real] = names - {"if", "for", "while", "switch", "return", "main"}
    return _defs[real]


def test_reference_citations_point_at_real_lines():
    out_of_range, wrong = [], []
    for f in _sources():
        with open(f, errors="replace") as fh:
            text = fh.read().splitlines()
        for ln, line in enumerate(text, 1):
            for m in CITE.finditer(line):
                real, lines = _ref_lines(m.group(1))
                if real is None:
                    continue
                a, b = int(m.group(2)), int(m.group(3) or m.group(2))
                where = (os.path.relpath(f, ROOT), ln, m.group(0))
                if a < 1 or a > b or b > len(lines):
                    out_of_range.append(where + (len(lines),))
                    continue
                # names the cited file defines, mentioned on this line or the
                # two before it (comments wrap), must appear in the cited lines
                ctx = " ".join(text[max(0, ln - 3):ln])
                named = set(re.findall(r"[A-Za-z_]\w*", ctx)) & _defined_names(real, lines)
                if named:
                    seg = "\n".join(lines[a - 1:b])
                    if not any(re.search(r"\b%s\b" % re.escape(n), seg) for n in named):
                        wrong.append(where + (sorted(named),))
    assert not out_of_range, out_of_range
    assert not wrong, wrong


def test_boundary_loader_citations():
    # the drop-in loaders of include/Sparse_io.h, as the C ABI cites them
    _, lines = _ref_lines("utils/Sparse_io.cpp")
    with open(os.path.join(ROOT, "include", "sc_api.h")) as f:
        hdr = f.read()
    for name, rng in (("loadCfmtxMatrices", "186-196"), ("readCSRMatrix", "198-206"),
                      ("readCompressedFormatMatrix", "208-215"), ("companionMtxPathFromCFMTX", "28-46"),
                      ("readCFMTXFile", "84-182"), ("readCSRMatrixFromMTX", "48-82")):
        a, b = map(int, rng.split("-"))
        assert re.search(r"\b%s\b" % name, lines[a - 1]), (name, lines[a - 1])
        assert f"Sparse_io.cpp:{rng}" in hdr or f":{rng}" in hdr, name
