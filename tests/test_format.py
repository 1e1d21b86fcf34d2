"""Product host path (libsc through sc_amd) against the pinned oracle, the
reference's fixtures and the golden vectors: .mtx reading, pattern
enumeration, the .cfmtx builder/writer (byte-exact), the reader, the
companion-path rule, value text, the seeded synthetic inputs and the errors
the C ABI reports.  CPU only."""
import glob
import itertools
import json
import math
import os
import random
import struct

import numpy as np
import pytest

import oracle as O
import sc_amd
from conftest import FIXTURE_STEM, REF_MATRICES

HERE = os.path.dirname(os.path.abspath(__file__))
GOLDEN = os.path.join(HERE, "golden")
FIX_MTX = os.path.join(REF_MATRICES, FIXTURE_STEM + ".mtx")
needs_ref = pytest.mark.skipif(not os.path.exists(FIX_MTX), reason="reference tree not mounted")


def golden_cases():
    with open(os.path.join(GOLDEN, "manifest.json")) as f:
        return [c for c in json.load(f) if "cfmtx" in c]


def csr_of_dense(d):
    ip = np.concatenate([[0], np.cumsum((d != 0).sum(1))]).astype(np.int32)
    ix = np.nonzero(d)[1].astype(np.int32)
    return ip, ix, d[d != 0].astype(np.float64)


def product_text(ip, ix, dx, m, n, km, kn, dictionary=None):
    A = sc_amd.Csr.from_arrays(m, n, ip, ix, dx)
    return sc_amd.Cfmtx.build(A, km, kn, dictionary).text()


def oracle_text(ip, ix, dx, m, n, km, kn, dictionary=None):
    pats = O.read_pattern_dictionary(dictionary) if dictionary else O.patterns_map(km, 1)
    return O.cfmtx_text(O.build(m, n, ip, ix, dx, km, kn, pats), pats)


# ---------------------------------------------------------------- patterns

@pytest.mark.parametrize("km,kn", [(1, 1), (2, 1), (3, 1), (4, 1), (5, 1), (6, 1), (2, 2), (3, 2)])
def test_pattern_enumeration_matches_oracle(km, kn):
    mine = sc_amd.patterns(km, kn)
    ora = ["".join("1" if b else "0" for b in k) for k in O.patterns_map(km, kn)]
    assert mine == ora


def test_python_pattern_dictionary_module():
    import pattern_utiles.pattern_dictionary as pd
    for km in range(1, 7):
        d = pd.generate_pattern_dictionary(km, 1)
        assert list(d.id_to_patten_bin.values()) == sc_amd.patterns(km, 1)
        assert pd.build_patterns_map(km, 1) == O.patterns_map(km, 1)
        assert all(d.pattern_id_to_number_of_nnz(i) == b.count("1")
                   for i, b in d.id_to_patten_bin.items())
    dpath = os.path.join(GOLDEN, "cfmtx", "dict4_sub.txt")
    d = pd.read_pattern_dictionary(dpath)
    assert d.id_to_patten_bin == {0: "1111", 1: "1000", 2: "0100", 3: "0010", 4: "0001", 5: "1100"}


# ---------------------------------------------------------------- builder

@needs_ref
def test_product_reproduces_every_reference_fixture():
    A = sc_amd.Csr.from_mtx(FIX_MTX)
    files = sorted(glob.glob(os.path.join(REF_MATRICES, FIXTURE_STEM + "-*.cfmtx")))
    files.append(os.path.join(REF_MATRICES, FIXTURE_STEM + ".cfmtx"))
    assert len(files) == 47
    for f in files:
        km, kn = (6, 8) if f.endswith("connected.cfmtx") else map(
            int, os.path.basename(f)[:-6].split("-")[-2:])
        with open(f) as fh:
            assert sc_amd.Cfmtx.build(A, km, kn).text() == fh.read(), f


@pytest.mark.parametrize("case", golden_cases(), ids=lambda c: c["tag"])
def test_product_reproduces_reference_cli_golden(case):
    A = sc_amd.Csr.from_mtx(os.path.join(GOLDEN, "cfmtx", case["mtx"]))
    d = os.path.join(GOLDEN, "cfmtx", case["dictionary"] + ".txt") if case["dictionary"] else None
    with open(os.path.join(GOLDEN, "cfmtx", case["cfmtx"])) as f:
        assert sc_amd.Cfmtx.build(A, case["km"], case["kn"], d).text() == f.read()


def test_builder_matches_oracle_on_random_matrices():
    rng = np.random.default_rng(7)
    shapes = [(1, 1), (1, 9), (9, 1), (3, 5), (7, 7), (13, 31), (40, 17), (64, 64), (5, 200)]
    for (m, n), density in itertools.product(shapes, [0.05, 0.3, 0.8, 1.0]):
        d = (rng.random((m, n)) < density) * rng.standard_normal((m, n))
        d = d.astype(np.float32).astype(np.float64)
        if m > 2:
            d[m // 2] = 0  # an empty row
        ip, ix, dx = csr_of_dense(d)
        for km in range(1, 7):
            for kn in (0, 1, 2, 3, 8):
                assert product_text(ip, ix, dx, m, n, km, kn) == oracle_text(ip, ix, dx, m, n, km, kn), \
                    (m, n, density, km, kn)


def test_builder_matches_oracle_in_dictionary_mode(tmp_path):
    rng = np.random.default_rng(8)
    d = (rng.random((29, 41)) < 0.3) * rng.standard_normal((29, 41))
    ip, ix, dx = csr_of_dense(d)
    for trial in range(12):
        km = int(rng.integers(2, 6))
        allbits = sc_amd.patterns(km, 1)
        chosen = list(rng.choice(len(allbits), size=int(rng.integers(1, len(allbits) + 1)),
                                 replace=False))
        ids = list(range(len(chosen)))
        rng.shuffle(ids)
        path = tmp_path / f"d{trial}.txt"
        with open(path, "w") as f:
            f.write(f"{km} 1 {len(chosen)}\n")
            for b, i in zip(chosen, ids):
                f.write(f"{allbits[b]} {i}\n")
        for kn in (0, 1, 3):
            assert product_text(ip, ix, dx, 29, 41, km, kn, str(path)) == \
                oracle_text(ip, ix, dx, 29, 41, km, kn, str(path))


def decode(cf):
    """.cfmtx -> {(row, col): value} of the real (non-padding) slots."""
    info = cf.info()
    out = {}
    for p in cf.patterns():
        rows = [r for r, ch in enumerate(p["bits"]) if ch == "1"]
        pop = len(rows)
        rpp = p["rpp"]
        for panel in range(info["npanels"]):
            seen = set()
            for j in range(rpp[panel], rpp[panel + 1]):
                c = int(p["cb"][j])
                if c in seen:  # padding repeats the last column with zero values
                    assert all(p["vals"][j * pop + k] == 0 for k in range(pop))
                    continue
                seen.add(c)
                for k, r in enumerate(rows):
                    out[(panel * info["km"] + r, c)] = float(p["vals"][j * pop + k])
    return out


def test_brute_force_round_trip_all_small_masks():
    """Every 0/1 pattern of a km x w block decodes back to the input."""
    for km, w in [(1, 4), (2, 3), (3, 3), (4, 3), (5, 2)]:
        for bits in range(1 << (km * w)):
            d = np.array([(bits >> i) & 1 for i in range(km * w)], np.float64).reshape(km, w)
            d = d * (1 + np.arange(km * w).reshape(km, w))  # distinct values
            ip, ix, dx = csr_of_dense(d)
            A = sc_amd.Csr.from_arrays(km, w, ip, ix, dx)
            for kn in (1, 2):
                got = decode(sc_amd.Cfmtx.build(A, km, kn))
                want = {(int(r), int(c)): float(d[r, c]) for r, c in zip(*np.nonzero(d))}
                assert got == want


def test_format_invariants():
    A = sc_amd.Csr.synth_uniform(103, 211, 0.2, 0.05, 5)
    for km, kn in [(4, 1), (3, 5), (6, 8), (2, 0)]:
        cf = sc_amd.Cfmtx.build(A, km, kn)
        info = cf.info()
        assert info["npanels"] == -(-103 // km)
        real = 0
        for p in cf.patterns():
            pack = kn if kn else 32 // p["pop"]
            rpp = p["rpp"]
            assert len(rpp) == info["npanels"] + 1 and rpp[0] == 0
            seg = np.diff(rpp)
            assert np.all(seg >= 0) and np.all(seg % pack == 0)
            assert len(p["vals"]) == len(p["cb"]) * p["pop"]
            for q in range(info["npanels"]):
                cols = p["cb"][rpp[q]:rpp[q + 1]]
                if len(cols):
                    assert cols[-1] == cols.max()  # padding repeats the segment maximum
                    assert np.all(np.diff(cols) >= 0)
            real += int(np.count_nonzero(p["vals"]))
        assert real == A.nnz


# ---------------------------------------------------------------- value text

def _repr_cases():
    vals = [0.0, -0.0, 1.0, -1.0, 0.1, 1e-4, 9.999e-5, 1e-5, 1e16, 9999999999999998.0, 1e15,
            123456789012345.6, 5e-324, 1.7976931348623157e308, 2.0 ** -1074 * 3, 0.5, 100.0,
            1e22, 1.5e-7, 3.14159, float(np.float32(0.1)), 2.0 ** 52, 2.0 ** 53 + 2]
    rnd = random.Random(3)
    for _ in range(3000):
        vals.append(struct.unpack("<d", struct.pack("<Q", rnd.getrandbits(64)))[0])
        vals.append(float(np.float32(rnd.gauss(0, 0.05))))
        vals.append(rnd.uniform(-1e-3, 1e-3))
    return [v for v in vals if math.isfinite(v)]


def test_value_text_is_python_repr():
    vals = _repr_cases()
    n = len(vals)
    A = sc_amd.Csr.from_arrays(1, n, [0, n], np.arange(n, dtype=np.int32), np.array(vals))
    text = sc_amd.Cfmtx.build(A, 1, 1).text()
    tokens = text.splitlines()[-1].split()
    assert tokens == [repr(v) for v in vals]


def test_numpy_float64_str_is_python_repr():
    """format_generator.py prints str(np.float64); the writer prints repr."""
    for v in _repr_cases()[:2000]:
        assert str(np.float64(v)) == repr(v)


# ---------------------------------------------------------------- readers

def test_reader_matches_oracle_reader(tmp_path):
    files = [os.path.join(GOLDEN, "cfmtx", c["cfmtx"]) for c in golden_cases()]
    A = sc_amd.Csr.synth_uniform(50, 70, 0.3, 1e-3, 9)
    for km, kn in [(4, 1), (5, 3)]:
        p = str(tmp_path / f"s-{km}-{kn}.cfmtx")
        sc_amd.Cfmtx.build(A, km, kn).write(p)
        files.append(p)
    for f in files:
        mine = sc_amd.Cfmtx.read(f)
        ref = O.read_cfmtx(f)
        info = mine.info()
        assert (info["m"], info["n"], info["km"], info["npat"]) == \
            (ref["num_rows"], ref["num_columns"], ref["kernel_rows"], ref["num_patterns"])
        for i, p in enumerate(mine.patterns()):
            assert p["pop"] == ref["pop"][i]
            assert np.array_equal(p["rpp"], ref["rpp"][i])
            assert np.array_equal(p["cb"], ref["cb"][i])
            assert np.array_equal(p["vals"].view(np.uint32), ref["nnz"][i].view(np.uint32))


@needs_ref
def test_reader_and_csr_loader_match_reference_loaders():
    if not O.ref_dump_available():
        pytest.skip("oracle/_ref not built")
    f = os.path.join(REF_MATRICES, FIXTURE_STEM + "-4-2.cfmtx")
    csr, cf = sc_amd.load_cfmtx_matrices(f)
    ref = O.ref_read_cfmtx(f)
    for i, p in enumerate(cf.patterns()):
        assert np.array_equal(p["rpp"], ref[i]["rpp"])
        assert np.array_equal(p["rpp"] * p["pop"], ref[i]["npp"])
        assert np.array_equal(p["cb"], ref[i]["cb"])
        assert np.array_equal(p["vals"], ref[i]["vals"])
    rc = O.ref_read_csr(f)
    ip, ix, dx = csr.arrays()
    assert csr.shape == (rc["m"], rc["n"]) and csr.nnz == rc["nnz"]
    assert np.array_equal(ip, rc["p"]) and np.array_equal(ix, rc["i"])
    assert np.array_equal(dx, rc["x"])


def test_built_values_equal_what_the_reader_gets(tmp_path):
    """The plan takes fp32 values from the built format; they must equal the
    reader's strtof of the written text, value for value."""
    vals = np.array(_repr_cases()[:600])
    vals = vals[np.abs(vals) < 3e38]
    n = len(vals)
    A = sc_amd.Csr.from_arrays(1, n, [0, n], np.arange(n, dtype=np.int32), vals)
    cf = sc_amd.Cfmtx.build(A, 1, 1)
    p = str(tmp_path / "v-1-1.cfmtx")
    cf.write(p)
    assert np.array_equal(cf.pattern(0)["vals"].view(np.uint32),
                          sc_amd.Cfmtx.read(p).pattern(0)["vals"].view(np.uint32))


@pytest.mark.parametrize("name", ["real_17x23", "integer_13x9", "pattern_11x14", "symmetric_12",
                                  "duplicates_9x10"])
def test_mtx_reader_matches_scipy(name):
    path = os.path.join(GOLDEN, "cfmtx", name + ".mtx")
    M, K, ip, ix, data, _ = O.mtx_to_csr(path)
    A = sc_amd.Csr.from_mtx(path)
    mip, mix, mdx = A.arrays()
    assert A.shape == (M, K)
    assert np.array_equal(mip, ip) and np.array_equal(mix, ix)
    assert np.array_equal(mdx, data.astype(np.float64))


def test_mtx_write_read_round_trip(tmp_path):
    A = sc_amd.Csr.synth_uniform(31, 47, 0.2, 0.05, 3)
    p = str(tmp_path / "a.mtx")
    A.write_mtx(p)
    B = sc_amd.Csr.from_mtx(p)
    for a, b in zip(A.arrays(), B.arrays()):
        assert np.array_equal(a, b)
    M, K, ip, ix, data, _ = O.mtx_to_csr(p)
    assert np.array_equal(ix, A.arrays()[1]) and np.array_equal(data, A.arrays()[2])


def test_companion_path_rule():
    cases = {
        "a/b/matrix-4-8.cfmtx": "a/b/matrix.mtx",
        "matrix-64-128.cfmtx": "matrix.mtx",
        "my-matrix-4-1.cfmtx": "my-matrix.mtx",
        "matrix.cfmtx": "matrix.mtx",
        "-4.cfmtx": "-4.mtx",
        "x-4.cfmtx": "x-4.mtx",
        ".cfmtx": ".cfmtx",
    }
    for src, want in cases.items():
        assert sc_amd.companion_mtx_path(src) == want, src


# ---------------------------------------------------------------- synthetic

def _splitmix_xoshiro(seed, count):
    M64 = (1 << 64) - 1
    x = seed
    s = []
    for _ in range(4):
        x = (x + 0x9E3779B97F4A7C15) & M64
        z = x
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M64
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M64
        s.append(z ^ (z >> 31))

    def rotl(v, k):
        return ((v << k) | (v >> (64 - k))) & M64

    out = []
    for _ in range(count):
        out.append((rotl((s[1] * 5) & M64, 7) * 9) & M64)
        t = (s[1] << 17) & M64
        s[2] ^= s[0]
        s[3] ^= s[1]
        s[1] ^= s[2]
        s[0] ^= s[3]
        s[2] ^= t
        s[3] = rotl(s[3], 45)
    return out


def test_rng_matches_published_algorithm():
    for seed in (0, 1, 0x5EED0000, 2 ** 63 + 5):
        assert list(sc_amd.synth_raw(seed, 64)) == _splitmix_xoshiro(seed, 64)


def test_synthetic_matrices_are_exact_and_deterministic():
    A = sc_amd.Csr.synth_uniform(512, 512, 0.30, 0.05, 0x5EED0000)
    assert A.nnz == round(0.30 * 512 * 512) == 78643
    ip, ix, dx = A.arrays()
    assert np.all(dx != 0) and np.array_equal(dx, dx.astype(np.float32).astype(np.float64))
    assert abs(np.std(dx) - 0.05) < 0.002
    for r in range(512):
        assert np.all(np.diff(ix[ip[r]:ip[r + 1]]) > 0)
    A2 = sc_amd.Csr.synth_uniform(512, 512, 0.30, 0.05, 0x5EED0000)
    assert all(np.array_equal(a, b) for a, b in zip(A.arrays(), A2.arrays()))
    S = sc_amd.Csr.synth_blocks(256, 256, 0.10, 0.05, 4)
    target = round(0.10 * 256 * 256)
    assert target <= S.nnz <= target + 15
    B = sc_amd.synth_dense(10000, 1)
    assert B.min() >= -1 and B.max() < 1 and np.array_equal(B, np.round(B * 2 ** 23) / 2 ** 23)


def test_structured_blocks_are_aligned_vectors_and_blocks():
    S = sc_amd.Csr.synth_blocks(64, 128, 0.15, 0.05, 11)
    ip, ix, _ = S.arrays()
    d = np.zeros((64, 128), bool)
    for r in range(64):
        d[r, ix[ip[r]:ip[r + 1]]] = True
    # every nonzero belongs to an aligned 8-wide row run or an aligned 4x4 block
    covered = np.zeros_like(d)
    for r in range(64):
        for c0 in range(0, 128, 8):
            if d[r, c0:c0 + 8].all():
                covered[r, c0:c0 + 8] = True
    for r0 in range(0, 64, 4):
        for c0 in range(0, 128, 4):
            if d[r0:r0 + 4, c0:c0 + 4].all():
                covered[r0:r0 + 4, c0:c0 + 4] = True
    assert np.array_equal(covered, d)


# ---------------------------------------------------------------- errors

def test_errors_are_reported_not_thrown(tmp_path):
    E = sc_amd.LibscError
    with pytest.raises(E, match="cannot open"):
        sc_amd.Csr.from_mtx(str(tmp_path / "missing.mtx"))
    bad = tmp_path / "bad.mtx"
    bad.write_text("%%MatrixMarket matrix coordinate complex general\n2 2 1\n1 1 1 0\n")
    with pytest.raises(E, match="unsupported"):
        sc_amd.Csr.from_mtx(str(bad))
    bad.write_text("%%MatrixMarket matrix array real general\n2 2\n1\n2\n3\n4\n")
    with pytest.raises(E, match="coordinate"):
        sc_amd.Csr.from_mtx(str(bad))
    bad.write_text("%%MatrixMarket matrix coordinate real general\n2 2 3\n1 1 1\n")
    with pytest.raises(E, match="truncated"):
        sc_amd.Csr.from_mtx(str(bad))
    with pytest.raises(E, match="Unable to open"):
        sc_amd.Cfmtx.read(str(tmp_path / "none.cfmtx"))
    with pytest.raises(E, match="expects a .cfmtx"):
        sc_amd.load_cfmtx_matrices(str(tmp_path / "x.mtx"))
    A = sc_amd.Csr.synth_uniform(8, 8, 0.5, 1, 1)
    with pytest.raises(E, match="kernel_n"):
        sc_amd.Cfmtx.build(A, 4, -1)
    with pytest.raises(E, match="kernel_m"):
        sc_amd.Cfmtx.build(A, 0, 1)
    with pytest.raises(E, match="sorted and unique"):
        sc_amd.Csr.from_arrays(1, 4, [0, 2], [2, 1], [1.0, 2.0])
        sc_amd.Cfmtx.build(sc_amd.Csr.from_arrays(1, 4, [0, 2], [2, 1], [1.0, 2.0]), 1, 1)
    zero_pat = tmp_path / "zero.txt"
    zero_pat.write_text("2 1 2\n00 0\n11 1\n")
    with pytest.raises(E, match="no ones"):
        sc_amd.Cfmtx.build(A, 2, 1, str(zero_pat))
    long_rpp = tmp_path / "long-1-1.cfmtx"
    long_rpp.write_text("2 2 1 1 1\n1 0 \n0 1 2 3\n0 1 1\n1.0 2.0 3.0\n")
    with pytest.raises(E, match="longer"):
        sc_amd.Cfmtx.read(str(long_rpp))


def _declared(path):
    import re
    with open(path) as f:
        return set(re.findall(r"\b(sc_[a-z0-9_]+)\s*\(", f.read())) - {"sc_gen_launch_fn"}


def test_c_abi_exports_every_declared_symbol():
    root = os.path.dirname(HERE)
    declared = set()
    for h in glob.glob(os.path.join(root, "include", "*.h")):
        if os.path.basename(h) != "sc_vendor.h":
            declared |= _declared(h)
    lib = sc_amd.lib()
    missing = [s for s in sorted(declared) if not hasattr(lib, s)]
    assert not missing, missing
    assert declared <= set(sc_amd.EXPORTS)


def test_python_plan_flags_match_the_header():
    import re
    text = open(os.path.join(os.path.dirname(HERE), "include", "sc_api.h")).read()
    defs = {m.group(1): int(m.group(2)) for m in re.finditer(r"#define SC_(PLAN_\w+|ACCUMULATE) (\d+)", text)}
    assert {"PLAN_DROP_PADDING", "PLAN_TILED", "PLAN_CHUNKED", "PLAN_F16_VALUES", "PLAN_ROWS",
            "PLAN_PATTERNS", "ACCUMULATE"} <= set(defs)
    for name, value in defs.items():
        assert getattr(sc_amd, name) == value, name
    plan_bits = [v for k, v in defs.items() if k.startswith("PLAN_")]
    assert len(set(plan_bits)) == len(plan_bits) and all(v & (v - 1) == 0 for v in plan_bits)


def test_vendor_library_exports_every_declared_symbol():
    from sc_amd import vendor
    declared = _declared(os.path.join(os.path.dirname(HERE), "include", "sc_vendor.h"))
    assert len(declared) == 7
    lib = vendor.vlib()
    missing = [s for s in sorted(declared) if not hasattr(lib, s)]
    assert not missing, missing


class _FakeDeviceTensor:
    """Stands in for a tensor on cuda:<index> in a process without a GPU: the
    operand checks of sc_amd.Plan read only these attributes."""

    def __init__(self, shape, dtype, cuda=True, index=0):
        import torch
        self.shape = shape
        self.dtype = dtype
        self.is_cuda = cuda
        self.device = torch.device(f"cuda:{index}") if cuda else torch.device("cpu")

    def dim(self):
        return len(self.shape)

    def numel(self):
        n = 1
        for s in self.shape:
            n *= s
        return n

    def is_contiguous(self):
        return True

    def data_ptr(self):  # a launch would need it: the checks must raise first
        raise AssertionError("operand checks let a launch through")


def _bare_plan(m, k):
    p = object.__new__(sc_amd.Plan)
    p._h = None
    p.device = 0
    p.info = lambda: {"m": m, "n": k}
    return p


def test_plan_rejects_host_or_foreign_operands_before_launch():
    import torch
    p = _bare_plan(8, 6)
    B16 = _FakeDeviceTensor((6, 4), torch.float16)
    # binary16 path: C on the host, or on another device than the plan's
    with pytest.raises(ValueError, match="C must"):
        p.spmm_f16(B16, torch.empty((8, 4), dtype=torch.float16))
    with pytest.raises(ValueError, match="plan's device"):
        p.spmm_f16(B16, _FakeDeviceTensor((8, 4), torch.float16, index=1))
    with pytest.raises(ValueError, match="plan's device"):
        p.spmm_f16(_FakeDeviceTensor((6, 4), torch.float16, index=1))
    # fp32 path: the same checks
    B32 = _FakeDeviceTensor((6, 4), torch.float32)
    with pytest.raises(ValueError, match="C must"):
        p.spmm(B32, torch.empty((8, 4), dtype=torch.float32))
    with pytest.raises(ValueError, match="plan's device"):
        p.spmm(B32, _FakeDeviceTensor((8, 4), torch.float32, index=1))
    with pytest.raises(ValueError, match="x must"):
        p.spmv(torch.empty(6, dtype=torch.float32))


def test_committed_reference_matrix_is_the_reference_file(reference_matrix_dir):
    # the gzipped copies under tests/golden/reference_matrix are the
    # reference's own fixture files byte for byte
    from conftest import GOLDEN_FILES
    if not os.path.isdir(REF_MATRICES):
        pytest.skip("reference tree not mounted")
    for name in GOLDEN_FILES:
        with open(os.path.join(REF_MATRICES, name), "rb") as a, \
                open(os.path.join(reference_matrix_dir, name), "rb") as b:
            assert a.read() == b.read(), name
    # and the unpacked pair loads like the reference's loader does
    A, cf = sc_amd.load_cfmtx_matrices(os.path.join(reference_matrix_dir, FIXTURE_STEM + "-4-2.cfmtx"))
    assert A.shape == (512, 512) and A.nnz == 104857
    built = sc_amd.Cfmtx.build(sc_amd.Csr.from_mtx(os.path.join(reference_matrix_dir, FIXTURE_STEM + ".mtx")), 4, 2)
    with open(os.path.join(reference_matrix_dir, FIXTURE_STEM + "-4-2.cfmtx")) as f:
        assert built.text() == f.read()
