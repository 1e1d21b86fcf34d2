"""Emit gfx950 HIP for the pattern kernels.

One call produces one translation unit for a row coarsen factor ``km`` and a
pattern dictionary:

* one straight-line ``__device__`` body per pattern -- the panel rows of the
  pattern are literal indices into the accumulator tile, the ``kn`` slots of a
  pack are unrolled (``kn`` B-row loads, ``pop * kn`` value loads and
  ``pop * kn`` FMA rows per step); the lanes-over-slots body is templated on
  where its B rows come from (global memory for the panel kernel, an LDS
  chunk of B for the chunk kernel);
* a dispatcher whose ``switch`` maps a segment's row mask to its body;
* an ``extern "C"`` launcher ``sc_gen_<name>_launch`` and a parameter record
  ``sc_gen_<name>_record`` (km, kn, waves, patterns, N variant, masks), so a
  plan built for other parameters is rejected rather than mis-computed.

The building blocks (lane mapping, B loads, wave64 reductions, the panel
kernel) are hand-written in ``csrc/sc_kernels.hpp``; this module writes what
the reference's generators write per pattern
(code_gen/spmm/spmm_format_code_generator.py:74-223,
code_gen/spmm_small_b_col/spmm_small_b_col_format_code_generator.py:4-323,
code_gen/spmv/spmv_format_code_generator.py:4-213), for wave64 rather than
warp32.
"""
from __future__ import annotations

import re

KINDS = ("spmm", "spmm_small_b_col", "spmv")


def _rows(bits: str):
    return [r for r, ch in enumerate(bits) if ch == "1"]


def _mask(bits: str) -> int:
    return sum(1 << r for r in _rows(bits))


def body_name(bits: str) -> str:
    return f"pattern_{bits}"


def _narrow_loop(kn: int, unroll: int, step, indent="  "):
    """Lanes-over-slots slot loop over the range [a.lo, a.hi) of a segment.

    The segment's packs go to the S lane groups in one of two ways, chosen by
    the argument type (A::kBlocked); either way group s gets q or q + 1 of
    them (q = packs / S, the first `packs mod S` groups one more):

    * blocked -- a contiguous block per group: the packs of a batch are
      adjacent, so their columns and values sit at constant offsets from one
      address;
    * interleaved -- group s takes packs s, s + S, s + 2S, ... (adjacent lanes
      read adjacent slots: one cache line for a read of columns from memory,
      no LDS bank conflicts for one lane per slot).

    Batches of `unroll` packs per group (their B loads all in flight), counted
    the same for the whole wave, then one last batch of exactly the packs
    left (1 .. unroll; a group with one pack fewer reads zeros for it), so a
    segment costs ceil(packs / unroll) round trips and issues no load beyond
    its longest group.  `step(u, masked, ind)` writes pack u of a batch (slot
    j{u})."""
    U = unroll
    i2 = indent + "  "
    i3 = indent + "    "
    out = [f"{indent}const int np = (a.hi - a.lo) / {kn};",
           f"{indent}const int sh = __builtin_ctz((unsigned)a.S);",
           f"{indent}const int q = np >> sh;",
           f"{indent}const int r = np & (a.S - 1);",
           f"{indent}const int cnt = q + (a.s < r ? 1 : 0);",
           f"{indent}const int jb = A::kBlocked ? a.lo + (a.s * q + min(a.s, r)) * {kn} : a.lo + a.s * {kn};",
           f"{indent}const int stride = A::kBlocked ? {kn} : a.S * {kn};",
           f"{indent}int b = 0;",
           f"{indent}for (; b + {U} <= q; b += {U}) {{",
           f"{i2}const int j = jb + b * stride;"]
    for u in range(U):
        out.append(f"{i2}const int j{u} = j + {u} * stride;")
    for u in range(U):
        out += step(u, False, i2)
    out += [f"{indent}}}",
            f"{indent}const int rem = q + (r > 0 ? 1 : 0) - b;  // 0 .. {U}",
            f"{indent}if (rem > 0) {{",
            f"{i2}const int j = jb + b * stride;"]
    for t in range(1, U + 1):
        if U == 1:
            out.append(f"{i2}{{")
        elif t == 1:
            out.append(f"{i2}if (rem == 1) {{")
        elif t < U:
            out.append(f"{i2}}} else if (rem == {t}) {{")
        else:
            out.append(f"{i2}}} else {{")
        for u in range(t):
            out.append(f"{i3}const bool ok{u} = b + {u} < cnt;")
            out.append(f"{i3}const int j{u} = ok{u} ? j + {u} * stride : a.lo;")
        for u in range(t):
            out += step(u, True, i3)
    out.append(f"{i2}}}")
    out.append(f"{indent}}}")
    return out


def _narrow_step(kn, pop, fmas):
    """Pack u of a narrow batch: kn B-row loads and pop * kn values; a masked
    pack (past the segment) loads a zero row and zero values."""
    def step(u, masked, ind):
        out = [f"{ind}const float *vp{u} = a.vals + a.vb + (j{u} - a.sb) * {pop};"]
        for q in range(kn):
            out.append(f"{ind}float b{u}_{q}[V];")
            if masked:
                out.append(f"{ind}sc::load_b_tail<V>(b{u}_{q}, a, a.cols[j{u} + {q}], ok{u});")
            else:
                out.append(f"{ind}sc::load_b<V>(b{u}_{q}, a, a.cols[j{u} + {q}]);")
        # a masked pack's slot index is clamped into the segment, so its
        # values are read unconditionally (no branch) and then cleared
        def value(q):
            def at(k):
                e = f"vp{u}[{q * pop + k}]" if isinstance(k, int) else f"vp{u}[{q * pop} + {k}]"
                return f"sc::keep_if(ok{u}, {e})" if masked else e
            return at
        return out, [(q, value(q)) for q in range(kn)]

    def emit(u, masked, ind):
        loads, vals = step(u, masked, ind)
        return loads + fmas(u, vals, ind)
    return emit


def emit_body(km: int, bits: str, pid: int, kn: int, unroll: int) -> str:
    rows = _rows(bits)
    pop = len(rows)
    out = []
    out.append(f"// pattern id {pid}: bits {bits} -> panel rows {', '.join(map(str, rows))} "
               f"(pop {pop}), packs of {kn} slot(s), {unroll} pack(s) per lane in flight")
    out.append("template <int V, class A>")
    out.append(f"__device__ __forceinline__ void {body_name(bits)}(float (&acc)[{km}][V], "
               "const A &a) {")

    def fmas(u, vals, ind):
        res = []
        for q, value in vals:
            for k in range(pop):
                res.append(f"{ind}const float v{u}_{q}_{k} = {value(k)};")
        for q, _ in vals:
            for k, r in enumerate(rows):
                res.append(f"{ind}sc::fma_row<V>(acc[{r}], v{u}_{q}_{k}, b{u}_{q});")
        return res
    out += _narrow_loop(kn, unroll, _narrow_step(kn, pop, fmas))
    out.append("}")
    return "\n".join(out)


def wide_name(bits: str) -> str:
    return f"wide_{bits}"


def _wide_step(rows, pop, slots, indent, loader="sc::load_row"):
    """Straight-line code for `slots` consecutive slots starting at j."""
    out = [f"{indent}const float *vp = a.vals + a.vb + (j - a.sb) * {pop};"]
    for q in range(slots):
        out.append(f"{indent}const int c{q} = a.cols[j + {q}];")
    for q in range(slots):
        out.append(f"{indent}float b{q}[V];")
        out.append(f"{indent}{loader}<V>(b{q}, a, c{q});")
    for q in range(slots):
        for k in range(pop):
            out.append(f"{indent}const float v{q}_{k} = vp[{q * pop + k}];")
    for q in range(slots):
        for k, r in enumerate(rows):
            out.append(f"{indent}sc::fma_row<V>(acc[{r}], v{q}_{k}, b{q});")
    return out


def emit_wide_body(km: int, bits: str, pid: int, kn: int, unroll_slots: int = 8) -> str:
    """Wide-path body: the whole wave shares each slot; full batches of
    `unroll_slots` (a multiple of kn) B-row loads in flight, then the
    remainder of the wave's range in power-of-two batches (4, 2, 1 packs for
    8 slots), so a segment tail costs at most three round trips instead of
    one per pack, with no loads or FMAs spent on slots past the end."""
    rows = _rows(bits)
    pop = len(rows)
    U = kn * max(1, -(-unroll_slots // kn))
    out = [f"// pattern id {pid}: bits {bits} -> panel rows {', '.join(map(str, rows))} "
           f"(pop {pop}); wave-wide slots, {U} per step",
           "template <int V>",
           f"__device__ __forceinline__ void {wide_name(bits)}(float (&acc)[{km}][V], "
           "const sc::WideArgs &a) {",
           "  int j = a.lo;",
           f"  if (j + {U} <= a.hi) {{"]
    for q in range(U):
        out.append(f"    int c{q} = a.cols[j + {q}];")
    out.append("    for (;;) {")
    for q in range(U):
        out.append(f"      float b{q}[V];")
        out.append(f"      sc::load_row<V>(b{q}, a, c{q});")
    out.append(f"      const float *vp = a.vals + a.vb + (j - a.sb) * {pop};")
    for q in range(U):
        for k in range(pop):
            out.append(f"      const float v{q}_{k} = vp[{q * pop + k}];")
    out.append(f"      const bool more = j + {2 * U} <= a.hi;")
    out.append("      if (more) {")
    for q in range(U):
        out.append(f"        c{q} = a.cols[j + {U + q}];")
    out.append("      }")
    for q in range(U):
        for k, r in enumerate(rows):
            out.append(f"      sc::fma_row<V>(acc[{r}], v{q}_{k}, b{q});")
    out.append(f"      j += {U};")
    out.append("      if (!more) break;")
    out.append("    }")
    out.append("  }")
    # the remainder (< U slots) in power-of-two batches: at most log2(U/kn)+1
    # round trips and no wasted loads or FMAs
    packs = U // kn
    t = 1
    while t * 2 < packs:
        t *= 2
    while t >= 1:
        out.append(f"  if (j + {t * kn} <= a.hi) {{")
        out += _wide_step(rows, pop, t * kn, "    ")
        out.append(f"    j += {t * kn};")
        out.append("  }")
        t //= 2
    out.append("}")
    return "\n".join(out)


def tile_name(bits: str) -> str:
    return f"tile_{bits}"


def _tile_step(rows, pop, slots, indent, fmas=None):
    """Straight-line code for `slots` consecutive slots of a tile sub-segment
    starting at slot j, values at vp.  The batch's values are read from LDS
    once, one per lane, and each is moved to a scalar register with readlane
    (a wave-wide broadcast read per value would cost the LDS as much as a B
    row); the columns are read wave-wide, then the B rows, then the FMAs."""
    out = []
    if fmas is None:
        nv = slots * pop
        out.append(f"{indent}const float vl = sc::batch_values(vp, {nv});")
        for q in range(slots):
            for k in range(pop):
                out.append(f"{indent}const float v{q}_{k} = sc::lane_value(vl, {q * pop + k});")
    for q in range(slots):
        out.append(f"{indent}const int c{q} = a.cols[j + {q}];")
    for q in range(slots):
        out.append(f"{indent}float b{q}[V];")
        out.append(f"{indent}sc::load_tile<V>(b{q}, a, c{q});")
    if fmas is None:
        for q in range(slots):
            for k, r in enumerate(rows):
                out.append(f"{indent}sc::fma_row<V>(acc[{r}], v{q}_{k}, b{q});")
    else:
        for q in range(slots):
            out += fmas(q, indent)
    return out


def _tile_loop(pop, unroll_slots, step):
    """Full batches of `unroll_slots` slots, then the remainder in
    power-of-two batches (4, 2, 1 for 8): no loads or FMAs past the end."""
    U = unroll_slots
    out = ["  int j = a.lo;",
           "  auto vp = a.vals + a.vb;",
           f"  for (; j + {U} <= a.hi; j += {U}, vp += {U * pop}) {{"]
    out += step(U, "    ")
    out.append("  }")
    t = U // 2
    while t >= 1:
        out.append(f"  if (j + {t} <= a.hi) {{")
        out += step(t, "    ")
        out.append(f"    j += {t};")
        out.append(f"    vp += {t * pop};")
        out.append("  }")
        t //= 2
    return out


def emit_tile_body(km: int, bits: str, pid: int, unroll_slots: int = 0) -> str:
    """Tiled-path body: wave-wide slots of one K tile, B rows read from the
    LDS tile, full batches of `unroll_slots` slots and a power-of-two tail.
    By default 8 slots per batch for up to two rows, 4 above: a batch's
    values live in scalar registers (pop per slot)."""
    rows = _rows(bits)
    pop = len(rows)
    if unroll_slots <= 0:
        unroll_slots = 4
    out = [f"// pattern id {pid}: bits {bits} -> panel rows {', '.join(map(str, rows))} "
           f"(pop {pop}); B rows from the LDS tile, {unroll_slots} per step",
           "template <int V>",
           f"__device__ __forceinline__ void {tile_name(bits)}(float (&acc)[{km}][V], "
           "const sc::TileArgs &a) {"]
    out += _tile_loop(pop, unroll_slots, lambda n, ind: _tile_step(rows, pop, n, ind))
    out.append("}")
    return "\n".join(out)


# ---------------------------------------------------------------------------
# Pop-count style (the reference's "nnz based" time-analysis variant,
# code_gen/spmm/spmm_time_analysis.py:73-205): one body per number of rows in
# the pattern instead of one per pattern; the rows a slot feeds are read from
# the segment's mask at run time (wave-uniform flags and value ranks), so the
# unit is smaller and every FMA row sits behind a uniform branch.  Used by
# main_time_analysis.py to compare the two code-generation styles.
# ---------------------------------------------------------------------------
def _mask_rows(km, indent):
    out = []
    for r in range(km):
        out.append(f"{indent}const bool h{r} = (mask & {1 << r}u) != 0;")
        out.append(f"{indent}const int k{r} = __builtin_popcount(mask & {(1 << r) - 1}u);")
    return out


def _generic_fmas(km, pop, q, indent, value):
    return [f"{indent}if (h{r}) sc::fma_row<V>(acc[{r}], {value(q, r)}, b{q});" for r in range(km)]


def _generic_step(km, pop, slots, indent, loader):
    out = [f"{indent}const float *vp = a.vals + a.vb + (j - a.sb) * {pop};"]
    for q in range(slots):
        out.append(f"{indent}float b{q}[V];")
        out.append(f"{indent}{loader}<V>(b{q}, a, a.cols[j + {q}]);")
    for q in range(slots):
        out += _generic_fmas(km, pop, q, indent, lambda q_, r: f"vp[{q_ * pop} + k{r}]")
    return out


def emit_pop_bodies(km: int, pop: int, kn: int, unroll: int, unroll_slots: int = 8) -> str:
    head = f"(float (&acc)[{km}][V], const A &a, unsigned mask)"
    out = [f"// pop-count bodies: {pop} row(s) per slot, rows from the mask"]
    # lanes over slots
    out.append("template <int V, class A>")
    out.append(f"__device__ __forceinline__ void pop{pop}_narrow{head} {{")
    out += _mask_rows(km, "  ")

    def fmas(u, vals, ind):
        res = []
        for q, value in vals:
            for r in range(km):
                res.append(f"{ind}if (h{r}) sc::fma_row<V>(acc[{r}], {value(f'k{r}')}, b{u}_{q});")
        return res
    out += _narrow_loop(kn, unroll, _narrow_step(kn, pop, fmas))
    out.append("}")
    # wave-wide slots
    U = kn * max(1, -(-unroll_slots // kn))
    out.append("template <int V, class A>")
    out.append(f"__device__ __forceinline__ void pop{pop}_wide{head} {{")
    out += _mask_rows(km, "  ")
    out.append("  int j = a.lo;")
    out.append(f"  for (; j + {U} <= a.hi; j += {U}) {{")
    out += _generic_step(km, pop, U, "    ", "sc::load_row")
    out.append("  }")
    packs = U // kn
    t = 1
    while t * 2 < packs:
        t *= 2
    while t >= 1:
        out.append(f"  if (j + {t * kn} <= a.hi) {{")
        out += _generic_step(km, pop, t * kn, "    ", "sc::load_row")
        out.append(f"    j += {t * kn};")
        out.append("  }")
        t //= 2
    out.append("}")
    # LDS tile
    out.append("template <int V, class A>")
    out.append(f"__device__ __forceinline__ void pop{pop}_tile{head} {{")
    out += _mask_rows(km, "  ")
    out += _tile_loop(pop, unroll_slots, lambda n, ind: _tile_step(
        None, pop, n, ind, fmas=lambda q, i2: _generic_fmas(km, pop, q, i2, lambda q_, r: f"vp[{q_ * pop} + k{r}]")))
    out.append("}")
    return "\n".join(out)


def _emit_tile_chain(usable, call):
    """run_tile: the sub-segments of one (K tile, panel) record, in descending
    row-mask order (the plan sorts them so), each run by its pattern's body.
    The patterns are visited in that fixed order by a chain of uniform
    branches, not a multiway switch, so the accumulators stay in place."""
    out = ["  template <int KM, int V>",
           "  __device__ __forceinline__ static void run_tile(const sc::lds_int4 *segs, int d, int d1,",
           "                                                 float (&acc)[KM][V], sc::TileArgs &a) {",
           "    sc::vec4i sd = {0, 0, 0, 0};",
           "    if (d < d1) sd = sc::uniform4(segs[d]);"]
    for bits, pid in sorted(usable, key=lambda bp: -_mask(bp[0])):
        out += [f"    if (sd.x == {_mask(bits)}) {{  // id {pid}",
                "      a.lo = sd.y;",
                "      a.hi = sd.y + sd.z;",
                "      a.vb = sd.w;",
                f"      {call(bits)}",
                "      sd.x = 0;",
                "      if (++d < d1) sd = sc::uniform4(segs[d]);",
                "    }"]
    out.append("  }")
    return out


def _emit_seg_chain(usable, name, targs, call):
    """run_segs: a panel's segment descriptors (SegLanes, in
    descending row-mask order), each clipped to the wave's slot range [a0, a1)
    and run by its pattern's body.  The patterns are visited in that fixed
    order by a chain of uniform branches, not a multiway switch, so the
    accumulators stay in place; a repeated mask is run again."""
    out = [f"  template <{targs}>",
           f"  __device__ __forceinline__ static void {name}(const sc::SegLanes &segs, int n, int a0, int a1,",
           "                                                 float (&acc)[KM][V], A &a) {",
           "    int i = 0;",
           "    sc::vec4i sd = {0, 0, 0, 0};",
           "    if (i < n) sd = segs(i);"]
    for bits, pid in sorted(usable, key=lambda bp: -_mask(bp[0])):
        out += [f"    while (sd.x == {_mask(bits)}) {{  // id {pid}",
                "      const int lo = max(sd.y, a0);",
                "      const int hi = min(sd.y + sd.z, a1);",
                "      if (lo < hi) {",
                "        a.lo = lo;",
                "        a.hi = hi;",
                "        a.sb = sd.y;",
                "        a.vb = sd.w;",
                f"        {call(bits)}",
                "      }",
                "      sd.x = 0;",
                "      if (++i < n) sd = segs(i);",
                "    }"]
    out.append("  }")
    return out


def _emit_dispatch(usable, km):
    """The dispatcher struct of a set of bodies (run_tile, run_segs, run_wide, run)."""
    out = ["struct dispatch {"]
    out += _emit_tile_chain(usable, lambda bits: f"{tile_name(bits)}<V>(acc, a);")
    out += _emit_seg_chain(usable, "run_segs", "int KM, int V, class A",
                           lambda bits: f"{body_name(bits)}<V, A>(acc, a);")
    out.append("  template <int KM, int V>")
    out.append("  __device__ __forceinline__ static void run_wide(int mask, float (&acc)[KM][V], "
               "const sc::WideArgs &a) {")
    out.append("    switch (mask) {")
    for bits, pid in usable:
        out.append(f"      case {_mask(bits)}: {wide_name(bits)}<V>(acc, a); break;  // id {pid}")
    out.append("      default: break;")
    out.append("    }")
    out.append("  }")
    out.append("  template <int KM, int V, class A>")
    out.append("  __device__ __forceinline__ static void run(int mask, float (&acc)[KM][V], "
               "const A &a) {")
    out.append(f"    static_assert(KM == {km}, \"dispatcher generated for km={km}\");")
    out.append("    switch (mask) {")
    for bits, pid in usable:
        out.append(f"      case {_mask(bits)}: {body_name(bits)}<V, A>(acc, a); break;  // id {pid}")
    out.append("      default: break;")
    out.append("    }")
    out.append("  }")
    out.append("};")
    return out


def _emit_rows_namespace():
    """The one-row (km = 1) bodies every unit carries: plans hold the same
    slots re-laid as one-row panels, and sc_spmm_generated runs them on that
    layout under the rule sc_spmm follows (small launches, where one
    workgroup per row beats the km-row panels' longer chains)."""
    usable = [("1", 0)]
    out = ["// one-row bodies: the same slots as one-row panels (kernel_m 1)",
           "namespace rows {", ""]
    out.append(emit_body(1, "1", 0, 1, 4))
    out.append("")
    out.append(emit_wide_body(1, "1", 0, 1))
    out.append("")
    out.append(emit_tile_body(1, "1", 0))
    out.append("")
    out += _emit_dispatch(usable, 1)
    out += ["", "}  // namespace rows", ""]
    return out


def sanitize(name: str) -> str:
    return re.sub(r"[^0-9A-Za-z_]", "_", name)


def emit_unit(name: str, km: int, patterns, kn: int = 1, waves: int = 0, variant: int = 0,
              unroll: int = 0, origin: str = "", alias: bool = False, style: str = "pattern") -> str:
    """Return the text of one generated translation unit.

    ``patterns``: iterable of (bit string, id) in dictionary order.  Patterns
    whose length differs from ``km`` or that have no ones never match a
    panel (the format builder drops them) and get no body.
    ``variant``: 0 = any N, otherwise the only N the launcher accepts.
    ``alias``: also export the unit as sc_gen_unit_record / sc_gen_unit_launch
    (the fixed names the demo drivers link against).
    ``style``: "pattern" (one straight-line body per pattern) or "popcount"
    (one body per number of rows, rows read from the mask at run time).
    """
    if style not in ("pattern", "popcount"):
        raise ValueError("style must be 'pattern' or 'popcount'")
    if km < 1 or km > 20:
        raise ValueError("km must be in 1..20")
    if kn < 1:
        raise ValueError("kernel_n (pack) must be >= 1 for generated kernels")
    name = sanitize(name)
    if unroll <= 0:
        unroll = max(1, 4 // kn)
    usable = []
    seen = set()
    for bits, pid in patterns:
        if len(bits) != km or "1" not in bits or set(bits) - {"0", "1"}:
            continue
        if bits in seen:
            continue
        seen.add(bits)
        usable.append((bits, int(pid)))
    out = []
    out.append("// Generated pattern kernels for gfx950 -- do not edit.")
    if origin:
        out.append(f"// {origin}")
    out.append(f"// km={km} kn={kn} waves={waves} variant={variant} patterns={len(usable)}")
    out.append('#include "sc_kernels.hpp"')
    out.append("")
    out.append(f"namespace sc_gen_{name} {{")
    out.append("")
    if style == "popcount":
        pops = sorted({bits.count("1") for bits, _ in usable})
        for p in pops:
            out.append(emit_pop_bodies(km, p, kn, unroll))
            out.append("")
        out.append("struct dispatch {")
        out += _emit_tile_chain(usable, lambda bits: f"pop{bits.count('1')}_tile<V>(acc, a, {_mask(bits)}u);")
        out += _emit_seg_chain(usable, "run_segs", "int KM, int V, class A",
                               lambda bits: f"pop{bits.count('1')}_narrow<V, A>(acc, a, {_mask(bits)}u);")
        for kind, args in (("run_wide", "sc::WideArgs"), ("run", None)):
            body = {"run_wide": "wide", "run": "narrow"}[kind]
            if args:
                out.append("  template <int KM, int V>")
                out.append(f"  __device__ __forceinline__ static void {kind}(int mask, float (&acc)[KM][V], "
                           f"const {args} &a) {{")
            else:
                out.append("  template <int KM, int V, class A>")
                out.append(f"  __device__ __forceinline__ static void {kind}(int mask, float (&acc)[KM][V], "
                           "const A &a) {")
            out.append(f"    static_assert(KM == {km}, \"dispatcher generated for km={km}\");")
            out.append("    switch (__builtin_popcount((unsigned)mask)) {")
            for p in pops:
                targs = "V" if args else "V, A"
                out.append(f"      case {p}: pop{p}_{body}<{targs}>(acc, a, (unsigned)mask); break;")
            out.append("      default: break;")
            out.append("    }")
            out.append("  }")
        out.append("};")
        out.append("")
        out.append(f"}}  // namespace sc_gen_{name}")
        out.append("")
        return _emit_exports(out, name, km, kn, waves, variant, usable, alias, rows=False)
    for bits, pid in usable:
        out.append(emit_body(km, bits, pid, kn, unroll))
        out.append("")
        out.append(emit_wide_body(km, bits, pid, kn))
        out.append("")
        out.append(emit_tile_body(km, bits, pid))
        out.append("")
    out += _emit_rows_namespace()
    out.append("struct dispatch {")
    out += _emit_tile_chain(usable, lambda bits: f"{tile_name(bits)}<V>(acc, a);")
    out += _emit_seg_chain(usable, "run_segs", "int KM, int V, class A",
                           lambda bits: f"{body_name(bits)}<V, A>(acc, a);")
    out.append("  template <int KM, int V>")
    out.append("  __device__ __forceinline__ static void run_wide(int mask, float (&acc)[KM][V], "
               "const sc::WideArgs &a) {")
    out.append("    switch (mask) {")
    for bits, pid in usable:
        out.append(f"      case {_mask(bits)}: {wide_name(bits)}<V>(acc, a); break;  // id {pid}")
    out.append("      default: break;")
    out.append("    }")
    out.append("  }")
    out.append("  template <int KM, int V, class A>")
    out.append("  __device__ __forceinline__ static void run(int mask, float (&acc)[KM][V], "
               "const A &a) {")
    out.append(f"    static_assert(KM == {km}, \"dispatcher generated for km={km}\");")
    out.append("    switch (mask) {")
    for bits, pid in usable:
        out.append(f"      case {_mask(bits)}: {body_name(bits)}<V, A>(acc, a); break;  // id {pid}")
    out.append("      default: break;")
    out.append("    }")
    out.append("  }")
    out.append("};")
    out.append("")
    out.append(f"}}  // namespace sc_gen_{name}")
    out.append("")
    return _emit_exports(out, name, km, kn, waves, variant, usable, alias)


def _emit_exports(out, name, km, kn, waves, variant, usable, alias, rows=True):
    """The unit's extern "C" record, masks, launcher(s) and optional alias."""
    masks = ", ".join(f"{_mask(b)}u" for b, _ in usable) or "0u"
    out.append(f'extern "C" __attribute__((visibility("default"))) const uint32_t '
               f"sc_gen_{name}_masks[] = {{{masks}}};")
    if rows:
        # the one-row launcher: the same unit's km = 1 body on a plan's one-row layout
        out.append(f'extern "C" __attribute__((visibility("default"))) hipError_t '
                   f"sc_gen_{name}_launch_rows(const sc::DevView *v, const float *B, float *C, int N,")
        out.append("                                              int accumulate, int waves, "
                   "hipStream_t stream) {")
        if variant:
            out.append(f"  if (N != {variant}) return hipErrorInvalidValue;")
        out.append("  if (waves <= 0) waves = 1;")
        out.append(f"  return sc::launch_panels<1, sc_gen_{name}::rows::dispatch>(*v, B, C, N, accumulate, "
                   "waves, 1, stream);")
        out.append("}")
    # a plain host global, its launcher pointer set at load time: a constant
    # initializer naming a host function would also be emitted for the device
    out.append(f'extern "C" __attribute__((visibility("default"))) sc_gen_record '
               f"sc_gen_{name}_record = {{{km}, {kn}, {waves}, {len(usable)}, {variant}, "
               f"sc_gen_{name}_masks, nullptr}};")
    if rows:
        out.append(f"__attribute__((constructor)) static void sc_gen_{name}_record_init() {{")
        out.append(f"  sc_gen_{name}_record.rows_launch = (sc_gen_launch_fn)sc_gen_{name}_launch_rows;")
        out.append("}")
    out.append("")
    out.append(f'extern "C" __attribute__((visibility("default"))) hipError_t '
               f"sc_gen_{name}_launch(const sc::DevView *v, const float *B, float *C, int N,")
    out.append("                                         int accumulate, int waves, "
               "hipStream_t stream) {")
    if variant:
        out.append(f"  if (N != {variant}) return hipErrorInvalidValue;")
    if waves:
        out.append(f"  if (waves <= 0) waves = {waves};")
    out.append("  if (waves <= 0) waves = 1;")
    out.append(f"  return sc::launch_panels<{km}, sc_gen_{name}::dispatch>(*v, B, C, N, accumulate, "
               f"waves, {kn}, stream);")
    out.append("}")
    out.append("")
    # binary16 values / B / C (N = 1, 2, 4; the plan holds a binary16 copy of its values)
    out.append(f'extern "C" __attribute__((visibility("default"))) hipError_t '
               f"sc_gen_{name}_launch_f16(const sc::DevView *v, const void *B, void *C, int N,")
    out.append("                                             int accumulate, int waves, "
               "hipStream_t stream) {")
    if variant:
        out.append(f"  if (N != {variant}) return hipErrorInvalidValue;")
    if waves:
        out.append(f"  if (waves <= 0) waves = {waves};")
    out.append("  if (waves <= 0) waves = 1;")
    out.append(f"  return sc::launch_panels_f16<{km}, sc_gen_{name}::dispatch>(*v, B, C, N, accumulate, "
               f"waves, {kn}, stream);")
    out.append("}")
    out.append("")
    if alias:
        out.append('extern "C" __attribute__((visibility("default"))) const sc_gen_record *'
                   f"sc_gen_unit_record = &sc_gen_{name}_record;")
        out.append('extern "C" __attribute__((visibility("default"))) hipError_t '
                   "sc_gen_unit_launch(const sc::DevView *v, const float *B, float *C, int N,")
        out.append("                                                   int accumulate, int waves, "
                   "hipStream_t stream) {")
        out.append(f"  return sc_gen_{name}_launch(v, B, C, N, accumulate, waves, stream);")
        out.append("}")
        out.append("")
    return "\n".join(out)


def dictionary_patterns(ptd) -> list:
    """(bits, id) pairs of a PatternTypeDictionary in insertion order."""
    return [(bits, pid) for pid, bits in ptd.id_to_patten_bin.items()]
