// sc_plan.hip -- device-resident plans and the GPU entry points of the C ABI.
//
// A plan is the .cfmtx flattened panel-major for one device:
//   seg[]         {rowmask, slot_begin, nslots, val_begin} of every non-empty
//                 (panel, pattern) segment, panels in order, patterns in
//                 descending row-mask order inside a panel;
//   panel_seg[]   segment range of each panel;
//   panel_slot[]  slot range of each panel;
//   cols[]        int32 column (B row) of every slot;
//   vals[]        fp32 values, pop per slot, ascending panel row.
// The reference keeps P separate per-pattern arrays behind a device pointer
// table and launches one block per (panel, pattern) pair
// (example_cuda/spmm_demo_gpu_utils.h:38-67, 207-245); here one workgroup
// reads one contiguous panel, and empty (panel, pattern) pairs cost nothing.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <array>
#include <cstring>
#include <memory>
#include <functional>
#include <mutex>
#include <queue>
#include <string>
#include <vector>

#include "sc_band.hpp"
#include "sc_errors.hpp"
#include "sc_format.hpp"
#include "sc_kernels.hpp"

const sc::Cfmtx &sc_cfmtx_ref(const sc_cfmtx *cf);

// generated units (csrc/gen/sc_gen_builtin_km*.hip)
#define SC_DECLARE_GEN(k)                                                                        \
  extern "C" sc_gen_record sc_gen_builtin_km##k##_record;                                        \
  extern "C" hipError_t sc_gen_builtin_km##k##_launch(const sc::DevView *, const float *, float *, \
                                                      int, int, int, hipStream_t);               \
  extern "C" hipError_t sc_gen_builtin_km##k##_launch_f16(const sc::DevView *, const void *, void *, \
                                                          int, int, int, hipStream_t);
SC_DECLARE_GEN(1)
SC_DECLARE_GEN(2)
SC_DECLARE_GEN(3)
SC_DECLARE_GEN(4)
SC_DECLARE_GEN(5)
SC_DECLARE_GEN(6)

namespace {

using LaunchFn = hipError_t (*)(const sc::DevView *, const float *, float *, int, int, int, hipStream_t);

using LaunchF16Fn = hipError_t (*)(const sc::DevView *, const void *, void *, int, int, int, hipStream_t);

struct GenEntry {
  const sc_gen_record *rec;
  LaunchFn launch;
  LaunchF16Fn launch_f16;
};

#define SC_GEN_ENTRY(k) {&sc_gen_builtin_km##k##_record, sc_gen_builtin_km##k##_launch, sc_gen_builtin_km##k##_launch_f16}
const GenEntry kBuiltin[] = {
    {nullptr, nullptr, nullptr}, SC_GEN_ENTRY(1), SC_GEN_ENTRY(2), SC_GEN_ENTRY(3),
    SC_GEN_ENTRY(4),             SC_GEN_ENTRY(5), SC_GEN_ENTRY(6),
};
#undef SC_GEN_ENTRY
constexpr int kMaxBuiltinKm = 6;

void hip_check(hipError_t e, const char *what) {
  if (e != hipSuccess) throw sc::Error{SC_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e)};
}

}  // namespace

struct sc_plan {
  int device = 0;
  int32_t M = 0, K = 0, km = 0, npanels = 0;
  int64_t nslots = 0, nvals = 0, nsegs = 0;
  int32_t max_slots_per_panel = 0;
  int32_t kn = 0;            // column pack of the .cfmtx header
  bool dropped_pad = false;  // padding slots omitted on the device
  int32_t rows_of_km = 0;    // a one-row layout of a kernel_m > 1 file: that kernel_m
  // The same slots as one-row panels (rows_of), owned by this plan; launches
  // whose B-row gathers in that layout stay small run on it (layout_for).
  // Null with SC_PLAN_ROWS, SC_PLAN_PATTERNS, SC_PLAN_TILED, SC_PLAN_CHUNKED
  // and for kernel_m 1.
  sc_plan *rows = nullptr;
  std::vector<uint32_t> masks;  // row masks of the patterns holding slots
  void *dmem = nullptr;  // one allocation holding every array
  // split-K partial sums and arrival counters of the tiled kernel
  // (SC_PLAN_TILED), allocated with the plan (kSplitWorkFloats floats,
  // kSplitCounters counters, zeroed; every launch leaves the counters at zero)
  float *work = nullptr;
  long long work_floats = 0;
  unsigned *tcount = nullptr;
  long long tcount_n = 0;
  sc::DevView view{};
  GenEntry gen{};
  // The band layout of a kernel_m 4 plan (SC_PLAN_BANDS): wave images in
  // band_mem, and the split-K workspace and arrival counters, allocated here
  // so that no launch allocates (counters zeroed once; every launch leaves
  // them at zero).
  sc::BandView band{};
  void *band_mem = nullptr;
  float *band_work = nullptr;
  unsigned *band_cnt = nullptr;
  size_t band_work_floats = 0;
  size_t band_cnt_n = 0;
};

namespace {

template <class T>
size_t align_up(size_t off) {
  return (off + 255) / 256 * 256;
}

struct PatInfo {
  uint32_t mask;
  int pop;
};

// The panel kernel's launch order (sc::PanelLaunch rows, one per workgroup).
// Workgroups x, x + G, x + 2G, ... share a CU when the grid fits the GPU at
// once (G = the CU count: the dispatcher deals workgroups to the CUs in
// turn), and a panel's time goes with the slots it gathers, so the panels are
// dealt longest first onto the least loaded of the G groups; group c's k-th
// panel runs as workgroup c + kG.  On the 4096^2 headline matrix this takes
// the most loaded CU from 1.11x the mean slots to 1.01x.
std::vector<sc::PanelLaunch> launch_order(const std::vector<int4> &seg, const std::vector<int32_t> &panel_seg,
                                          const std::vector<int32_t> &panel_slot,
                                          const std::vector<int32_t> &panel_val, int ncu) {
  const int32_t np = (int32_t)panel_slot.size() - 1;
  std::vector<sc::PanelLaunch> out((size_t)std::max(0, np));
  if (np <= 0) return out;
  const int32_t G = std::max(1, std::min(ncu, np));
  std::vector<int64_t> weight((size_t)np, 0);
  for (int32_t q = 0; q < np; ++q)
    for (int32_t i = panel_seg[(size_t)q]; i < panel_seg[(size_t)q + 1]; ++i) weight[(size_t)q] += seg[(size_t)i].z;
  std::vector<int32_t> order((size_t)np);
  for (int32_t q = 0; q < np; ++q) order[(size_t)q] = q;
  std::stable_sort(order.begin(), order.end(),
                   [&](int32_t a, int32_t b) { return weight[(size_t)a] > weight[(size_t)b]; });
  // group c holds the workgroups x < np with x % G == c
  std::vector<int32_t> room((size_t)G), filled((size_t)G, 0);
  for (int32_t c = 0; c < G; ++c) room[(size_t)c] = (np - c + G - 1) / G;
  using Load = std::pair<int64_t, int32_t>;  // (slots so far, group)
  std::priority_queue<Load, std::vector<Load>, std::greater<Load>> heap;
  for (int32_t c = 0; c < G; ++c) heap.push({0, c});
  for (int32_t q : order) {
    const Load top = heap.top();
    heap.pop();
    const int32_t c = top.second;
    const int32_t x = c + filled[(size_t)c] * G;
    sc::PanelLaunch &r = out[(size_t)x];
    r.panel = q;
    r.slot0 = panel_slot[(size_t)q];
    r.slot1 = panel_slot[(size_t)q + 1];
    r.seg0 = panel_seg[(size_t)q];
    r.seg1 = panel_seg[(size_t)q + 1];
    r.val0 = panel_val[(size_t)q];
    r.val1 = panel_val[(size_t)q + 1];
    r.pad = 0;
    if (++filled[(size_t)c] < room[(size_t)c]) heap.push({top.first + weight[(size_t)q], c});
  }
  return out;
}

// Validate every pattern block against the header so no kernel can read
// outside the plan or write outside C; returns each block's row mask and pop.
std::vector<PatInfo> validate(const sc::Cfmtx &cf) {
  if (cf.km < 1) throw sc::Error{SC_ERR_FORMAT, "kernel_m must be >= 1"};
  if (cf.km > kMaxBuiltinKm)
    throw sc::Error{SC_ERR_UNSUPPORTED, "no pattern kernels built for kernel_m " + std::to_string(cf.km) +
                                            " (1.." + std::to_string(kMaxBuiltinKm) + ")"};
  const int32_t km = cf.km, K = cf.n, npanels = cf.npanels();
  const GenEntry gen = kBuiltin[km];
  std::vector<uint32_t> supported(gen.rec->masks, gen.rec->masks + gen.rec->npatterns);
  std::vector<PatInfo> info(cf.patterns.size());
  for (size_t i = 0; i < cf.patterns.size(); ++i) {
    const sc::Pattern &p = cf.patterns[i];
    uint32_t mask = 0;
    int pop = 0;
    for (size_t r = 0; r < p.bits.size(); ++r)
      if (p.bits[r] == '1') {
        if ((int)r >= km) throw sc::Error{SC_ERR_FORMAT, "pattern " + p.bits + " has a row outside the panel"};
        mask |= 1u << r;
        ++pop;
      }
    info[i] = {mask, pop};
    if ((int64_t)p.rpp.size() < (int64_t)npanels + 1)
      throw sc::Error{SC_ERR_FORMAT, "row-panel pointer shorter than ceil(rows/km)+1"};
    if (p.rpp[0] < 0) throw sc::Error{SC_ERR_FORMAT, "negative row-panel pointer"};
    for (int32_t q = 0; q < npanels; ++q)
      if (p.rpp[(size_t)q + 1] < p.rpp[(size_t)q])
        throw sc::Error{SC_ERR_FORMAT, "row-panel pointer is not monotone"};
    const int64_t used = p.rpp[(size_t)npanels] - p.rpp[0];
    if (used == 0) continue;
    if (pop == 0) throw sc::Error{SC_ERR_FORMAT, "pattern with no rows holds slots"};
    if ((int64_t)p.rpp[(size_t)npanels] > (int64_t)p.cb.size())
      throw sc::Error{SC_ERR_FORMAT, "row-panel pointer runs past the column list"};
    if ((int64_t)p.rpp[(size_t)npanels] * pop > (int64_t)p.val32.size())
      throw sc::Error{SC_ERR_FORMAT, "fewer values than slots * pop"};
    for (int64_t j = p.rpp[0]; j < p.rpp[(size_t)npanels]; ++j)
      if (p.cb[(size_t)j] < 0 || p.cb[(size_t)j] >= K)
        throw sc::Error{SC_ERR_FORMAT, "column index outside 0..cols-1"};
    if (std::find(supported.begin(), supported.end(), mask) == supported.end())
      throw sc::Error{SC_ERR_UNSUPPORTED, "no kernel body for pattern " + p.bits};
  }
  return info;
}

// End of slot range [a, b) of a segment without its trailing padding: the
// builder pads a segment to a multiple of kernel_n by repeating its last
// column with all-zero values (code_gen/ss_format/format_generator.py:48-63).
int32_t unpadded_end(const sc::Pattern &p, int pop, int32_t a, int32_t b) {
  while (b - 1 > a && p.cb[(size_t)b - 1] == p.cb[(size_t)b - 2]) {
    for (int k = 0; k < pop; ++k) {
      const float v = p.val32[(size_t)(b - 1) * pop + k];
      if (v != 0.0f || std::signbit(v)) return b;
    }
    --b;
  }
  return b;
}

// The same slots re-laid as one-row panels (kernel_m 1): row q*km + r holds,
// in ascending column order, every slot of panel q whose pattern contains
// row r, with that row's value.  The file's coarsening decides which values
// sit together; this layout gives each row its own workgroup, four to six
// times the workgroups of a km = 4..6 plan on the same matrix.
sc::Cfmtx rows_of(const sc::Cfmtx &cf, const std::vector<PatInfo> &info, bool drop_pad) {
  const int32_t km = cf.km, M = cf.m, npanels = cf.npanels();
  sc::Cfmtx r;
  r.m = M;
  r.n = cf.n;
  r.km = 1;
  r.kn = 1;
  r.kind = cf.kind;
  r.header_order = {0};
  sc::Pattern rp;
  rp.bits = "1";
  rp.id = 0;
  rp.pop = 1;
  rp.rpp.assign((size_t)M + 1, 0);
  auto each_entry = [&](auto &&fn) {
    for (size_t i = 0; i < cf.patterns.size(); ++i) {
      const sc::Pattern &p = cf.patterns[i];
      const int pop = info[i].pop;
      if (pop == 0) continue;
      int rows[32], nr = 0;
      for (int b = 0; b < km; ++b)
        if (info[i].mask >> b & 1u) rows[nr++] = b;
      for (int32_t q = 0; q < npanels; ++q) {
        const int32_t a = p.rpp[(size_t)q];
        const int32_t e = drop_pad ? unpadded_end(p, pop, a, p.rpp[(size_t)q + 1]) : p.rpp[(size_t)q + 1];
        for (int k = 0; k < nr; ++k) {
          const int32_t row = q * km + rows[k];
          if (row >= M) continue;  // rows of the last panel past the matrix hold only zeros
          for (int32_t j = a; j < e; ++j) fn(row, p.cb[(size_t)j], p.val32[(size_t)j * pop + k]);
        }
      }
    }
  };
  each_entry([&](int32_t row, int32_t, float) { ++rp.rpp[(size_t)row + 1]; });
  for (int32_t i = 0; i < M; ++i) {
    rp.rpp[(size_t)i + 1] += rp.rpp[(size_t)i];
    if (rp.rpp[(size_t)i + 1] < 0) throw sc::Error{SC_ERR_UNSUPPORTED, "plan larger than int32 offsets"};
  }
  const size_t n = (size_t)rp.rpp[(size_t)M];
  std::vector<std::pair<int32_t, float>> ent(n);
  std::vector<int32_t> fill(rp.rpp.begin(), rp.rpp.end() - 1);
  each_entry([&](int32_t row, int32_t c, float v) { ent[(size_t)fill[(size_t)row]++] = {c, v}; });
  rp.cb.resize(n);
  rp.val32.resize(n);
  for (int32_t i = 0; i < M; ++i) {
    auto b = ent.begin() + rp.rpp[(size_t)i], e = ent.begin() + rp.rpp[(size_t)i + 1];
    std::stable_sort(b, e, [](const auto &x, const auto &y) { return x.first < y.first; });
  }
  for (size_t j = 0; j < n; ++j) {
    rp.cb[j] = ent[j].first;
    rp.val32[j] = ent[j].second;
  }
  r.patterns.push_back(std::move(rp));
  return r;
}

sc_plan *create_plan(const sc::Cfmtx &cf, int32_t flags);

// SC_PLAN_ROWS: a km = 1 plan of the same slots (rows_of); a km = 1 file
// already is one.
sc_plan *create_rows_plan(const sc::Cfmtx &cf, int32_t flags) {
  const std::vector<PatInfo> info = validate(cf);
  if (cf.km == 1) return create_plan(cf, flags & ~SC_PLAN_ROWS);
  sc_plan *p = create_plan(rows_of(cf, info, (flags & SC_PLAN_DROP_PADDING) != 0), flags & ~SC_PLAN_ROWS);
  p->rows_of_km = cf.km;
  return p;
}

sc_plan *build_plan(const sc::Cfmtx &cf, int32_t flags, const std::vector<PatInfo> &info);
void build_band(sc_plan *plan, const sc::Cfmtx &cf, const std::vector<PatInfo> &info);

sc_plan *create_plan(const sc::Cfmtx &cf, int32_t flags) {
  if (flags & SC_PLAN_ROWS) return create_rows_plan(cf, flags);
  const std::vector<PatInfo> info = validate(cf);
  std::unique_ptr<sc_plan, void (*)(sc_plan *)> plan(build_plan(cf, flags, info), sc_plan_destroy);
  if (flags & SC_PLAN_BANDS) build_band(plan.get(), cf, info);
  if (cf.km > 1 && !(flags & (SC_PLAN_PATTERNS | SC_PLAN_TILED | SC_PLAN_CHUNKED))) {
    plan->rows = create_plan(rows_of(cf, info, (flags & SC_PLAN_DROP_PADDING) != 0),
                             flags & (SC_PLAN_DROP_PADDING | SC_PLAN_F16_VALUES));
    plan->rows->rows_of_km = cf.km;
  }
  return plan.release();
}

// The layout a launch at N columns runs on.  The one-row layout gathers one
// B row per stored entry and runs one workgroup per row; the km-row panels
// gather one B row per slot (pop rows share it) with km times fewer, longer
// workgroups.  While the one-row layout's gathers total under 128 MiB the
// launch is bound by the panels' dependent chains, not by gathered bytes, and
// the one-row layout wins: measured on MI355X 1.1-3.8x on 512x512 at km 2..6
// and N = 1..128 and on 2048x512 / 512x2048 at 80-98 % sparsity, N = 128.
// Above it the panels' B-row reuse wins: 1.1-1.5x on 4096x4096 structured at
// N = 32, 128 and 2048x512 at 50-70 %.
const sc_plan *layout_for(const sc_plan *p, int N) {
  if (p->rows && 4.0 * (double)p->rows->view.nslots * N < 134217728.0) return p->rows;
  return p;
}

sc_plan *build_plan(const sc::Cfmtx &cf, int32_t flags, const std::vector<PatInfo> &info) {
  const int32_t km = cf.km, M = cf.m, K = cf.n, npanels = cf.npanels();
  const bool drop_pad = (flags & SC_PLAN_DROP_PADDING) != 0;
  const GenEntry gen = kBuiltin[km];

  // flatten panel-major, a panel's segments in descending row-mask order: the
  // generated dispatchers visit the patterns in that fixed order
  std::vector<size_t> pat_order(cf.patterns.size());
  for (size_t i = 0; i < pat_order.size(); ++i) pat_order[i] = i;
  std::stable_sort(pat_order.begin(), pat_order.end(),
                   [&](size_t x, size_t y) { return info[x].mask > info[y].mask; });
  std::vector<int4> seg;
  std::vector<int32_t> panel_seg((size_t)npanels + 1), panel_slot((size_t)npanels + 1);
  std::vector<int32_t> panel_val((size_t)npanels + 1);
  int32_t max_pv = 0;
  std::vector<int32_t> cols;
  std::vector<float> vals;
  int32_t max_pp = 0;
  int64_t real_slots = 0, real_vals = 0;  // without the alignment padding
  for (int32_t q = 0; q < npanels; ++q) {
    panel_seg[(size_t)q] = (int32_t)seg.size();
    panel_slot[(size_t)q] = (int32_t)cols.size();
    panel_val[(size_t)q] = (int32_t)vals.size();
    for (size_t i : pat_order) {
      const sc::Pattern &p = cf.patterns[i];
      const int pop = info[i].pop;
      int32_t a = p.rpp[(size_t)q], b = p.rpp[(size_t)q + 1];
      if (b <= a) continue;
      if (drop_pad) b = unpadded_end(p, pop, a, b);
      if ((int64_t)cols.size() + (b - a) > INT32_MAX || (int64_t)vals.size() + (int64_t)(b - a) * pop > INT32_MAX)
        throw sc::Error{SC_ERR_UNSUPPORTED, "plan larger than int32 offsets"};
      seg.push_back(make_int4((int)info[i].mask, (int)cols.size(), b - a, (int)vals.size()));
      cols.insert(cols.end(), p.cb.begin() + a, p.cb.begin() + b);
      vals.insert(vals.end(), p.val32.begin() + (size_t)a * pop, p.val32.begin() + (size_t)b * pop);
    }
    real_slots += (int64_t)cols.size() - panel_slot[(size_t)q];
    real_vals += (int64_t)vals.size() - panel_val[(size_t)q];
    // every panel's columns and values start on a 16-byte boundary, so a
    // panel is staged with 16-byte loads; the padding (column 0, value 0)
    // belongs to no segment and is never computed
    while (cols.size() % 4) cols.push_back(0);
    while (vals.size() % 4) vals.push_back(0.0f);
    max_pp = std::max(max_pp, (int32_t)cols.size() - panel_slot[(size_t)q]);
    max_pv = std::max(max_pv, (int32_t)vals.size() - panel_val[(size_t)q]);
  }
  panel_seg[(size_t)npanels] = (int32_t)seg.size();
  panel_slot[(size_t)npanels] = (int32_t)cols.size();
  panel_val[(size_t)npanels] = (int32_t)vals.size();
  // km = 1: the slots of each row's segment, for the N = 1 row kernel
  std::vector<int32_t> row_len;
  if (km == 1) {
    row_len.assign((size_t)npanels, 0);
    for (int32_t q = 0; q < npanels; ++q)
      for (int32_t si = panel_seg[(size_t)q]; si < panel_seg[(size_t)q + 1]; ++si) row_len[(size_t)q] += seg[(size_t)si].z;
  }

  // K-block-major copy of the stream: for K block kb and panel p, the part
  // of each of p's segments whose columns fall in the block, contiguous per
  // (kb, p) and so per (kb, group of panels).  Built for the split-K tiled
  // kernel (SC_PLAN_TILED: 64-row tiles, row blocks of kTilePanels panels)
  // or for the chunk kernel (SC_PLAN_CHUNKED, 512-row blocks, groups of
  // kChunkPanels panels).  Needs every segment in ascending column order,
  // which is what the format builder writes; a file that is not gets no copy.
  const bool want_tiled = (flags & SC_PLAN_TILED) != 0;
  const bool want_chunk = (flags & SC_PLAN_CHUNKED) != 0;
  const int tkb = want_chunk ? sc::kChunkTileRows : sc::kTileRows;
  const int tnkb = K > 0 ? (K + tkb - 1) / tkb : 0;
  int tnrb = 0, tppb = 0;
  bool tiled = false;
  int kind = 0;
  bool sorted = true;
  for (size_t si = 0; si < seg.size() && sorted; ++si)
    for (int j = seg[si].y + 1; j < seg[si].y + seg[si].z; ++j)
      if (cols[(size_t)j] < cols[(size_t)j - 1]) {
        sorted = false;
        break;
      }
  if (tnkb > 0 && npanels > 0 && !cols.empty() && sorted && want_tiled) {
    tppb = sc::kTilePanels;
    tnrb = (npanels + tppb - 1) / tppb;
    tiled = true;
    kind = 1;
  }
  if (tnkb > 0 && npanels > 0 && !cols.empty() && sorted && want_chunk) {
    tppb = std::min(npanels, sc::kChunkPanels);
    tnrb = (npanels + tppb - 1) / tppb;
    tiled = true;
    kind = 2;
  }
  std::vector<int4> tseg;
  std::vector<int32_t> kp_seg, kp_slot, kp_val, tcols;
  std::vector<float> tvals;
  int tstage_cols = 0, tstage_vals = 0, tstage_segs = 0;
  int tchunk_dw = 0;  // most dwords of one (row block, K tile) chunk (tiled kernel)
  std::vector<int32_t> timg, toff;  // tiled kernel: chunk images and their offsets
  if (tiled && kind == 1) {
    // One chunk per (row block, K tile), row-block-major, each already laid
    // out as the kernel's LDS stage holds it (a multiple of 4 dwords):
    //   [0 .. tppb]     first descriptor of each panel's record (+ end)
    //   [tppb + 1]      dword offset of the columns, [tppb + 2] of the values
    //   [header ..)     descriptors {row mask, first slot, slots, first value}
    //                   (chunk-relative), a record's in descending mask order
    //   columns         B row of each slot relative to the tile
    //   values          pop per slot
    // toff[rb * tnkb + kb] is the chunk's first dword; one sentinel at the end.
    toff.reserve((size_t)tnrb * tnkb + 1);
    timg.reserve((size_t)tnrb * tnkb * sc::kTileChunkHeader + 2 * cols.size() + vals.size() + 4 * seg.size());
    std::vector<int32_t> cursor(seg.size());  // next slot of every segment
    for (size_t si = 0; si < seg.size(); ++si) cursor[si] = seg[si].y;
    std::vector<int4> cseg;
    std::vector<int32_t> crec, ccol, cval;
    for (int rb = 0; rb < tnrb; ++rb)
      for (int kb = 0; kb < tnkb; ++kb) {
        const int64_t klim = (int64_t)(kb + 1) * tkb;
        cseg.clear();
        crec.clear();
        ccol.clear();
        cval.clear();
        for (int32_t q = rb * tppb; q < (rb + 1) * tppb; ++q) {
          crec.push_back((int32_t)cseg.size());
          if (q >= npanels) continue;
          // sub-segments of a record in descending row-mask order: the kernel
          // visits the patterns in that fixed order
          std::vector<int32_t> order;
          for (int32_t si = panel_seg[(size_t)q]; si < panel_seg[(size_t)q + 1]; ++si) order.push_back(si);
          std::stable_sort(order.begin(), order.end(),
                           [&](int32_t x, int32_t y) { return (unsigned)seg[(size_t)x].x > (unsigned)seg[(size_t)y].x; });
          for (int32_t si : order) {
            const int4 sd = seg[(size_t)si];
            const int pop = __builtin_popcount((unsigned)sd.x);
            const int lo = cursor[(size_t)si];
            int hi = lo;
            while (hi < sd.y + sd.z && cols[(size_t)hi] < klim) ++hi;
            if (hi == lo) continue;
            cursor[(size_t)si] = hi;
            cseg.push_back(make_int4(sd.x, (int)ccol.size(), hi - lo, (int)cval.size()));
            for (int j = lo; j < hi; ++j) ccol.push_back(cols[(size_t)j] - kb * tkb);  // tile-relative
            const size_t vs = (size_t)sd.w + (size_t)(lo - sd.y) * pop;
            for (size_t v = vs; v < vs + (size_t)(hi - lo) * pop; ++v) {
              int32_t bits;
              std::memcpy(&bits, &vals[v], sizeof bits);
              cval.push_back(bits);
            }
          }
        }
        crec.push_back((int32_t)cseg.size());
        const int64_t ocol = sc::kTileChunkHeader + 4 * (int64_t)cseg.size();
        const int64_t oval = ocol + (int64_t)ccol.size();
        const int64_t dw = (oval + (int64_t)cval.size() + 3) / 4 * 4;
        if ((int64_t)timg.size() + dw > INT32_MAX) throw sc::Error{SC_ERR_UNSUPPORTED, "plan larger than int32 offsets"};
        toff.push_back((int32_t)timg.size());
        const size_t c0 = timg.size();
        timg.resize(c0 + (size_t)dw, 0);
        for (size_t i = 0; i < crec.size(); ++i) timg[c0 + i] = crec[i];
        timg[c0 + sc::kTileHdrCols] = (int32_t)ocol;
        timg[c0 + sc::kTileHdrVals] = (int32_t)oval;
        for (size_t i = 0; i < cseg.size(); ++i) {
          timg[c0 + sc::kTileChunkHeader + 4 * i + 0] = cseg[i].x;
          timg[c0 + sc::kTileChunkHeader + 4 * i + 1] = cseg[i].y;
          timg[c0 + sc::kTileChunkHeader + 4 * i + 2] = cseg[i].z;
          timg[c0 + sc::kTileChunkHeader + 4 * i + 3] = cseg[i].w;
        }
        std::copy(ccol.begin(), ccol.end(), timg.begin() + (ptrdiff_t)(c0 + ocol));
        std::copy(cval.begin(), cval.end(), timg.begin() + (ptrdiff_t)(c0 + oval));
        tchunk_dw = (int)std::max<int64_t>(tchunk_dw, dw);
      }
    toff.push_back((int32_t)timg.size());
    for (size_t si = 0; si < seg.size(); ++si)
      if (cursor[si] != seg[si].y + seg[si].z) throw sc::Error{SC_ERR_INTERNAL, "tiled layout lost slots"};
  } else if (tiled) {
    kp_seg.resize((size_t)tnkb * (npanels + 1));
    kp_slot.resize(kp_seg.size());
    kp_val.resize(kp_seg.size());
    tcols.reserve(cols.size());
    tvals.reserve(vals.size());
    std::vector<int32_t> cursor(seg.size());  // next slot of every segment
    for (size_t si = 0; si < seg.size(); ++si) cursor[si] = seg[si].y;
    for (int kb = 0; kb < tnkb; ++kb) {
      const int64_t klim = (int64_t)(kb + 1) * tkb;
      const size_t base = (size_t)kb * (npanels + 1);
      for (int32_t q = 0; q < npanels; ++q) {
        kp_seg[base + q] = (int32_t)tseg.size();
        kp_slot[base + q] = (int32_t)tcols.size();
        kp_val[base + q] = (int32_t)tvals.size();
        for (int32_t si = panel_seg[(size_t)q]; si < panel_seg[(size_t)q + 1]; ++si) {
          const int4 sd = seg[(size_t)si];
          const int pop = __builtin_popcount((unsigned)sd.x);
          const int lo = cursor[(size_t)si];
          int hi = lo;
          while (hi < sd.y + sd.z && cols[(size_t)hi] < klim) ++hi;
          if (hi == lo) continue;
          cursor[(size_t)si] = hi;
          tseg.push_back(make_int4(sd.x, (int)tcols.size(), hi - lo, (int)tvals.size()));
          tcols.insert(tcols.end(), cols.begin() + lo, cols.begin() + hi);
          const size_t v0 = (size_t)sd.w + (size_t)(lo - sd.y) * pop;
          tvals.insert(tvals.end(), vals.begin() + v0, vals.begin() + v0 + (size_t)(hi - lo) * pop);
        }
      }
      kp_seg[base + npanels] = (int32_t)tseg.size();
      kp_slot[base + npanels] = (int32_t)tcols.size();
      kp_val[base + npanels] = (int32_t)tvals.size();
      for (int rb = 0; rb < tnrb; ++rb) {
        const int pf = rb * tppb, pl = std::min(npanels, pf + tppb);
        tstage_cols = std::max(tstage_cols, kp_slot[base + pl] - kp_slot[base + pf]);
        tstage_vals = std::max(tstage_vals, kp_val[base + pl] - kp_val[base + pf]);
        tstage_segs = std::max(tstage_segs, kp_seg[base + pl] - kp_seg[base + pf]);
      }
    }
    tstage_cols = (tstage_cols + 3) / 4 * 4;
    for (size_t si = 0; si < seg.size(); ++si)
      if (cursor[si] != seg[si].y + seg[si].z) throw sc::Error{SC_ERR_INTERNAL, "tiled layout lost slots"};
  }

  auto plan = std::make_unique<sc_plan>();
  hip_check(hipGetDevice(&plan->device), "hipGetDevice");
  plan->M = M;
  plan->K = K;
  plan->km = km;
  plan->npanels = npanels;
  plan->nslots = real_slots;
  plan->nvals = real_vals;
  plan->nsegs = (int64_t)seg.size();
  plan->max_slots_per_panel = max_pp;
  plan->gen = gen;
  plan->kn = cf.kn;
  plan->dropped_pad = drop_pad;
  for (size_t i = 0; i < cf.patterns.size(); ++i) {
    const sc::Pattern &p = cf.patterns[i];
    if (p.rpp[(size_t)npanels] > p.rpp[0] &&
        std::find(plan->masks.begin(), plan->masks.end(), info[i].mask) == plan->masks.end())
      plan->masks.push_back(info[i].mask);
  }

  size_t off_seg = 0;
  size_t off_pseg = align_up<int>(off_seg + seg.size() * sizeof(int4));
  size_t off_pslot = align_up<int>(off_pseg + panel_seg.size() * sizeof(int32_t));
  size_t off_pval = align_up<int>(off_pslot + panel_slot.size() * sizeof(int32_t));
  size_t off_cols = align_up<int>(off_pval + panel_val.size() * sizeof(int32_t));
  size_t off_vals = align_up<int>(off_cols + cols.size() * sizeof(int32_t));
  size_t off_tseg = align_up<int>(off_vals + vals.size() * sizeof(float));
  size_t off_kpseg = align_up<int>(off_tseg + tseg.size() * sizeof(int4));
  size_t off_kpslot = align_up<int>(off_kpseg + kp_seg.size() * sizeof(int32_t));
  size_t off_kpval = align_up<int>(off_kpslot + kp_slot.size() * sizeof(int32_t));
  size_t off_tcols = align_up<int>(off_kpval + kp_val.size() * sizeof(int32_t));
  size_t off_tvals = align_up<int>(off_tcols + tcols.size() * sizeof(int32_t));
  // binary16 copy of the values (SC_PLAN_F16_VALUES), rounded to nearest even
  std::vector<_Float16> vals16;
  if (flags & SC_PLAN_F16_VALUES) {
    vals16.resize(vals.size());
    for (size_t i = 0; i < vals.size(); ++i) vals16[i] = (_Float16)vals[i];
  }
  size_t off_timg = align_up<int>(off_tvals + tvals.size() * sizeof(float));
  size_t off_toff = align_up<int>(off_timg + timg.size() * sizeof(int32_t));
  size_t off_v16 = align_up<int>(off_toff + toff.size() * sizeof(int32_t));
  size_t off_rowlen = align_up<int>(off_v16 + vals16.size() * sizeof(_Float16));
  int ncu = 0;
  hip_check(hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, plan->device),
            "hipDeviceGetAttribute(multiprocessor count)");
  const std::vector<sc::PanelLaunch> launch = launch_order(seg, panel_seg, panel_slot, panel_val, ncu);
  size_t off_launch = align_up<int>(off_rowlen + row_len.size() * sizeof(int32_t));
  size_t total = align_up<int>(off_launch + launch.size() * sizeof(sc::PanelLaunch));
  hip_check(hipMalloc(&plan->dmem, total), "hipMalloc(plan)");
  std::vector<unsigned char> host(total, 0);
  std::memcpy(host.data() + off_seg, seg.data(), seg.size() * sizeof(int4));
  std::memcpy(host.data() + off_pseg, panel_seg.data(), panel_seg.size() * sizeof(int32_t));
  std::memcpy(host.data() + off_pslot, panel_slot.data(), panel_slot.size() * sizeof(int32_t));
  std::memcpy(host.data() + off_pval, panel_val.data(), panel_val.size() * sizeof(int32_t));
  std::memcpy(host.data() + off_tseg, tseg.data(), tseg.size() * sizeof(int4));
  std::memcpy(host.data() + off_kpseg, kp_seg.data(), kp_seg.size() * sizeof(int32_t));
  std::memcpy(host.data() + off_kpslot, kp_slot.data(), kp_slot.size() * sizeof(int32_t));
  std::memcpy(host.data() + off_kpval, kp_val.data(), kp_val.size() * sizeof(int32_t));
  std::memcpy(host.data() + off_tcols, tcols.data(), tcols.size() * sizeof(int32_t));
  std::memcpy(host.data() + off_tvals, tvals.data(), tvals.size() * sizeof(float));
  std::memcpy(host.data() + off_cols, cols.data(), cols.size() * sizeof(int32_t));
  std::memcpy(host.data() + off_vals, vals.data(), vals.size() * sizeof(float));
  std::memcpy(host.data() + off_v16, vals16.data(), vals16.size() * sizeof(_Float16));
  std::memcpy(host.data() + off_timg, timg.data(), timg.size() * sizeof(int32_t));
  std::memcpy(host.data() + off_toff, toff.data(), toff.size() * sizeof(int32_t));
  std::memcpy(host.data() + off_rowlen, row_len.data(), row_len.size() * sizeof(int32_t));
  std::memcpy(host.data() + off_launch, launch.data(), launch.size() * sizeof(sc::PanelLaunch));
  hipError_t e = hipMemcpy(plan->dmem, host.data(), total, hipMemcpyHostToDevice);
  if (e != hipSuccess) {
    (void)hipFree(plan->dmem);
    hip_check(e, "hipMemcpy(plan)");
  }
  unsigned char *base = (unsigned char *)plan->dmem;
  plan->view.seg = (const int4 *)(base + off_seg);
  plan->view.panel_seg = (const int *)(base + off_pseg);
  plan->view.panel_slot = (const int *)(base + off_pslot);
  plan->view.panel_val = (const int *)(base + off_pval);
  plan->view.cols = (const int *)(base + off_cols);
  plan->view.vals = (const float *)(base + off_vals);
  plan->view.M = M;
  plan->view.K = K;
  plan->view.km = km;
  plan->view.npanels = npanels;
  plan->view.max_pslots = max_pp;
  plan->view.max_pvals = max_pv;
  plan->view.tseg = (tiled && kind == 2) ? (const int4 *)(base + off_tseg) : nullptr;
  plan->view.kp_seg = (const int *)(base + off_kpseg);
  plan->view.kp_slot = (const int *)(base + off_kpslot);
  plan->view.kp_val = (const int *)(base + off_kpval);
  plan->view.tcols = (const int *)(base + off_tcols);
  plan->view.tvals = (const float *)(base + off_tvals);
  plan->view.timg = timg.empty() ? nullptr : (const int *)(base + off_timg);
  plan->view.toff = toff.empty() ? nullptr : (const int *)(base + off_toff);
  plan->view.tkb = tkb;
  plan->view.tnkb = tnkb;
  plan->view.tppb = tppb;
  plan->view.tnrb = tnrb;
  plan->view.tstage_cols = tstage_cols;
  plan->view.tstage_vals = tstage_vals;
  plan->view.tstage_segs = tstage_segs;
  plan->view.tchunk_dw = tchunk_dw;
  plan->view.nslots = (long long)cols.size();
  plan->view.work = nullptr;
  plan->view.work_floats = 0;
  plan->view.tcount = nullptr;
  plan->view.tcount_n = 0;
  plan->view.kblock_kind = kind;
  plan->view.a_bytes = 4ll * ((long long)cols.size() + (long long)vals.size());
  plan->view.vals16 = vals16.empty() ? nullptr : (const _Float16 *)(base + off_v16);
  plan->view.row_len = row_len.empty() ? nullptr : (const int *)(base + off_rowlen);
  plan->view.launch = launch.empty() ? nullptr : (const int *)(base + off_launch);
  if (plan->view.timg) {
    hip_check(hipMalloc((void **)&plan->work, sc::kSplitWorkFloats * sizeof(float)), "hipMalloc(split-K workspace)");
    plan->work_floats = (long long)sc::kSplitWorkFloats;
    hip_check(hipMalloc((void **)&plan->tcount, sc::kSplitCounters * sizeof(unsigned)), "hipMalloc(split-K counters)");
    hip_check(hipMemset(plan->tcount, 0, sc::kSplitCounters * sizeof(unsigned)), "hipMemset(split-K counters)");
    hip_check(hipDeviceSynchronize(), "hipDeviceSynchronize(split-K workspace)");
    plan->tcount_n = (long long)sc::kSplitCounters;
  }
  return plan.release();
}

// ---- band layout (SC_PLAN_BANDS, kernel_m 4) -----------------------------
// A panel's slots for the band kernel, every pattern together in ascending
// column order, each with its four row values (0 for the rows its pattern
// lacks).
struct BandPanel {
  std::vector<std::pair<int32_t, std::array<float, 4>>> slots;
};

struct BandHost {
  std::vector<int32_t> img, woff;
  int nbands = 0, nks = 0, KR = 0;
};

std::vector<BandPanel> band_panels(const sc::Cfmtx &cf, const std::vector<PatInfo> &info, bool drop_pad) {
  const int32_t npanels = cf.npanels();
  std::vector<BandPanel> out((size_t)npanels);
  for (size_t i = 0; i < cf.patterns.size(); ++i) {
    const sc::Pattern &p = cf.patterns[i];
    const int pop = info[i].pop;
    if (pop == 0) continue;
    int rows[4], nr = 0;
    for (int b = 0; b < 4; ++b)
      if (info[i].mask >> b & 1u) rows[nr++] = b;
    for (int32_t q = 0; q < npanels; ++q) {
      const int32_t a = p.rpp[(size_t)q];
      const int32_t e = drop_pad ? unpadded_end(p, pop, a, p.rpp[(size_t)q + 1]) : p.rpp[(size_t)q + 1];
      BandPanel &bp = out[(size_t)q];
      for (int32_t j = a; j < e; ++j) {
        const float *v = &p.val32[(size_t)j * pop];
        std::array<float, 4> x = {0.f, 0.f, 0.f, 0.f};
        for (int k = 0; k < nr; ++k) x[(size_t)rows[k]] = v[k];
        bp.slots.push_back({p.cb[(size_t)j], x});
      }
    }
  }
  auto by_col = [](const auto &x, const auto &y) { return x.first < y.first; };
  for (BandPanel &bp : out) std::stable_sort(bp.slots.begin(), bp.slots.end(), by_col);
  return out;
}

// The wave records (layout: sc_band.hpp, BandView).  K ranges of up to
// kBandMaxRange rows; bands of one to kBandWavePanels panels per wave, sized
// so that bands x K ranges is about kBandTargetPairs; per (band, K range)
// a panel's items are the windows of four consecutive columns (aligned to 4
// in the range) that hold its entries, and the panels go to the waves
// longest first, each onto the least loaded wave that holds fewer than
// kBandWavePanels (load: its groups plus one per panel for the hand-over);
// a wave runs its panels in ascending order.
void band_records(const std::vector<BandPanel> &panels, int32_t K, BandHost &h) {
  const int32_t npanels = (int32_t)panels.size();
  h = BandHost{};
  h.KR = (int)std::min<int64_t>(sc::kBandMaxRange, ((int64_t)K + 3) / 4 * 4);
  h.nks = (int)(((int64_t)K + h.KR - 1) / h.KR);
  const int64_t want = ((int64_t)npanels * h.nks + sc::kBandTargetPairs - 1) / sc::kBandTargetPairs;
  const int32_t P = (int32_t)std::min<int64_t>((int64_t)sc::kBandWaves * sc::kBandWavePanels,
                                               std::max<int64_t>(sc::kBandWaves, want));
  h.nbands = (npanels + P - 1) / P;
  // a cursor into each panel's column-sorted slots: its K ranges are visited
  // in order
  std::vector<size_t> cur((size_t)npanels, 0);
  h.woff.reserve((size_t)h.nbands * h.nks * sc::kBandWaves + 1);
  struct Window {
    int32_t w;      // window index in the range (B rows 4w .. 4w + 3)
    float v[16];    // A(i, t) at 4t + i
  };
  std::vector<int32_t> rec;
  for (int b = 0; b < h.nbands; ++b) {
    const int32_t q0 = b * P, q1 = std::min(npanels, q0 + P), nq = q1 - q0;
    std::vector<std::vector<Window>> win((size_t)nq);
    std::vector<int32_t> ngr((size_t)nq), order((size_t)nq);
    for (int ks = 0; ks < h.nks; ++ks) {
      const int32_t klo = ks * h.KR;
      const int64_t khi = std::min<int64_t>((int64_t)K, (int64_t)klo + h.KR);
      for (int32_t i = 0; i < nq; ++i) {
        const BandPanel &bp = panels[(size_t)(q0 + i)];
        size_t &c = cur[(size_t)(q0 + i)];
        std::vector<Window> &ws = win[(size_t)i];
        ws.clear();
        while (c < bp.slots.size() && bp.slots[c].first < khi) {
          const int32_t col = bp.slots[c].first;
          if (col < klo) throw sc::Error{SC_ERR_INTERNAL, "band layout lost a slot"};
          const int32_t wi = (col - klo) >> 2, t = (col - klo) & 3;
          if (ws.empty() || ws.back().w != wi) ws.push_back(Window{wi, {0.f}});
          for (int r = 0; r < 4; ++r) {
            float &dst = ws.back().v[4 * t + r];
            if (dst != 0.f && bp.slots[c].second[(size_t)r] != 0.f)
              throw sc::Error{SC_ERR_INTERNAL, "band layout met one entry twice"};
            dst += bp.slots[c].second[(size_t)r];
          }
          ++c;
        }
        ngr[(size_t)i] = (int32_t)std::max<size_t>(1, (ws.size() + 3) / 4);  // an empty panel: one group of zeros
        order[(size_t)i] = i;
      }
      std::stable_sort(order.begin(), order.end(),
                       [&](int32_t x, int32_t y) { return ngr[(size_t)x] > ngr[(size_t)y]; });
      std::vector<std::vector<int32_t>> wp(sc::kBandWaves);
      int64_t load[sc::kBandWaves] = {0};
      for (int32_t i : order) {
        int best = -1;
        for (int w = 0; w < sc::kBandWaves; ++w)
          if ((int)wp[(size_t)w].size() < sc::kBandWavePanels && (best < 0 || load[w] < load[best])) best = w;
        wp[(size_t)best].push_back(i);
        load[best] += ngr[(size_t)i] + 1;
      }
      for (int w = 0; w < sc::kBandWaves; ++w) {
        std::vector<int32_t> &mine = wp[(size_t)w];
        std::sort(mine.begin(), mine.end());
        int32_t groups = 0;
        for (int32_t i : mine) groups += ngr[(size_t)i];
        const size_t ptab_dw = (2 * mine.size() + 3) / 4 * 4;
        const size_t nblk = std::max<size_t>(1, ((size_t)groups + 3) / 4);
        rec.assign((size_t)sc::kBandRecHeader + ptab_dw + nblk * sc::kBandBlockDw, 0);
        rec[0] = (int32_t)mine.size();
        rec[1] = groups;
        rec[2] = (int32_t)nblk;
        for (size_t k = 0; k < mine.size(); ++k) {
          rec[sc::kBandRecHeader + 2 * k] = q0 + mine[k];
          rec[sc::kBandRecHeader + 2 * k + 1] = ngr[(size_t)mine[k]];
        }
        // padding items: values 0 on window 0
        const size_t base = sc::kBandRecHeader + ptab_dw;
        size_t gi = 0;  // the wave's group index
        for (int32_t i : mine) {
          const std::vector<Window> &ws = win[(size_t)i];
          for (int32_t G = 0; G < ngr[(size_t)i]; ++G, ++gi) {
            int32_t *bk = &rec[base + (gi / 4) * sc::kBandBlockDw];
            const int g4 = (int)(gi % 4);
            for (int u = 0; u < 4; ++u) {
              const size_t m = 4 * (size_t)G + u;
              if (m >= ws.size()) continue;
              bk[256 + 4 * g4 + u] = ws[m].w * 4 * sc::kBandRowBytes;
              for (int t = 0; t < 4; ++t)
                for (int r = 0; r < 4; ++r) std::memcpy(&bk[4 * (16 * u + 4 * t + r) + g4], &ws[m].v[4 * t + r], 4);
            }
          }
        }
        if ((int64_t)h.img.size() + (int64_t)rec.size() > INT32_MAX)
          throw sc::Error{SC_ERR_UNSUPPORTED, "band layout larger than int32 offsets"};
        h.woff.push_back((int32_t)h.img.size());
        h.img.insert(h.img.end(), rec.begin(), rec.end());
        h.img.resize((h.img.size() + 3) / 4 * 4, 0);  // 16-byte aligned records
      }
    }
  }
  h.woff.push_back((int32_t)h.img.size());
  for (int32_t q = 0; q < npanels; ++q)
    if (cur[(size_t)q] != panels[(size_t)q].slots.size()) throw sc::Error{SC_ERR_INTERNAL, "band layout lost slots"};
}

// Build and upload the band layout of a kernel_m 4 plan, with the split-K
// workspace (partial tiles for N up to 64 * kBandMaxChunks) and arrival
// counters it needs, so that no launch allocates.
void build_band(sc_plan *plan, const sc::Cfmtx &cf, const std::vector<PatInfo> &info) {
  if (cf.km != 4) throw sc::Error{SC_ERR_UNSUPPORTED, "the band layout needs kernel_m 4"};
  if (cf.n <= 0 || cf.npanels() <= 0) return;
  // the format's zero padding slots (kernel_n packs) are never computed here:
  // they repeat their segment's last column with value 0
  const std::vector<BandPanel> panels = band_panels(cf, info, true);
  // more K ranges than this and the partial sums outweigh the staging saved
  if (((int64_t)cf.n + sc::kBandMaxRange - 1) / sc::kBandMaxRange > sc::kBandMaxRanges) return;
  BandHost h;
  band_records(panels, cf.n, h);
  if (sc::band_lds_bytes(h.KR) > sc::kBandLdsBytes) return;  // the plan runs its other kernels
  const size_t off_woff = align_up<int>(h.img.size() * sizeof(int32_t));
  const size_t total = align_up<int>(off_woff + h.woff.size() * sizeof(int32_t));
  hip_check(hipMalloc(&plan->band_mem, total), "hipMalloc(band layout)");
  std::vector<unsigned char> host(total, 0);
  std::memcpy(host.data(), h.img.data(), h.img.size() * sizeof(int32_t));
  std::memcpy(host.data() + off_woff, h.woff.data(), h.woff.size() * sizeof(int32_t));
  hip_check(hipMemcpy(plan->band_mem, host.data(), total, hipMemcpyHostToDevice), "hipMemcpy(band layout)");
  plan->band_work_floats = sc::band_partial_floats(h.nks, cf.npanels(), sc::kBandMaxChunks);
  plan->band_cnt_n = h.nks > 1 ? (size_t)cf.npanels() * sc::kBandMaxChunks : 0;
  if (plan->band_work_floats) {
    hip_check(hipMalloc((void **)&plan->band_work, plan->band_work_floats * sizeof(float)),
              "hipMalloc(band workspace)");
    hip_check(hipMalloc((void **)&plan->band_cnt, plan->band_cnt_n * sizeof(unsigned)), "hipMalloc(band counters)");
    hip_check(hipMemset(plan->band_cnt, 0, plan->band_cnt_n * sizeof(unsigned)), "hipMemset(band counters)");
  }
  hip_check(hipDeviceSynchronize(), "hipDeviceSynchronize(band layout)");
  plan->band.img = (const int *)plan->band_mem;
  plan->band.woff = (const int *)((unsigned char *)plan->band_mem + off_woff);
  plan->band.nbands = h.nbands;
  plan->band.nks = h.nks;
  plan->band.KR = h.KR;
  plan->band.npanels = cf.npanels();
}

// Waves per panel: enough waves in the grid to cover the 256 CUs several
// times, but no wave with less than ~2 steps of S slots unless the panel has
// many pattern segments (a wave runs its segments one after another, each a
// full memory round trip, so short segments are spread over more waves), and
// the LDS of the cross-wave reduction within 64 KiB.
int auto_waves(const sc_plan *p, int N) {
  if (p->npanels == 0) return 1;
  const sc::Geometry g1 = sc::geometry(p->km, N, 1, p->K, p->view.max_pslots, p->view.max_pvals, p->view.a_bytes,
                                   p->nslots / std::max(1, p->npanels), p->npanels);
  const int S = 64 / g1.L;
  const double avg = (double)p->nslots / p->npanels;
  const double segs = (double)p->nsegs / p->npanels;
  int w_occ = (int)std::max<int64_t>(1, 4096 / std::max(1, p->npanels));
  int w_work = (int)std::max(1.0, std::max(avg / (2.0 * S), segs / 2.0));
  int w = std::min(std::min(w_occ, w_work), 16);
  // small-N gather kernel at N = 2, 4: the cross-wave reduction grows with
  // W * N; on 512^2 at 80 % sparsity, km 4, N = 4, 4 waves run in 6.5 us
  // against 7.2 with 7
  if ((N == 2 || N == 4) && sc::gather_lds_f32(N, 1, p->km, p->view.max_pslots, p->view.max_pvals)) w = std::min(w, 4);
  while (w > 1 && sc::geometry(p->km, N, w, p->K, p->view.max_pslots, p->view.max_pvals, p->view.a_bytes,
                                   p->nslots / std::max(1, p->npanels), p->npanels).lds > 65536) --w;
  return std::max(w, 1);
}

// Does a generated unit fit this plan?  (km, pack, pattern bodies, N)
void check_record(const sc_plan *p, const sc_gen_record *rec, int32_t N) {
  if (!rec) throw sc::Error{SC_ERR_ARG, "null generated-kernel record"};
  if (rec->km != p->km)
    throw sc::Error{SC_ERR_ARG, "kernels generated for km=" + std::to_string(rec->km) + ", plan has km=" +
                                    std::to_string(p->km)};
  if (rec->kn > 1) {
    if (p->dropped_pad)
      throw sc::Error{SC_ERR_ARG, "kernels unrolled for packs of " + std::to_string(rec->kn) +
                                      " need the padded plan (no SC_PLAN_DROP_PADDING)"};
    if (p->kn <= 0 || p->kn % rec->kn != 0)
      throw sc::Error{SC_ERR_ARG, "kernels unrolled for packs of " + std::to_string(rec->kn) +
                                      " do not divide the .cfmtx kernel_n " + std::to_string(p->kn)};
  }
  if (rec->variant != 0 && rec->variant != N)
    throw sc::Error{SC_ERR_ARG, "kernels generated for N=" + std::to_string(rec->variant) + ", called with N=" +
                                    std::to_string(N)};
  for (uint32_t m : p->masks) {
    bool found = false;
    for (int32_t i = 0; i < rec->npatterns && !found; ++i) found = rec->masks[i] == m;
    if (!found) throw sc::Error{SC_ERR_UNSUPPORTED, "generated kernels have no body for row mask " + std::to_string(m)};
  }
}

// A workspace the caller brings for the split-K kernels, in place of the
// plan's own (sc_spmm_noalloc: the library's static scratch).
struct Scratch {
  float *work;
  size_t work_floats;
  unsigned *counters;
  size_t counters_n;
};

__global__ void zero_counters(unsigned *c, int n) {
  for (int i = threadIdx.x; i < n; i += blockDim.x) c[i] = 0u;
}

// Arrival counters must start at zero: a small fill kernel, not a memset, so
// the call stays capturable in a HIP graph.
void clear_counters(unsigned *c, size_t n, hipStream_t stream) {
  hipLaunchKernelGGL(zero_counters, dim3(1), dim3(256), 0, stream, c, (int)n);
  hip_check(hipGetLastError(), "counter clear launch");
}

int launch(const sc_plan *p, const sc_gen_record *rec, sc_gen_launch_fn fn, const float *B, float *C,
           int32_t N, int32_t flags, int32_t waves, void *stream, const Scratch *scratch = nullptr) {
  if (!p) throw sc::Error{SC_ERR_ARG, "null plan"};
  if (!fn) throw sc::Error{SC_ERR_ARG, "null generated-kernel launcher"};
  if (N < 1) throw sc::Error{SC_ERR_ARG, "N must be >= 1"};
  if (!B || !C) throw sc::Error{SC_ERR_ARG, "null device buffer"};
  if (waves < 0 || waves > 16) throw sc::Error{SC_ERR_ARG, "waves per panel must be 0..16"};
  check_record(p, rec, N);
  int dev = -1;
  hip_check(hipGetDevice(&dev), "hipGetDevice");
  if (dev != p->device) throw sc::Error{SC_ERR_ARG, "plan lives on another device than the current one"};
  if ((N % 4 == 0 && ((uintptr_t)B % 16 || (uintptr_t)C % 16)) ||
      (N % 2 == 0 && ((uintptr_t)B % 8 || (uintptr_t)C % 8)) || (uintptr_t)B % 4 || (uintptr_t)C % 4)
    throw sc::Error{SC_ERR_ARG, "B and C must be aligned to their vector width (16 B when N % 4 == 0)"};
  int w = waves ? waves : (rec->waves ? rec->waves : auto_waves(p, N));
  if (sc::geometry(p->km, N, w, p->K, p->view.max_pslots, p->view.max_pvals, p->view.a_bytes,
                                   p->nslots / std::max(1, p->npanels), p->npanels).lds > 65536)
    throw sc::Error{SC_ERR_ARG, "too many waves per panel for this N"};
  sc::DevView view = p->view;
  // the split-K workspace: the plan's, or the caller's scratch (nothing is
  // allocated here)
  view.work = scratch ? scratch->work : p->work;
  view.work_floats = scratch ? (long long)scratch->work_floats : p->work_floats;
  view.tcount = scratch ? scratch->counters : p->tcount;
  view.tcount_n = scratch ? (long long)scratch->counters_n : p->tcount_n;
  if (scratch) {
    const sc::TileGeometry tg = sc::tile_geometry(view, N);
    if (tg.use && tg.nks > 1) clear_counters(scratch->counters, (size_t)tg.counters, (hipStream_t)stream);
  }
  int e = fn(&view, B, C, N, (flags & SC_ACCUMULATE) ? 1 : 0, w, stream);
  hip_check((hipError_t)e, "pattern kernel launch");
  return SC_OK;
}

// The band kernel when the plan has a band layout and N fits it and the
// given workspace; false otherwise.  work / counters: the split-K workspace
// to use (work_cap floats, counter_cap counters); clear: zero the counters
// first (a caller's scratch).
bool launch_band(const sc_plan *p, const float *B, float *C, int32_t N, int32_t flags, void *stream, float *work,
                 unsigned *counters, size_t work_cap, size_t counter_cap, bool clear = false) {
  if (!p->band.img) return false;
  const sc::BandGeometry g = sc::band_geometry(p->band, N, work_cap, counter_cap);
  if (!g.use) return false;
  if (!B || !C) throw sc::Error{SC_ERR_ARG, "null device buffer"};
  int dev = -1;
  hip_check(hipGetDevice(&dev), "hipGetDevice");
  if (dev != p->device) throw sc::Error{SC_ERR_ARG, "plan lives on another device than the current one"};
  if ((uintptr_t)B % 16 || (uintptr_t)C % 16)
    throw sc::Error{SC_ERR_ARG, "B and C must be aligned to their vector width (16 B when N % 4 == 0)"};
  if (clear && g.counters > 0) clear_counters(counters, (size_t)g.counters, (hipStream_t)stream);
  hip_check(sc::launch_band(p->band, g, B, C, work, counters, p->M, p->K, N, (flags & SC_ACCUMULATE) ? 1 : 0,
                            (hipStream_t)stream),
            "band kernel launch");
  return true;
}

// ---- the static scratch of sc_spmm_noalloc --------------------------------
// partial sums: the band kernel's at N = 128 on a 4096-row plan with 8 K
// ranges (16 MiB), which also holds the tiled kernel's (kSplitWorkFloats)
constexpr size_t kScratchWorkFloats = (size_t)4 << 20;
static_assert(kScratchWorkFloats >= sc::kSplitWorkFloats, "the scratch holds the tiled kernel's workspace");
constexpr size_t kScratchWorkBytes = kScratchWorkFloats * sizeof(float);
constexpr size_t kScratchBytes = kScratchWorkBytes + sc::kSplitCounters * sizeof(unsigned);

}  // namespace

// The split-K partial sums and arrival counters of sc_spmm_noalloc: one copy
// on every GPU the library runs on, held until the process ends.  In host
// code `scratch` names a host-side stand-in, not device memory: host code uses
// only the device address that hipGetSymbolAddress returns for the current
// device (scratch_base).
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
unsigned char *g_scratch_base[kMaxDevices] = {};

// Device address of `scratch` on device dev, which must be current: looked up
// with hipGetSymbolAddress on the first call on that device, then kept.
unsigned char *scratch_base(int dev) {
  if (dev < 0 || dev >= kMaxDevices) throw sc::Error{SC_ERR_UNSUPPORTED, "device index beyond the scratch table"};
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_base[dev]) {
    void *ptr = nullptr;
    hip_check(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
    if (!ptr) throw sc::Error{SC_ERR_HIP, "hipGetSymbolAddress(scratch) returned a null address"};
    g_scratch_base[dev] = (unsigned char *)ptr;
  }
  return g_scratch_base[dev];
}

}  // namespace

extern "C" {

int sc_plan_create(const sc_cfmtx *cf, int32_t flags, sc_plan **out) {
  SC_GUARD([&] {
    if (!cf || !out) throw sc::Error{SC_ERR_ARG, "null argument"};
    if (flags & ~(SC_PLAN_DROP_PADDING | SC_PLAN_TILED | SC_PLAN_CHUNKED | SC_PLAN_F16_VALUES | SC_PLAN_ROWS |
                  SC_PLAN_PATTERNS | SC_PLAN_BANDS))
      throw sc::Error{SC_ERR_ARG, "unknown plan flags"};
    if ((flags & SC_PLAN_ROWS) && (flags & SC_PLAN_PATTERNS))
      throw sc::Error{SC_ERR_ARG, "SC_PLAN_ROWS and SC_PLAN_PATTERNS are exclusive"};
    if ((flags & SC_PLAN_TILED) && (flags & SC_PLAN_CHUNKED))
      throw sc::Error{SC_ERR_ARG, "SC_PLAN_TILED and SC_PLAN_CHUNKED are exclusive"};
    if ((flags & SC_PLAN_BANDS) && (flags & SC_PLAN_ROWS))
      throw sc::Error{SC_ERR_ARG, "SC_PLAN_BANDS needs the kernel_m 4 panels (not SC_PLAN_ROWS)"};
    *out = create_plan(sc_cfmtx_ref(cf), flags);
  });
}

int sc_plan_info(const sc_plan *p, int32_t *m, int32_t *n, int32_t *km, int32_t *npanels, int64_t *nslots,
                 int64_t *nvals, int64_t *nsegs) {
  SC_GUARD([&] {
    if (!p) throw sc::Error{SC_ERR_ARG, "null plan"};
    if (m) *m = p->M;
    if (n) *n = p->K;
    if (km) *km = p->km;
    if (npanels) *npanels = p->npanels;
    if (nslots) *nslots = p->nslots;
    if (nvals) *nvals = p->nvals;
    if (nsegs) *nsegs = p->nsegs;
  });
}

int sc_plan_describe(const sc_plan *p, int32_t N, char *buf, size_t buflen) {
  SC_GUARD([&] {
    if (!p || !buf || buflen == 0) throw sc::Error{SC_ERR_ARG, "null argument"};
    if (N < 1) throw sc::Error{SC_ERR_ARG, "N must be >= 1"};
    std::string d;
    const sc::BandGeometry bg = sc::band_geometry(p->band, N, p->band_work_floats, p->band_cnt_n);
    if (bg.use) {
      d = "band_kernel km=4 cols=" + std::to_string(sc::kBandCols) + " range_rows=" + std::to_string(p->band.KR) +
          " bands=" + std::to_string(p->band.nbands) + " ks=" + std::to_string(p->band.nks) + " chunks=" +
          std::to_string(bg.nch) + " grid=" + std::to_string(bg.grid);
      if (d.size() + 1 > buflen) throw sc::Error{SC_ERR_ARG, "buffer too small"};
      std::memcpy(buf, d.c_str(), d.size() + 1);
      return;
    }
    p = layout_for(p, N);
    const sc::TileGeometry tg = sc::tile_geometry(p->view, N);
    const sc::ChunkGeometry cg = sc::chunk_geometry(p->view, N);
    if (!tg.use && cg.use) {
      d = "chunk_kernel km=" + std::to_string(p->km) + " V=4 cols=" + std::to_string(sc::kChunkCols) +
          " tile_rows=" + std::to_string(std::min(cg.KT, p->K)) + " waves=" + std::to_string(cg.W) + " grid=" +
          std::to_string(cg.grid) + " (" + std::to_string(cg.ngroups) + " row groups x " +
          std::to_string(cg.nchunks) + " chunks)";
    } else if (tg.use) {
      d = "tiled_kernel km=" + std::to_string(p->km) + " V=" + std::to_string(tg.V) + " waves=" +
          std::to_string(sc::kTilePanels) + " tile_rows=" + std::to_string(sc::kTileRows) + " grid=" +
          std::to_string(p->view.tnrb) + "x" + std::to_string(tg.nks) + "x" + std::to_string(tg.chunks) +
          " tiles_per_unit=" + std::to_string(tg.tpu);
    } else {
      const int w = auto_waves(p, N);
      const sc::Geometry g = sc::geometry(p->km, N, w, p->K, p->view.max_pslots, p->view.max_pvals, p->view.a_bytes,
                                   p->nslots / std::max(1, p->npanels), p->npanels);
      if (sc::use_row_spmv(p->view, p->km, N, w)) {
        const bool st = sc::row_spmv_staged(p->view, N);
        const int rows = st ? sc::kRowStagedRows : sc::kRowSpmvRows;
        d = "row_spmv_kernel km=1 V=" + std::to_string(N) + " rows_per_workgroup=" + std::to_string(rows) +
            (st ? " B_in_lds=1" : "") + " grid=" + std::to_string((p->M + rows - 1) / rows);
      } else if (!g.wide && sc::gather_lds_f32(N, w, p->km, p->view.max_pslots, p->view.max_pvals)) {
        d = "gather_kernel km=" + std::to_string(p->km) + " V=" + std::to_string(N) + " waves=" +
            std::to_string(w) + " grid=" + std::to_string(p->npanels);
      } else {
        d = std::string(g.wide ? "wide_kernel" : "panel_kernel") + " km=" + std::to_string(p->km) + " V=" +
            std::to_string(g.V) + (g.wide ? "" : " L=" + std::to_string(g.L)) + " stage=" +
            std::to_string(g.stage ? 1 : 0) + " waves=" + std::to_string(w) + " grid=" + std::to_string(p->npanels) +
            (g.ny > 1 ? "x" + std::to_string(g.ny) : "");
      }
    }
    if (p->rows_of_km > 1) d += " (rows of km=" + std::to_string(p->rows_of_km) + ")";
    if (d.size() + 1 > buflen) throw sc::Error{SC_ERR_ARG, "buffer too small"};
    std::memcpy(buf, d.c_str(), d.size() + 1);
  });
}

int sc_spmm(const sc_plan *plan, const float *dB, float *dC, int32_t N, int32_t flags,
            int32_t waves_per_panel, void *hip_stream) {
  SC_GUARD([&] {
    if (flags & ~SC_ACCUMULATE) throw sc::Error{SC_ERR_ARG, "unknown flags"};
    if (!plan) throw sc::Error{SC_ERR_ARG, "null plan"};
    if (N >= 1 && launch_band(plan, dB, dC, N, flags, hip_stream, plan->band_work, plan->band_cnt,
                              plan->band_work_floats, plan->band_cnt_n))
      return;
    if (N >= 1) plan = layout_for(plan, N);
    launch(plan, plan->gen.rec, (sc_gen_launch_fn)plan->gen.launch, dB, dC, N, flags, waves_per_panel, hip_stream);
  });
}

int sc_spmm_noalloc(const sc_plan *plan, const float *dB, float *dC, int32_t N, int32_t flags,
                    int32_t waves_per_panel, void *hip_stream) {
  SC_GUARD([&] {
    if (flags & ~SC_ACCUMULATE) throw sc::Error{SC_ERR_ARG, "unknown flags"};
    if (!plan) throw sc::Error{SC_ERR_ARG, "null plan"};
    int dev = -1;
    hip_check(hipGetDevice(&dev), "hipGetDevice");
    if (dev != plan->device) throw sc::Error{SC_ERR_ARG, "plan lives on another device than the current one"};
    unsigned char *base = scratch_base(dev);
    const Scratch sc{(float *)base, sc::kSplitWorkFloats, (unsigned *)(base + kScratchWorkBytes), sc::kSplitCounters};
    // the tiled kernel sizes its K split to the plan's workspace, which this
    // scratch holds, so its launches match sc_spmm's; the band kernel's K
    // split is the plan's, and a launch whose partial sums or counters exceed
    // the scratch is refused
    if (N >= 1 && plan->band.img) {
      const sc::BandGeometry want = sc::band_geometry(plan->band, N, plan->band_work_floats, plan->band_cnt_n);
      if (want.use && (want.work_floats > kScratchWorkFloats || (size_t)want.counters > sc::kSplitCounters))
        throw sc::Error{SC_ERR_UNSUPPORTED, "the band kernel would need more than the " +
                                                std::to_string(kScratchBytes) + "-byte static scratch"};
      if (want.use && launch_band(plan, dB, dC, N, flags, hip_stream, sc.work, sc.counters, kScratchWorkFloats,
                                  sc::kSplitCounters, true))
        return;
    }
    if (N >= 1) plan = layout_for(plan, N);
    launch(plan, plan->gen.rec, (sc_gen_launch_fn)plan->gen.launch, dB, dC, N, flags, waves_per_panel, hip_stream,
           &sc);
  });
}

int sc_spmm_generated(const sc_plan *plan, const sc_gen_record *rec, sc_gen_launch_fn fn, const float *dB,
                      float *dC, int32_t N, int32_t flags, int32_t waves_per_panel, void *hip_stream) {
  SC_GUARD([&] {
    if (flags & ~SC_ACCUMULATE) throw sc::Error{SC_ERR_ARG, "unknown flags"};
    if (!plan) throw sc::Error{SC_ERR_ARG, "null plan"};
    if (N >= 1 && rec && rec->rows_launch && layout_for(plan, N) != plan) {
      // the unit fits the file's layout, and its one-row body runs the same
      // slots re-laid as one-row panels
      check_record(plan, rec, N);
      static const uint32_t one = 1u;
      const sc_gen_record rows_rec = {1, 1, 0, 1, rec->variant, &one, nullptr};  // waves chosen per launch
      launch(plan->rows, &rows_rec, rec->rows_launch, dB, dC, N, flags, waves_per_panel, hip_stream);
      return;
    }
    launch(plan, rec, fn, dB, dC, N, flags, waves_per_panel, hip_stream);
  });
}

int sc_spmv(const sc_plan *plan, const float *dx, float *dy, int32_t flags, void *hip_stream) {
  SC_GUARD([&] {
    if (flags & ~SC_ACCUMULATE) throw sc::Error{SC_ERR_ARG, "unknown flags"};
    if (!plan) throw sc::Error{SC_ERR_ARG, "null plan"};
    plan = layout_for(plan, 1);
    launch(plan, plan->gen.rec, (sc_gen_launch_fn)plan->gen.launch, dx, dy, 1, flags, 0, hip_stream);
  });
}

int sc_spmm_f16(const sc_plan *plan, const void *dB, void *dC, int32_t N, int32_t flags,
                int32_t waves_per_panel, void *hip_stream) {
  SC_GUARD([&] {
    if (flags & ~SC_ACCUMULATE) throw sc::Error{SC_ERR_ARG, "unknown flags"};
    if (!plan) throw sc::Error{SC_ERR_ARG, "null plan"};
    if (!plan->view.vals16)
      throw sc::Error{SC_ERR_ARG, "plan has no binary16 values (create it with SC_PLAN_F16_VALUES)"};
    if (!(N == 1 || N == 2 || N == 4))
      throw sc::Error{SC_ERR_UNSUPPORTED, "the binary16 path takes N = 1, 2 or 4"};
    if (!dB || !dC) throw sc::Error{SC_ERR_ARG, "null device buffer"};
    if ((uintptr_t)dB % (2 * N) || (uintptr_t)dC % 2)
      throw sc::Error{SC_ERR_ARG, "B must be aligned to 2*N bytes and C to 2 bytes"};
    if (waves_per_panel < 0 || waves_per_panel > 16) throw sc::Error{SC_ERR_ARG, "waves per panel must be 0..16"};
    int dev = -1;
    hip_check(hipGetDevice(&dev), "hipGetDevice");
    if (dev != plan->device) throw sc::Error{SC_ERR_ARG, "plan lives on another device than the current one"};
    // the one-row layout under the same rule as sc_spmm, when its rows fit
    // the binary16 path's LDS staging
    const sc_plan *r = layout_for(plan, N);
    if (r != plan) {
      const int wr = waves_per_panel ? waves_per_panel : auto_waves(r, N);
      if (r->view.vals16 && sc::gather_lds(N, wr, r->km, r->view.max_pslots, r->view.max_pvals)) plan = r;
    }
    int w = waves_per_panel ? waves_per_panel : auto_waves(plan, N);
    if (!sc::gather_lds(N, w, plan->km, plan->view.max_pslots, plan->view.max_pvals))
      throw sc::Error{SC_ERR_UNSUPPORTED, "a panel of this plan does not fit the binary16 path's LDS staging"};
    hip_check(plan->gen.launch_f16(&plan->view, dB, dC, N, (flags & SC_ACCUMULATE) ? 1 : 0, w,
                                   (hipStream_t)hip_stream),
              "binary16 pattern kernel launch");
  });
}

void sc_plan_destroy(sc_plan *plan) {
  if (!plan) return;
  sc_plan_destroy(plan->rows);
  if (plan->dmem) (void)hipFree(plan->dmem);
  if (plan->work) (void)hipFree(plan->work);
  if (plan->tcount) (void)hipFree(plan->tcount);
  if (plan->band_mem) (void)hipFree(plan->band_mem);
  if (plan->band_work) (void)hipFree(plan->band_work);
  if (plan->band_cnt) (void)hipFree(plan->band_cnt);
  delete plan;
}

}  // extern "C"
