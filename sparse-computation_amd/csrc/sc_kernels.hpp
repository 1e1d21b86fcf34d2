// sc_kernels.hpp -- hand-written gfx950 building blocks of the pattern kernels.
//
// The code generators (code_gen/main_spmm.py, main_spmm_small_b_col.py,
// main_spmv.py) emit one straight-line device function per enumerated
// pattern and a `switch` over the pattern masks; this header supplies what
// those functions are made of and the panel kernel that calls them.
//
// Execution model (wave64, CDNA4):
//   * one workgroup owns one row panel of km rows, so every C row is written
//     by exactly one workgroup -- no atomics, no pre-zeroed C (the reference
//     launches one block per (panel, pattern) and atomically adds into a
//     zeroed C: example_cuda/spmm_demo_gpu_utils.h:1357-1416);
//   * the panel's slots (all its pattern segments, concatenated) are split
//     between the W waves of the workgroup in pack-aligned ranges;
//   * inside a wave, lanes are (slot sub-lane s, column group g): L lanes of a
//     slot cover N columns with V floats each (V = 4, 2, 1 -> dwordx4/x2/x1
//     loads of the B row), and S = 64 / L slots are in flight per step;
//   * per lane the C tile is acc[KM][V] in VGPRs; a pattern body adds
//     value(slot,row) * B[col(slot), c0 .. c0+V) into the rows of its mask
//     only, with the row indices compile-time constants;
//   * the S slot sub-lanes are reduced into the first lanes with DPP row
//     shifts and the gfx950 lane swaps (v_permlane16_swap, v_permlane32_swap),
//     then the W waves through LDS in a fixed order, so results are
//     deterministic run to run.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <type_traits>

#include "sc_api.h"

namespace sc {

// Buffer descriptor word 3 for gfx9-family untyped loads (32-bit data format).
constexpr int kBufferWord3 = 0x00020000;
// Cache-policy operand of the buffer-load builtins: SC1 (system coherence
// bit of gfx940-family loads and stores).
constexpr int kCachePolicySc1 = 16;
// Cache-policy operand: NT (non-temporal: the line is not kept for reuse).
constexpr int kCachePolicyNt = 2;

// Clang vector types (HIP's float2/float4 classes cannot be assigned in
// LDS address space 3).
typedef float vec2f __attribute__((ext_vector_type(2)));
typedef float vec4f __attribute__((ext_vector_type(4)));
typedef int vec4i __attribute__((ext_vector_type(4)));

// Device view of a plan: the .cfmtx flattened panel-major.
struct DevView {
  const int4 *seg;        // per segment {rowmask, slot_begin, nslots, val_begin}
  const int *panel_seg;   // [npanels + 1] segment range of each panel
  const int *panel_slot;  // [npanels + 1] slot range of each panel
  const int *panel_val;   // [npanels + 1] value range of each panel
  const int *cols;        // [nslots] B row (column of A) of every slot
  const float *vals;      // [nvals] pop values per slot, ascending panel row
  int M;                  // rows of A / C
  int K;                  // columns of A / rows of B
  int km;                 // rows per panel
  int npanels;
  int max_pslots;         // most slots in one panel
  int max_pvals;          // most values in one panel
  // K-block copy of the stream for the tiled and chunk kernels (null if the
  // plan was not created for them): for K block kb and panel p the
  // sub-segments (the part of each segment whose columns fall in the block)
  // are tseg[kp_seg[r] .. kp_seg[r+1]), their slots and values contiguous in
  // tcols / tvals.  Record r of (kb, p) is kb*(npanels+1)+p for the chunk
  // kernel (kblock_kind 2) and (rb*tnkb+kb)*tppb + p - rb*tppb, rb = p/tppb,
  // for the tiled kernel (kblock_kind 1: row-block-major, so one unit's
  // stream is contiguous; one sentinel record at the end).
  const int4 *tseg;       // {rowmask, slot_begin, nslots, val_begin} in tcols/tvals
  const int *kp_seg;      // first sub-segment of each record (+ end)
  const int *kp_slot;     // first tcols slot of each record (+ end)
  const int *kp_val;      // first tvals value of each record (+ end)
  const int *tcols;
  const float *tvals;
  int tkb;                // B rows per K block
  int tnkb;               // K blocks
  int tppb;               // panels per workgroup
  int tnrb;               // row blocks
  int tstage_cols;        // most slots of one (row block, K block) unit
  int tstage_vals;        // most values of one unit
  int tstage_segs;        // most sub-segments of one unit
  int tchunk_dw;          // tiled kernel: most dwords of one (row block, K tile) chunk
  const int *timg;        // tiled kernel: chunk images, row-block-major (LDS layout)
  const int *toff;        // tiled kernel: first dword of chunk rb * tnkb + kb (+ end)
  long long nslots;       // slots of the whole plan
  float *work;            // split-K partial sums (plan workspace), or null
  long long work_floats;  // its size in floats
  unsigned *tcount;       // split-K arrival counters (zero between launches), or null
  long long tcount_n;     // their number
  int kblock_kind;        // what the K-block-major copy was built for: 0 none,
                          // 1 the split-K tiled kernel, 2 the chunk kernel
  const _Float16 *vals16; // binary16 copy of vals (SC_PLAN_F16_VALUES), or null
  long long a_bytes;      // bytes of the plan's column and value streams
  const int *row_len;     // km = 1 plans: slots of each panel (row) that its segment
                          // holds, without the 16-byte alignment padding; else null
  const int *launch;      // [npanels * kLaunchInts] the panel and wide kernels' workgroups
                          // in launch order (PanelLaunch), one row per workgroup
};

// A row of DevView::launch: the panel that workgroup x runs and its ranges, so a
// workgroup finds all of them in one 32-byte scalar load.  Workgroups x,
// x + C, x + 2C, ... (C the GPU's CU count) share a CU when the grid fits
// the GPU at once (the dispatcher deals workgroups to the CUs in turn), so
// the plan orders the panels to even out the slots each CU gathers (longest
// panel first onto the least loaded CU).
struct PanelLaunch {
  int panel, slot0, slot1, seg0, seg1, val0, val1, pad;
};
constexpr int kLaunchInts = 8;
static_assert(sizeof(PanelLaunch) == kLaunchInts * sizeof(int), "one 32-byte row per workgroup");

// Chunk kernel: columns of B per chunk, B rows per K block (LDS tile), and
// panels per row group (waves per workgroup).
constexpr int kChunkCols = 32;
constexpr int kChunkTileRows = 512;
constexpr int kChunkPanels = 16;

// The segment descriptors of a panel, descriptor i of a group of up to 64 in
// lane i: one vector load per group instead of a scalar round trip per
// segment; the generated dispatchers read each back as scalars (readlane).
// A panel's segments are in descending row-mask order (the plan sorts them),
// the order in which the dispatchers visit the patterns.
struct SegLanes {
  int x, y, z, w;
  __device__ __forceinline__ vec4i operator()(int i) const {
    return vec4i{__builtin_amdgcn_readlane(x, i), __builtin_amdgcn_readlane(y, i),
                 __builtin_amdgcn_readlane(z, i), __builtin_amdgcn_readlane(w, i)};
  }
};

__device__ __forceinline__ SegLanes load_seg_lanes(const int4 *__restrict__ seg, int s0, int n) {
  const int l = __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
  SegLanes r{0, 0, 0, 0};
  if (l < n) {
    const int4 d = seg[s0 + l];
    r.x = d.x;
    r.y = d.y;
    r.z = d.z;
    r.w = d.w;
  }
  return r;
}

// Everything a pattern body needs for one (segment, wave) range.
struct SegArgs {
  const int *__restrict__ cols;
  const float *__restrict__ vals;
  const float *__restrict__ Bc;  // B + c0 (first column of this lane's group)
  int N;                         // columns of B and C
  int lo, hi;                    // slot range [lo, hi) of this wave in the segment
  int sb;                        // first slot of the segment
  int vb;                        // first value of the segment
  int s, S;                      // slot sub-lane and number of sub-lanes
  bool cval;                     // this lane's column group lies inside N
};

// Body arguments with the slot mapping of the pattern bodies fixed: blocked
// (a lane group runs a contiguous block of a segment's slots, whose columns
// and values sit at constant offsets from one LDS address) when the panel is
// staged in LDS; interleaved when the bodies read columns and values from
// memory, where the S lane groups' reads then share one cache line.
template <class A, bool BLOCKED>
struct Mapped : A {
  static constexpr bool kBlocked = BLOCKED;
};

// Lanes whose column group lies past N read the last full group instead
// (Bc clamped, always in bounds) and are never stored, so the loads need no
// branch.
template <int V>
__device__ __forceinline__ void load_b(float (&b)[V], const SegArgs &a, int col) {
  const float *p = a.Bc + (size_t)col * (size_t)a.N;
  if constexpr (V == 4) {
    const float4 t = *reinterpret_cast<const float4 *>(p);
    b[0] = t.x;
    b[1] = t.y;
    b[2] = t.z;
    b[3] = t.w;
  } else if constexpr (V == 2) {
    const float2 t = *reinterpret_cast<const float2 *>(p);
    b[0] = t.x;
    b[1] = t.y;
  } else {
    b[0] = *p;
  }
}

// The same body arguments with B read through a buffer descriptor (B below
// 2 GiB, K below 2^24): the B-row offset is one full-rate 24-bit
// multiply-add (row * N * 4 plus the lane's column bytes), not 64-bit
// pointer arithmetic.
struct SegArgsBuf : SegArgs {
  __amdgpu_buffer_rsrc_t Bbuf;  // whole B
  unsigned voff;                // this lane's (clamped) column group, bytes
  unsigned row_bytes;           // N * 4
};

// A byte offset past every B the buffer path takes (B below 2 GiB): a buffer
// load from it returns zeros without touching memory.
constexpr unsigned kBufferOutOfRange = 0x80000000u;

template <int V>
__device__ __forceinline__ void load_b_at(float (&b)[V], const SegArgsBuf &a, unsigned off) {
  if constexpr (V == 4) {
    const float4 t = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(a.Bbuf, off, 0, 0));
    b[0] = t.x;
    b[1] = t.y;
    b[2] = t.z;
    b[3] = t.w;
  } else if constexpr (V == 2) {
    const float2 t = __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(a.Bbuf, off, 0, 0));
    b[0] = t.x;
    b[1] = t.y;
  } else {
    b[0] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(a.Bbuf, off, 0, 0));
  }
}

template <int V>
__device__ __forceinline__ void load_b(float (&b)[V], const SegArgsBuf &a, int col) {
  load_b_at<V>(b, a, __umul24((unsigned)col, a.row_bytes) + a.voff);
}

// load_b for the last batch of a segment's slot loop: a lane whose slot lies
// past the segment (ok false; col is then a column in range) gets a zero row.
// Through the buffer descriptor the load itself returns the zeros; the other
// sources read the in-range row and clear it.
template <int V, class A>
__device__ __forceinline__ void load_b_tail(float (&b)[V], const A &a, int col, bool ok) {
  if constexpr (std::is_base_of<SegArgsBuf, A>::value) {
    // col is pinned (an empty asm) so that its read stays ahead of the
    // select instead of moving into a branch of its own that waits on it
    asm volatile("" : "+v"(col));
    load_b_at<V>(b, a, ok ? __umul24((unsigned)col, a.row_bytes) + a.voff : kBufferOutOfRange);
  } else {
    load_b<V>(b, a, col);
#pragma unroll
    for (int e = 0; e < V; ++e) b[e] = ok ? b[e] : 0.f;
  }
}

// Arguments of a lanes-over-slots body whose B rows come from a chunk of B
// resident in LDS: rows k0 .. k0+KT-1, kChunkCols columns, row-major.
struct ChunkArgs {
  const int *__restrict__ cols;
  const float *__restrict__ vals;
  const char *lds;    // the B chunk in LDS
  int k0;             // its first B row
  unsigned lane_off;  // column group * V * 4 bytes
  int lo, hi;         // slot range [lo, hi) of the segment inside the tile
  int sb;             // first slot of the segment
  int vb;             // first value of the segment
  int s;              // slot sub-lane
  // sub-lanes per wave (V = 4: 8 lanes per slot); a compile-time constant so
  // that the bodies' slot loops need no division for their trip counts
  static constexpr int S = 64 / (kChunkCols / 4);
  static constexpr bool kBlocked = false;  // slots interleaved over the lane groups
};

template <int V>
__device__ __forceinline__ void load_b(float (&b)[V], const ChunkArgs &a, int col) {
  static_assert(V == 4, "the chunk kernel runs V = 4 (ChunkArgs::S assumes it)");
  const float *p = reinterpret_cast<const float *>(
      a.lds + ((unsigned)(col - a.k0) * (unsigned)(kChunkCols * sizeof(float)) + a.lane_off));
  if constexpr (V == 4) {
    const float4 t = *reinterpret_cast<const float4 *>(p);
    b[0] = t.x;
    b[1] = t.y;
    b[2] = t.z;
    b[3] = t.w;
  } else if constexpr (V == 2) {
    const float2 t = *reinterpret_cast<const float2 *>(p);
    b[0] = t.x;
    b[1] = t.y;
  } else {
    b[0] = *p;
  }
}

// x if ok, else 0; x is an argument, so it is read whatever ok is (a select,
// not a branch around the read).
__device__ __forceinline__ float keep_if(bool ok, float x) { return ok ? x : 0.f; }

template <int V>
__device__ __forceinline__ void fma_row(float (&acc)[V], float v, const float (&b)[V]) {
#pragma unroll
  for (int e = 0; e < V; ++e) acc[e] = __builtin_fmaf(v, b[e], acc[e]);
}

// The value of lane l + OFF (OFF a power of two up to 32) for the lanes a
// reduction into the low lanes reads, without an LDS round trip:
//   OFF < 16: a DPP row shift (row_shl: lane l reads lane l + OFF of its row of
//             16; the add it feeds takes the DPP operand directly);
//   OFF = 16: v_permlane16_swap (rows 0 and 2 read rows 1 and 3);
//   OFF = 32: v_permlane32_swap (lanes 0..31 read lanes 32..63).
// The lane swaps are written as inline asm: with only the second result of
// __builtin_amdgcn_permlane{16,32}_swap used, the compiler of this image read
// the first one (measured: sums came out wrong), while the instruction itself
// behaves as documented (rows 1 and 3 of the second operand end in rows 0 and
// 2 of it; checked lane by lane on MI355X).  The s_nop covers the wait the
// compiler itself places between a VALU write and these instructions.
template <int OFF>
__device__ __forceinline__ float lane_down(float x) {
  static_assert(OFF == 1 || OFF == 2 || OFF == 4 || OFF == 8 || OFF == 16 || OFF == 32, "power of two up to 32");
  unsigned a = __builtin_bit_cast(unsigned, x), b = a;
  if constexpr (OFF < 16) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, (int)a, 0x100 + OFF, 0xf, 0xf, true));
  } else if constexpr (OFF == 16) {
    asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
    return __builtin_bit_cast(float, b);
  } else {
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
    return __builtin_bit_cast(float, b);
  }
}

// Sum of the S slot sub-lanes (lanes g, g+L, g+2L, ..., L a power of two) into
// lanes 0..L-1, in the pairing order of a butterfly (offsets L, 2L, ..., 32);
// the other lanes are left with partial sums.
template <int KM, int V>
__device__ __forceinline__ void reduce_slot_lanes(float (&acc)[KM][V], int L) {
#define SC_REDUCE_STEP(OFF)                                                      \
  if (L <= OFF) {                                                                \
    _Pragma("unroll") for (int r = 0; r < KM; ++r)                               \
      _Pragma("unroll") for (int e = 0; e < V; ++e) acc[r][e] += lane_down<OFF>(acc[r][e]); \
  }
  SC_REDUCE_STEP(1)
  SC_REDUCE_STEP(2)
  SC_REDUCE_STEP(4)
  SC_REDUCE_STEP(8)
  SC_REDUCE_STEP(16)
  SC_REDUCE_STEP(32)
#undef SC_REDUCE_STEP
}

template <int V>
__device__ __forceinline__ void store_c(float *dst, const float (&v)[V], int accumulate) {
  if constexpr (V == 4) {
    float4 t = make_float4(v[0], v[1], v[2], v[3]);
    if (accumulate) {
      float4 o = *reinterpret_cast<const float4 *>(dst);
      t.x += o.x;
      t.y += o.y;
      t.z += o.z;
      t.w += o.w;
    }
    *reinterpret_cast<float4 *>(dst) = t;
  } else if constexpr (V == 2) {
    float2 t = make_float2(v[0], v[1]);
    if (accumulate) {
      float2 o = *reinterpret_cast<const float2 *>(dst);
      t.x += o.x;
      t.y += o.y;
    }
    *reinterpret_cast<float2 *>(dst) = t;
  } else {
    *dst = accumulate ? *dst + v[0] : v[0];
  }
}

// Pin a loaded value in its registers (an empty asm that may "modify" it):
// the compiler must finish the load before this point and cannot sink the
// load into the guarded store that uses it, which would serialise a batch of
// loads into load-wait-store round trips.
__device__ __forceinline__ void keep(float &x) { asm volatile("" : "+v"(x)); }
__device__ __forceinline__ void keep(int &x) { asm volatile("" : "+v"(x)); }
__device__ __forceinline__ void keep(float2 &x) { asm volatile("" : "+v"(x.x), "+v"(x.y)); }
__device__ __forceinline__ void keep(float4 &x) {
  asm volatile("" : "+v"(x.x), "+v"(x.y), "+v"(x.z), "+v"(x.w));
}
__device__ __forceinline__ void keep(int4 &x) {
  asm volatile("" : "+v"(x.x), "+v"(x.y), "+v"(x.z), "+v"(x.w));
}
__device__ __forceinline__ void keep(vec4i &x) { asm volatile("" : "+v"(x)); }
__device__ __forceinline__ void keep(vec4f &x) { asm volatile("" : "+v"(x)); }

// Copy n elements global -> LDS with every thread keeping UNR loads in flight
// (a plain strided loop waits for each load before the next).
// Loads past the end re-read element n-1 (in bounds) so that the registers
// are written unconditionally; only the stores are guarded.
template <int UNR, class T>
__device__ __forceinline__ void stage_copy(T *dst, const T *__restrict__ src, int n) {
  if (n <= 0) return;
  const int step = blockDim.x;
  for (int base = threadIdx.x; base < n; base += step * UNR) {
    T r[UNR];
#pragma unroll
    for (int u = 0; u < UNR; ++u) {
      // streamed once: non-temporal, so it does not push B rows out of L2
      if constexpr (sizeof(T) == 4) r[u] = __builtin_nontemporal_load(&src[min(base + u * step, n - 1)]);
      else r[u] = src[min(base + u * step, n - 1)];
    }
#pragma unroll
    for (int u = 0; u < UNR; ++u) keep(r[u]);
#pragma unroll
    for (int u = 0; u < UNR; ++u)
      if (base + u * step < n) dst[base + u * step] = r[u];
  }
}

// Two such copies (a panel's column indices and its values) with the loads
// of both in flight together: one memory round trip per pass instead of one
// per array.
template <int U1, int U2, class T1, class T2>
__device__ __forceinline__ void stage_copy2(T1 *d1, const T1 *__restrict__ s1, int n1, T2 *d2,
                                            const T2 *__restrict__ s2, int n2) {
  const int step = blockDim.x;
  for (int pass = 0;; ++pass) {
    const int b1 = threadIdx.x + pass * step * U1;
    const int b2 = threadIdx.x + pass * step * U2;
    if (b1 >= n1 && b2 >= n2) break;
    T1 r1[U1];
    T2 r2[U2];
    if (n1 > 0) {
#pragma unroll
      for (int u = 0; u < U1; ++u) r1[u] = __builtin_nontemporal_load(&s1[min(b1 + u * step, n1 - 1)]);
    }
    if (n2 > 0) {
#pragma unroll
      for (int u = 0; u < U2; ++u) r2[u] = __builtin_nontemporal_load(&s2[min(b2 + u * step, n2 - 1)]);
    }
#pragma unroll
    for (int u = 0; u < U1; ++u) keep(r1[u]);
#pragma unroll
    for (int u = 0; u < U2; ++u) keep(r2[u]);
#pragma unroll
    for (int u = 0; u < U1; ++u)
      if (b1 + u * step < n1) d1[b1 + u * step] = r1[u];
#pragma unroll
    for (int u = 0; u < U2; ++u)
      if (b2 + u * step < n2) d2[b2 + u * step] = r2[u];
  }
}

// A panel's columns and values (16-byte aligned, lengths multiples of 4:
// the plan pads every panel) copied to LDS with 16-byte loads, a quarter of
// the requests of 4-byte ones.
__device__ __forceinline__ void stage_panel(int *lc, const int *__restrict__ cols, int nc, float *lv,
                                            const float *__restrict__ vals, int nv) {
  stage_copy2<1, 2>(reinterpret_cast<vec4i *>(lc), reinterpret_cast<const vec4i *>(cols), nc / 4,
                    reinterpret_cast<vec4f *>(lv), reinterpret_cast<const vec4f *>(vals), nv / 4);
}

// The panel kernel (any N; lane groups of L lanes per slot, S = 64/L slots
// in flight per wave).  D is the generated dispatcher: D::run<KM, V>(mask,
// acc, args) runs the straight-line body of the pattern whose row mask is
// `mask`.  blockDim.x = 64 * W.  With STAGE the panel's columns and values
// are first copied to LDS (batched loads), and the same LDS is reused for the
// cross-wave reduction.
template <int KM, int V, bool STAGE, class D, class A>
__global__ void __launch_bounds__(1024)
    panel_kernel(const int4 *__restrict__ seg, const PanelLaunch *__restrict__ launch,
                 const int *__restrict__ cols, const float *__restrict__ vals,
                 const float *__restrict__ B, float *__restrict__ C, int M, int K, int N, int L,
                 int accumulate, int pack, int stage_cols) {
  extern __shared__ float red[];
  const PanelLaunch pl = launch[blockIdx.x];
  const int panel = pl.panel;
  const int W = blockDim.x >> 6;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int S = 64 / L;
  const int g = lane & (L - 1);
  const int s = lane / L;
  const int p0 = pl.slot0;
  const int p1 = pl.slot1;
  // pack-aligned share of the panel's slots for this wave
  const int npk = (p1 - p0 + pack - 1) / pack;
  const int per = ((npk + W - 1) / W) * pack;
  const int a0 = p0 + w * per;
  const int a1 = min(p1, a0 + per);
  const int sg0 = pl.seg0;
  const int sg1 = pl.seg1;
  const int row0 = panel * KM;
  const int LV = L * V;
  const int *cs = cols;
  const float *vs = vals;
  // LDS: the cross-wave reduction area (W * KM * L * V floats), then the
  // staged stream, so the reduction never overwrites the stream
  const int red_floats = W > 1 ? W * KM * LV : 0;  // as sized by geometry()
  auto stage = [&]() {
    const int q0 = pl.val0;
    const int q1 = pl.val1;
    int *lc = reinterpret_cast<int *>(red + red_floats);
    float *lv = red + red_floats + stage_cols;
    stage_panel(lc, cols + p0, p1 - p0, lv, vals + q0, q1 - q0);
    __syncthreads();
    cs = lc - p0;  // indexed with global slot numbers
    vs = lv - q0;
  };
  // The panel's first 64 segment descriptors (all of them, nearly always)
  // load together with the stream rather than after the stage barrier, and
  // serve every N chunk.
  const SegLanes first = load_seg_lanes(seg, sg0, min(64, sg1 - sg0));
  if constexpr (STAGE) stage();
  // N chunks of LV columns: this workgroup's are blockIdx.y, + gridDim.y, ...
  const int cstride = (int)gridDim.y * LV;
  for (int cbase = (int)blockIdx.y * LV; cbase < N; cbase += cstride) {
    const int c0 = cbase + g * V;
    const int cl = min(c0, N - V);  // lanes past N read the last group, never stored
    Mapped<A, STAGE> args;
    args.cols = cs;
    args.vals = vs;
    args.Bc = B + cl;
    args.N = N;
    args.s = s;
    args.S = S;
    args.cval = c0 < N;
    if constexpr (std::is_same<A, SegArgsBuf>::value) {
      args.Bbuf = __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(B), (short)0,
                                                    (int)((size_t)K * N * sizeof(float)), kBufferWord3);
      args.voff = (unsigned)(cl * sizeof(float));
      args.row_bytes = (unsigned)(N * sizeof(float));
    }
    float acc[KM][V];
#pragma unroll
    for (int r = 0; r < KM; ++r)
#pragma unroll
      for (int e = 0; e < V; ++e) acc[r][e] = 0.f;
    for (int g = sg0; g < sg1; g += 64) {
      const int n = min(64, sg1 - g);
      D::template run_segs<KM, V>(g == sg0 ? first : load_seg_lanes(seg, g, n), n, a0, a1, acc, args);
    }
    reduce_slot_lanes<KM, V>(acc, L);
    if (W == 1) {
      if (s == 0 && c0 < N) {
#pragma unroll
        for (int r = 0; r < KM; ++r)
          if (row0 + r < M) store_c<V>(C + (size_t)(row0 + r) * N + c0, acc[r], accumulate);
      }
    } else {
      if (s == 0) {
#pragma unroll
        for (int r = 0; r < KM; ++r)
#pragma unroll
          for (int e = 0; e < V; ++e) red[(w * KM + r) * LV + g * V + e] = acc[r][e];
      }
      __syncthreads();
      for (int t = threadIdx.x; t < KM * LV; t += blockDim.x) {
        const int r = t / LV;
        const int c = t - r * LV;
        float sum = 0.f;
        for (int ww = 0; ww < W; ++ww) sum += red[(ww * KM + r) * LV + c];
        const int row = row0 + r;
        const int col = cbase + c;
        if (row < M && col < N) {
          float *dst = C + (size_t)row * N + col;
          *dst = accumulate ? *dst + sum : sum;
        }
      }
      if (cbase + cstride < N) __syncthreads();  // the next chunk reuses the reduction area
    }
  }
}

// ---------------------------------------------------------------------------
// Chunk path (N a multiple of kChunkCols, kn = 1 bodies): B reused from LDS.
// A workgroup of W waves owns (row group of W panels, N chunk of kChunkCols
// columns) and walks K in blocks of kChunkTileRows rows.  Per block it copies
// into LDS the B tile B[k0:k0+KT, n0:n0+32] and the group's slice of the
// K-block-major stream (columns and values of its panels' slots with a
// column in the block, one contiguous range), then each wave runs its
// panel's sub-segments with lanes-over-slots bodies that read columns,
// values and B rows from LDS.  Accumulators stay in registers across the K
// blocks, so C is written once, by one workgroup, without split-K.
//
// Each B row of a tile is read from L2 once per workgroup and then reused by
// every slot of the group's panels that names it, instead of one L2 gather
// per slot.  The N chunks of a row group are placed on one XCD (blocks are
// dealt to the 8 XCDs round-robin) so that the group's slice of the stream
// is fetched into that XCD's L2 once and read from there by the others.
// ---------------------------------------------------------------------------
// Copy B[k0:k0+rows, 4*n04 : 4*n04+kChunkCols] (row-major, row4 float4 per
// row) into dst, UNR float4 loads in flight per thread.  Offsets are 32-bit
// (K * N < 2^31 is checked at launch) from a uniform base.
template <int UNR>
__device__ __forceinline__ void stage_chunk(float4 *dst, const float4 *__restrict__ B4, int rows,
                                            int row4, int k0, int n04) {
  constexpr unsigned per_row = kChunkCols / 4;
  const unsigned n = (unsigned)rows * per_row;
  const unsigned step = blockDim.x;
  const float4 *src = B4 + (size_t)k0 * row4 + n04;
  for (unsigned base = threadIdx.x; base < n; base += step * UNR) {
    float4 r[UNR];
#pragma unroll
    for (int u = 0; u < UNR; ++u) {
      const unsigned i = min(base + u * step, n - 1);
      r[u] = src[(i / per_row) * (unsigned)row4 + (i % per_row)];
    }
#pragma unroll
    for (int u = 0; u < UNR; ++u) keep(r[u]);
#pragma unroll
    for (int u = 0; u < UNR; ++u)
      if (base + u * step < n) dst[base + u * step] = r[u];
  }
}

template <int KM, int V, class D>
__global__ void __launch_bounds__(1024)
    chunk_kernel(const int4 *__restrict__ tseg, const int *__restrict__ kp_seg,
                 const int *__restrict__ kp_slot, const int *__restrict__ kp_val,
                 const int *__restrict__ tcols, const float *__restrict__ tvals,
                 const float *__restrict__ B, float *__restrict__ C, int M, int K, int N, int npanels,
                 int ppg, int ngroups, int nchunks, int KT, int nkb, int stage_cols, int accumulate) {
  constexpr int L = kChunkCols / V;  // lanes per slot
  constexpr int S = 64 / L;          // slots in flight per wave
  extern __shared__ float4 smem4[];
  float4 *btile = smem4;
  // the B tile holds min(KT, K) rows (the LDS size the launch allocated)
  int *lcols = reinterpret_cast<int *>(smem4 + (size_t)min(KT, K) * (kChunkCols / 4));
  float *lvals = reinterpret_cast<float *>(lcols + stage_cols);
  // XCD-aware order: block b runs on XCD b % 8; the chunks of a row group
  // share an XCD.
  const int xcd = blockIdx.x & 7;
  const int i = blockIdx.x >> 3;
  const int g = (i / nchunks) * 8 + xcd;
  const int chunk = i % nchunks;
  if (g >= ngroups) return;  // uniform for the block, before any barrier
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int gl = lane % L;
  const int s = lane / L;
  const int p0 = g * ppg;
  const int p1 = min(npanels, p0 + ppg);
  const int panel = p0 + w;
  const bool has_panel = panel < p1;
  const int n0 = chunk * kChunkCols;

  ChunkArgs args;
  args.lds = reinterpret_cast<const char *>(btile);
  args.lane_off = (unsigned)(gl * V * sizeof(float));
  args.s = s;
  static_assert(ChunkArgs::S == S, "lanes per slot");
  float acc[KM][V];
#pragma unroll
  for (int r = 0; r < KM; ++r)
#pragma unroll
    for (int e = 0; e < V; ++e) acc[r][e] = 0.f;

  for (int kb = 0; kb < nkb; ++kb) {
    const int k0 = kb * KT;
    const int rows = min(KT, K - k0);
    const size_t base = (size_t)kb * (npanels + 1);
    const int us0 = kp_slot[base + p0], us1 = kp_slot[base + p1];
    const int uv0 = kp_val[base + p0], uv1 = kp_val[base + p1];
    if (kb > 0) __syncthreads();  // every wave is done with the previous block
    stage_chunk<8>(btile, reinterpret_cast<const float4 *>(B), rows, N / 4, k0, n0 / 4);
    stage_copy2<4, 8>(lcols, tcols + us0, us1 - us0, lvals, tvals + uv0, uv1 - uv0);
    __syncthreads();
    if (has_panel) {
      args.cols = lcols - us0;  // indexed with positions in tcols / tvals
      args.vals = lvals - uv0;
      args.k0 = k0;
      const int sg0 = kp_seg[base + panel];
      const int sg1 = kp_seg[base + panel + 1];
      for (int si = sg0; si < sg1; ++si) {
        const int4 sd = tseg[si];
        args.lo = sd.y;
        args.hi = sd.y + sd.z;
        args.sb = sd.y;
        args.vb = sd.w;
        D::template run<KM, V>(sd.x, acc, args);
      }
    }
  }
  reduce_slot_lanes<KM, V>(acc, L);
  if (has_panel && s == 0) {
    const int row0 = panel * KM;
#pragma unroll
    for (int r = 0; r < KM; ++r)
      if (row0 + r < M) store_c<V>(C + (size_t)(row0 + r) * N + n0 + gl * V, acc[r], accumulate);
  }
}

// Launch shape of the chunk kernel for N columns, or use = false.
struct ChunkGeometry {
  bool use = false;
  int W = 0;        // waves per workgroup = panels per row group
  int ngroups = 0;  // row groups
  int nchunks = 0;  // N / kChunkCols
  int KT = 0;       // B rows per LDS tile
  unsigned grid = 0;
  size_t lds = 0;
};

constexpr size_t kChunkLdsBytes = 160 * 1024;

inline ChunkGeometry chunk_geometry(const DevView &v, int N) {
  ChunkGeometry c;
  if (!v.tseg || v.kblock_kind != 2 || N % kChunkCols != 0 || v.npanels <= 0 || v.K <= 0) return c;
  if ((long long)v.K * N >= (1LL << 31)) return c;
  c.nchunks = N / kChunkCols;
  c.KT = v.tkb;
  c.W = v.tppb;
  c.ngroups = v.tnrb;
  c.lds = (size_t)std::min(v.tkb, v.K) * kChunkCols * sizeof(float) +
          ((size_t)v.tstage_cols + (size_t)v.tstage_vals) * sizeof(float);
  if (c.lds > kChunkLdsBytes) return c;
  c.grid = (unsigned)(8 * ((c.ngroups + 7) / 8) * c.nchunks);
  c.use = true;
  return c;
}

// ---------------------------------------------------------------------------
// Small-N path (N = 1, 2 or 4, one lane per slot, 64 slots per wave step).
// At these widths a panel is latency-bound: its pattern segments run one
// after another in a wave, and each would wait on its own B gather from L2.
// So the workgroup first stages the panel's values in LDS and gathers
// B[col(slot), 0..N) of every slot of the panel into LDS, all loads
// independent and in flight together; the pattern bodies then read only LDS
// (GatherArgs maps a slot number to its position in the gathered rows, so
// the generated bodies are used unchanged).
// ---------------------------------------------------------------------------
struct GatherArgs {
  struct Pos {
    int base;
    __device__ __forceinline__ int operator[](int j) const { return j - base; }
  };
  Pos cols;                        // slot number -> position in the gathered rows
  const float *__restrict__ vals;  // LDS, indexed with value numbers of the plan
  const float *gb;                 // LDS, V floats (= N) per position
  int lo, hi;                      // slot range [lo, hi) of this wave in the segment
  int sb, vb;                      // first slot / first value of the segment
  int s, S;                        // slot sub-lane (the lane) and sub-lanes (64)
  // slots interleaved over the lanes: adjacent lanes read adjacent gathered
  // rows and values, free of LDS bank conflicts
  static constexpr bool kBlocked = false;
};

template <int V>
__device__ __forceinline__ void load_b(float (&b)[V], const GatherArgs &a, int pos) {
  const float *p = a.gb + pos * V;
  if constexpr (V == 4) {
    const float4 t = *reinterpret_cast<const float4 *>(p);
    b[0] = t.x;
    b[1] = t.y;
    b[2] = t.z;
    b[3] = t.w;
  } else if constexpr (V == 2) {
    const float2 t = *reinterpret_cast<const float2 *>(p);
    b[0] = t.x;
    b[1] = t.y;
  } else {
    b[0] = *p;
  }
}

template <int V>
struct VecOf;
template <>
struct VecOf<1> {
  using T = float;
};
template <>
struct VecOf<2> {
  using T = float2;
};
template <>
struct VecOf<4> {
  using T = float4;
};

// Rows of V binary16 values, loaded as one 2-, 4- or 8-byte word.
template <int V>
struct HalfRowOf;
template <>
struct HalfRowOf<1> {
  using T = unsigned short;
};
template <>
struct HalfRowOf<2> {
  using T = unsigned int;
};
template <>
struct HalfRowOf<4> {
  using T = uint2;
};
__device__ __forceinline__ void keep(unsigned short &x) {
  unsigned int t = x;
  asm volatile("" : "+v"(t));
  x = (unsigned short)t;
}
__device__ __forceinline__ void keep(unsigned int &x) { asm volatile("" : "+v"(x)); }
__device__ __forceinline__ void keep(uint2 &x) { asm volatile("" : "+v"(x.x), "+v"(x.y)); }

__device__ __forceinline__ float half_bits_to_float(unsigned int h16) {
  return (float)__builtin_bit_cast(_Float16, (unsigned short)h16);
}

// Row of V binary16 values -> V floats (exact).
template <int V>
__device__ __forceinline__ typename VecOf<V>::T widen_row(typename HalfRowOf<V>::T r) {
  if constexpr (V == 4) {
    return make_float4(half_bits_to_float(r.x & 0xffffu), half_bits_to_float(r.x >> 16),
                       half_bits_to_float(r.y & 0xffffu), half_bits_to_float(r.y >> 16));
  } else if constexpr (V == 2) {
    return make_float2(half_bits_to_float(r & 0xffffu), half_bits_to_float(r >> 16));
  } else {
    return half_bits_to_float(r);
  }
}

// B (K x V, row-major, V == N; fp32, or binary16 when HALF) rows of the n
// slots starting at cols[0] -> dst[i] as fp32, UNR independent column loads
// and then UNR row loads in flight.
template <int V, int UNR, bool HALF>
__device__ __forceinline__ void gather_rows(typename VecOf<V>::T *dst, const int *__restrict__ cols,
                                            const void *__restrict__ B, int n) {
  using T = typename std::conditional<HALF, typename HalfRowOf<V>::T, typename VecOf<V>::T>::type;
  const T *Bv = reinterpret_cast<const T *>(B);
  const int step = blockDim.x;
  for (int base = threadIdx.x; base < n; base += step * UNR) {
    int c[UNR];
#pragma unroll
    for (int u = 0; u < UNR; ++u) c[u] = __builtin_nontemporal_load(&cols[min(base + u * step, n - 1)]);
#pragma unroll
    for (int u = 0; u < UNR; ++u) keep(c[u]);
    T r[UNR];
#pragma unroll
    for (int u = 0; u < UNR; ++u) r[u] = Bv[c[u]];
#pragma unroll
    for (int u = 0; u < UNR; ++u) keep(r[u]);
#pragma unroll
    for (int u = 0; u < UNR; ++u)
      if (base + u * step < n) {
        if constexpr (HALF) dst[base + u * step] = widen_row<V>(r[u]);
        else dst[base + u * step] = r[u];
      }
  }
}

// The fp32 small-N staging in one pipeline, with 16-byte loads: a panel's
// columns and values start on 16-byte boundaries and are padded to multiples
// of 4 (column 0, value 0), so a thread loads groups of four columns (one
// int4) and four values (one float4), gathers the four B rows as soon as the
// columns arrive (the values still in flight), then stores everything to LDS.
// U groups of each per thread are in flight.
template <int V, int U>
__device__ __forceinline__ void stage_values_gather_rows(float *lv, const float *__restrict__ vals, int nv,
                                                         typename VecOf<V>::T *gb, const int *__restrict__ cols,
                                                         const void *__restrict__ B, int nc) {
  using T = typename VecOf<V>::T;
  const T *Bv = reinterpret_cast<const T *>(B);
  const vec4i *c4 = reinterpret_cast<const vec4i *>(cols);
  const vec4f *v4 = reinterpret_cast<const vec4f *>(vals);
  vec4f *l4 = reinterpret_cast<vec4f *>(lv);
  const int nc4 = nc / 4;
  const int nv4 = nv / 4;
  const int step = blockDim.x;
  for (int base = threadIdx.x; base < nc4 || base < nv4; base += step * U) {
    vec4i c[U];
    vec4f v[U];
    T r[U][4];
    if (nc4 > 0) {
#pragma unroll
      for (int u = 0; u < U; ++u) c[u] = __builtin_nontemporal_load(&c4[min(base + u * step, nc4 - 1)]);
    }
    if (nv4 > 0) {
#pragma unroll
      for (int u = 0; u < U; ++u) v[u] = __builtin_nontemporal_load(&v4[min(base + u * step, nv4 - 1)]);
    }
    if (nc4 > 0) {
#pragma unroll
      for (int u = 0; u < U; ++u) keep(c[u]);
#pragma unroll
      for (int u = 0; u < U; ++u) {
        r[u][0] = Bv[c[u].x];
        r[u][1] = Bv[c[u].y];
        r[u][2] = Bv[c[u].z];
        r[u][3] = Bv[c[u].w];
      }
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int e = 0; e < 4; ++e) keep(r[u][e]);
#pragma unroll
      for (int u = 0; u < U; ++u)
        if (base + u * step < nc4) {
#pragma unroll
          for (int e = 0; e < 4; ++e) gb[(base + u * step) * 4 + e] = r[u][e];
        }
    }
    if (nv4 > 0) {
#pragma unroll
      for (int u = 0; u < U; ++u) keep(v[u]);
#pragma unroll
      for (int u = 0; u < U; ++u)
        if (base + u * step < nv4) l4[base + u * step] = v[u];
    }
  }
}

// n binary16 values (bits) -> fp32 in dst, UNR loads in flight per thread.
template <int UNR>
__device__ __forceinline__ void stage_half_values(float *dst, const unsigned short *__restrict__ src, int n) {
  if (n <= 0) return;
  const int step = blockDim.x;
  for (int base = threadIdx.x; base < n; base += step * UNR) {
    unsigned short r[UNR];
#pragma unroll
    for (int u = 0; u < UNR; ++u) r[u] = src[min(base + u * step, n - 1)];
#pragma unroll
    for (int u = 0; u < UNR; ++u) keep(r[u]);
#pragma unroll
    for (int u = 0; u < UNR; ++u)
      if (base + u * step < n) dst[base + u * step] = half_bits_to_float(r[u]);
  }
}

// C row segment of V values: fp32, or binary16 (rounded to nearest even)
// when HALF; with accumulate the old value is added in fp32 first.
template <int V, bool HALF>
__device__ __forceinline__ void store_row(void *C, size_t off, const float (&v)[V], int accumulate) {
  if constexpr (HALF) {
    _Float16 *c = reinterpret_cast<_Float16 *>(C) + off;
#pragma unroll
    for (int e = 0; e < V; ++e) c[e] = (_Float16)(accumulate ? (float)c[e] + v[e] : v[e]);
  } else {
    store_c<V>(reinterpret_cast<float *>(C) + off, v, accumulate);
  }
}

// HALF: values (vals16 of the plan), B and C are binary16; staging widens
// them to fp32 in LDS, the bodies accumulate in fp32 and C is rounded once.
template <int KM, int V, bool HALF, class D>
__global__ void __launch_bounds__(1024)
    gather_kernel(const int4 *__restrict__ seg, const int *__restrict__ panel_seg,
                  const int *__restrict__ panel_slot, const int *__restrict__ panel_val,
                  const int *__restrict__ cols, const void *__restrict__ vals,
                  const void *__restrict__ B, void *__restrict__ C, int M, int accumulate, int pack,
                  int stage_vals) {
  extern __shared__ float smem[];
  const int panel = blockIdx.x;
  const int W = blockDim.x >> 6;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int p0 = panel_slot[panel];
  const int p1 = panel_slot[panel + 1];
  const int npk = (p1 - p0 + pack - 1) / pack;
  const int per = ((npk + W - 1) / W) * pack;
  const int a0 = p0 + w * per;
  const int a1 = min(p1, a0 + per);
  const int sg0 = panel_seg[panel];
  const int sg1 = panel_seg[panel + 1];
  const int q0 = panel_val[panel];
  const int q1 = panel_val[panel + 1];
  const int row0 = panel * KM;
  float *lv = smem;
  float *gb = smem + stage_vals;
  if constexpr (HALF) {
    stage_half_values<8>(lv, reinterpret_cast<const unsigned short *>(vals) + q0, q1 - q0);
    gather_rows<V, 8, HALF>(reinterpret_cast<typename VecOf<V>::T *>(gb), cols + p0, B, p1 - p0);
  } else {
    stage_values_gather_rows<V, 2>(lv, reinterpret_cast<const float *>(vals) + q0, q1 - q0,
                                      reinterpret_cast<typename VecOf<V>::T *>(gb), cols + p0, B, p1 - p0);
  }
  __syncthreads();

  GatherArgs args;
  args.cols.base = p0;
  args.vals = lv - q0;
  args.gb = gb;
  args.s = lane;
  args.S = 64;
  float acc[KM][V];
#pragma unroll
  for (int r = 0; r < KM; ++r)
#pragma unroll
    for (int e = 0; e < V; ++e) acc[r][e] = 0.f;
  for (int g = sg0; g < sg1; g += 64) {
    const int n = min(64, sg1 - g);
    D::template run_segs<KM, V>(load_seg_lanes(seg, g, n), n, a0, a1, acc, args);
  }
  reduce_slot_lanes<KM, V>(acc, 1);
  if (W == 1) {
    if (lane == 0) {
#pragma unroll
      for (int r = 0; r < KM; ++r)
        if (row0 + r < M) store_row<V, HALF>(C, (size_t)(row0 + r) * V, acc[r], accumulate);
    }
  } else {
    float *red = smem;
    __syncthreads();  // every wave is done with the staged data
    if (lane == 0) {
#pragma unroll
      for (int r = 0; r < KM; ++r)
#pragma unroll
        for (int e = 0; e < V; ++e) red[(w * KM + r) * V + e] = acc[r][e];
    }
    __syncthreads();
    for (int t = threadIdx.x; t < KM * V; t += blockDim.x) {
      const int r = t / V;
      const int e = t - r * V;
      float sum = 0.f;
      for (int ww = 0; ww < W; ++ww) sum += red[(ww * KM + r) * V + e];
      const int row = row0 + r;
      if (row < M) {
        const float one[1] = {sum};
        store_row<1, HALF>(C, (size_t)row * V + e, one, accumulate);
      }
    }
  }
}

// LDS bytes of the small-N path for a plan, 0 if it does not apply.
inline size_t gather_lds(int N, int W, int km, int max_pslots, int max_pvals) {
  if (!(N == 1 || N == 2 || N == 4) || max_pslots < 0) return 0;
  const size_t sv = (size_t)(max_pvals + 3) / 4 * 4;
  const size_t st = (sv + (size_t)max_pslots * N) * sizeof(float);
  const size_t red = (size_t)W * km * N * sizeof(float);
  const size_t lds = std::max(st, red);
  return lds <= 64 * 1024 ? std::max<size_t>(lds, 16) : 0;
}

// The fp32 small-N path runs the gather kernel only for km >= 2.  Its
// reason is a panel's pattern segments waiting one after another on their
// own B gathers; a km = 1 panel has one segment, and there the lanes-over-
// slots kernel is faster (SpMV 512^2 at 30 %: 3.16 us against 3.44).  The
// binary16 path has only the gather kernel.
inline size_t gather_lds_f32(int N, int W, int km, int max_pslots, int max_pvals) {
  return km >= 2 ? gather_lds(N, W, km, max_pslots, max_pvals) : 0;
}

// ---------------------------------------------------------------------------
// Wide path (N a multiple of 64): the whole wave works on one slot at a time,
// lane l owning columns cbase + l*V .. + V-1.  Column indices and values are
// then wave-uniform: they come through the scalar cache (s_load), the B-row
// address is formed on the SALU, and the VALU only runs the FMAs.  Bodies
// unroll UW slots so UW B-row loads are in flight per wave.
// ---------------------------------------------------------------------------
constexpr int UW = 8;

struct WideArgs {
  const int *__restrict__ cols;
  const float *__restrict__ vals;
  __amdgpu_buffer_rsrc_t B;  // buffer over B + cbase (wave-uniform)
  unsigned lane_off;         // lane * V * 4 bytes
  unsigned row_bytes;        // N * 4
  int N;
  int lo, hi;  // slot range of this wave in the segment
  int sb, vb;  // first slot / first value of the segment
};


// B-row load of the wide path: the row offset col * N * 4 (< 2^32, checked at
// launch) goes into the scalar soffset of a buffer load and the lane's column
// offset into voffset, so forming the address costs no vector instruction.
template <int V>
__device__ __forceinline__ void load_row(float (&b)[V], const WideArgs &a, int col) {
  const unsigned soff = (unsigned)__builtin_amdgcn_readfirstlane(col) * a.row_bytes;
  if constexpr (V == 4) {
    const float4 t = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(a.B, a.lane_off, soff, 0));
    b[0] = t.x;
    b[1] = t.y;
    b[2] = t.z;
    b[3] = t.w;
  } else if constexpr (V == 2) {
    const float2 t = __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(a.B, a.lane_off, soff, 0));
    b[0] = t.x;
    b[1] = t.y;
  } else {
    b[0] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(a.B, a.lane_off, soff, 0));
  }
}

// One workgroup per row panel, W waves splitting its slots.  With STAGE the
// workgroup first copies the panel's column indices and values (contiguous in
// the plan) into LDS with coalesced loads, so the slot loop reads them at LDS
// latency instead of waiting on a cache miss per batch; the staging area is
// reused for the cross-wave reduction afterwards.
template <int KM, int V, bool STAGE, class D>
__global__ void __launch_bounds__(1024)
    wide_kernel(const int4 *__restrict__ seg, const PanelLaunch *__restrict__ launch,
                const int *__restrict__ cols, const float *__restrict__ vals,
                const float *__restrict__ B, float *__restrict__ C, int M, int K, int N,
                int accumulate, int pack, int stage_cols) {
  extern __shared__ float smem[];
  const PanelLaunch pl = launch[blockIdx.x];
  const int panel = pl.panel;
  const int W = blockDim.x >> 6;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int p0 = pl.slot0;
  const int p1 = pl.slot1;
  const int npk = (p1 - p0 + pack - 1) / pack;
  const int per = ((npk + W - 1) / W) * pack;
  const int a0 = p0 + w * per;
  const int a1 = min(p1, a0 + per);
  const int sg0 = pl.seg0;
  const int sg1 = pl.seg1;
  const int row0 = panel * KM;
  constexpr int CW = 64 * V;  // columns per chunk

  const int *cs = cols;
  const float *vs = vals;
  if constexpr (STAGE) {
    const int q0 = pl.val0;
    const int q1 = pl.val1;
    int *lc = reinterpret_cast<int *>(smem);
    float *lv = smem + stage_cols;
    stage_panel(lc, cols + p0, p1 - p0, lv, vals + q0, q1 - q0);
    __syncthreads();
    cs = lc - p0;  // indexed with global slot numbers
    vs = lv - q0;
  }

  for (int cbase = 0; cbase < N; cbase += CW) {
    WideArgs args;
    args.cols = cs;
    args.vals = vs;
    // bytes of B from column cbase of row 0 to the end (< 2^32, checked at launch)
    const unsigned span = (unsigned)(((size_t)K * N - cbase) * sizeof(float));
    args.B = __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(B + cbase), (short)0, (int)span,
                                               kBufferWord3);
    args.lane_off = (unsigned)(lane * V * sizeof(float));
    args.row_bytes = (unsigned)(N * sizeof(float));
    args.N = N;
    float acc[KM][V];
#pragma unroll
    for (int r = 0; r < KM; ++r)
#pragma unroll
      for (int e = 0; e < V; ++e) acc[r][e] = 0.f;
    // A wave's slot range meets only a few of the panel's segments: the
    // others are skipped on the descriptor alone (scalar loads, shared by the
    // panel's waves through the scalar cache).
    for (int si = sg0; si < sg1; ++si) {
      const int4 sd = seg[si];
      const int lo = max(sd.y, a0);
      const int hi = min(sd.y + sd.z, a1);
      if (lo < hi) {
        args.lo = lo;
        args.hi = hi;
        args.sb = sd.y;
        args.vb = sd.w;
        D::template run_wide<KM, V>(sd.x, acc, args);
      }
    }
    const int c0 = cbase + lane * V;
    if (W == 1) {
#pragma unroll
      for (int r = 0; r < KM; ++r)
        if (row0 + r < M) store_c<V>(C + (size_t)(row0 + r) * N + c0, acc[r], accumulate);
    } else {
      float *red = smem;
      if constexpr (STAGE) __syncthreads();  // every wave is done with the staged stream
#pragma unroll
      for (int r = 0; r < KM; ++r)
#pragma unroll
        for (int e = 0; e < V; ++e) red[(w * KM + r) * CW + lane * V + e] = acc[r][e];
      __syncthreads();
      for (int t = threadIdx.x; t < KM * CW; t += blockDim.x) {
        const int r = t / CW;
        const int c = t - r * CW;
        float sum = 0.f;
        for (int ww = 0; ww < W; ++ww) sum += red[(ww * KM + r) * CW + c];
        const int row = row0 + r;
        if (row < M) {
          float *dst = C + (size_t)row * N + cbase + c;
          *dst = accumulate ? *dst + sum : sum;
        }
      }
      __syncthreads();
    }
    if constexpr (STAGE) {
      if (cbase + CW < N) {  // restage: the reduction overwrote the stream
        const int q0 = pl.val0;
        const int q1 = pl.val1;
        int *lc = reinterpret_cast<int *>(smem);
        float *lv = smem + stage_cols;
        stage_panel(lc, cols + p0, p1 - p0, lv, vals + q0, q1 - q0);
        __syncthreads();
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Tiled path (N a multiple of 64): split-K with double-buffered LDS stages.
// The plan's row-block-major copy of the stream lists, for every row block of
// kTilePanels panels and K tile of kTileRows B rows, one record per panel:
// the part of each of the panel's pattern segments whose columns fall in the
// tile (its sub-segments, in descending row-mask order), with tile-relative
// columns.  The records of one (row block, tile) form a contiguous chunk.
//
// A workgroup of kTilePanels waves owns one unit = (row block, range of `tpu`
// K tiles, N chunk of 64V columns); wave w owns panel rb * kTilePanels + w.
// Each stage holds one tile's B rows and the row block's chunk for that tile
// (header, descriptors, columns, values).  While the waves run tile t from
// one stage, every thread already holds its share of tile t+1 in registers
// and writes it into the other stage afterwards: one barrier per tile, and
// the whole dependent chain of a sub-segment (descriptor, then columns and
// values, then B rows) runs at LDS latency.  Every staged B row serves all
// panels of the row block, where the panel kernels gather it from L2 once
// per slot.
//
// With more than one K range per row block, each unit writes its partial
// sums to the plan workspace and bumps the row block's counter; the unit that
// arrives last adds the partials in K-range order (the result does not depend
// on which unit is last), writes C and resets the counter for the next
// launch.  Launches that share a plan must therefore be stream-ordered.
// ---------------------------------------------------------------------------
// LDS pointers of the tiled path
typedef __attribute__((address_space(3))) float lds_float;
typedef __attribute__((address_space(3))) int lds_int;
typedef __attribute__((address_space(3))) vec2f lds_float2;
typedef __attribute__((address_space(3))) vec4f lds_float4;
typedef __attribute__((address_space(3))) vec4i lds_int4;

constexpr int kTileRows = 64;     // B rows per LDS tile
constexpr int kTilePanels = 16;   // panels per row block = waves per workgroup
// chunk header in LDS (dwords): record starts [0..kTilePanels], then the
// offsets of the columns and of the values; descriptors start at the header's
// end (16-byte aligned)
constexpr int kTileChunkHeader = 20;
constexpr int kTileHdrCols = kTilePanels + 1;
constexpr int kTileHdrVals = kTilePanels + 2;
constexpr int kTileMaxPerUnit = 63;  // K tiles of one unit, at most
constexpr size_t kTileTableBytes = 3 * (kTileMaxPerUnit + 1) * sizeof(int);  // chunk table of a unit

// Values read from LDS at a wave-uniform address are the same in every lane,
// but the compiler cannot prove it: readfirstlane makes them scalar, so the
// control flow on them stays scalar branches.
__device__ __forceinline__ int uniform(int x) { return __builtin_amdgcn_readfirstlane(x); }
__device__ __forceinline__ vec4i uniform4(vec4i x) {
  return vec4i{uniform(x.x), uniform(x.y), uniform(x.z), uniform(x.w)};
}

// The first n (<= 64) values at vp, value i in lane i (lanes >= n read
// value 0 and are never used).
__device__ __forceinline__ float batch_values(const lds_float *vp, int n) {
  const int l = __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
  return vp[l < n ? l : 0];
}
// Value i of a batch as a scalar.
__device__ __forceinline__ float lane_value(float vl, int i) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, vl), i));
}

struct TileArgs {
  const lds_int *cols;    // tile-relative B row of each slot of the chunk
  const lds_float *vals;  // values of the chunk, pop per slot
  const lds_float *tile;  // this lane's first column in the B tile
  int lo, hi;             // slot range [lo, hi) of the sub-segment (chunk-relative)
  int vb;                 // its first value (chunk-relative)
};

// B row `row` of the tile: one LDS read of V floats per lane; the address is
// one vector shift-add of the slot's row.
template <int V>
__device__ __forceinline__ void load_tile(float (&b)[V], const TileArgs &a, int row) {
  const lds_float *p = a.tile + (unsigned)row * (64u * V);
  if constexpr (V == 4) {
    const vec4f t = *reinterpret_cast<const lds_float4 *>(p);
    b[0] = t.x;
    b[1] = t.y;
    b[2] = t.z;
    b[3] = t.w;
  } else if constexpr (V == 2) {
    const vec2f t = *reinterpret_cast<const lds_float2 *>(p);
    b[0] = t.x;
    b[1] = t.y;
  } else {
    b[0] = *p;
  }
}

// Two workgroups per CU when both fit the LDS (V <= 2): registers are capped
// for 8 waves per SIMD.
template <int KM, int V, class D>
__global__ void __launch_bounds__(1024) __attribute__((amdgpu_waves_per_eu(V <= 2 ? 8 : 4)))
    tiled_kernel(const int *__restrict__ timg, const int *__restrict__ toff,
                 const float *__restrict__ B, float *__restrict__ C, float *__restrict__ work,
                 unsigned *__restrict__ counters, int M, int K, int N, int npanels, int ntiles,
                 int nks, int tpu, int chunk_dw, int accumulate) {
  extern __shared__ float4 smem4[];
  constexpr int NC = 64 * V;                // columns of the N chunk
  constexpr int Q4 = NC / 4;                // float4 per B-tile row
  constexpr int TQ = kTileRows * Q4;        // float4 of one B tile
  constexpr int NT = 64 * kTilePanels;      // threads per workgroup
  constexpr int SPT = TQ / NT;              // B float4 staged per thread (= V)
  static_assert(SPT * NT == TQ, "tile must split evenly over the workgroup");
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int ks = blockIdx.x % nks;
  const int rb = blockIdx.x / nks;
  const int n0 = blockIdx.y * NC;
  const int panel = rb * kTilePanels + w;
  const bool has_panel = panel < npanels;
  const int t0 = ks * tpu;
  const int t1 = min(ntiles, t0 + tpu);
  const int stage_q = TQ + chunk_dw / 4;    // float4 per stage (chunk_dw % 4 == 0)
  lds_float4 *lds4 = (lds_float4 *)smem4;
  const vec4i *img4 = reinterpret_cast<const vec4i *>(timg);
  // chunk table of the unit in LDS (after the two stages): first float4 of
  // every tile's chunk and of the end
  lds_int *table = (lds_int *)(lds4 + 2 * stage_q);

  // what one thread stages: V float4 of B and one float4 of the chunk; plain
  // copies, so the loads stay in flight while the current tile runs
  vec4f preb[SPT];
  vec4i prea;
  int na = 0;  // float4 of the chunk being fetched
  auto fetch = [&](int t) {
#pragma unroll
    for (int s = 0; s < SPT; ++s) {
      const int idx = (int)threadIdx.x + s * NT;
      const int r = idx / Q4;
      const int c = idx - r * Q4;
      const int row = t * kTileRows + r;
      if (row < K) preb[s] = *reinterpret_cast<const vec4f *>(B + (size_t)row * N + n0 + c * 4);
    }
    const int a0 = uniform(table[t - t0]);
    na = uniform(table[t - t0 + 1]) - a0;
    if ((int)threadIdx.x < na) prea = img4[a0 + threadIdx.x];
  };
  auto put = [&](int stage, int t) {
    lds_float4 *st = lds4 + stage * stage_q;
#pragma unroll
    for (int s = 0; s < SPT; ++s) {
      const int idx = (int)threadIdx.x + s * NT;
      if (t * kTileRows + idx / Q4 < K) st[idx] = preb[s];
    }
    if ((int)threadIdx.x < na) ((lds_int4 *)(st + TQ))[threadIdx.x] = prea;
  };

  float acc[KM][V];
#pragma unroll
  for (int r = 0; r < KM; ++r)
#pragma unroll
    for (int e = 0; e < V; ++e) acc[r][e] = 0.f;

  const int u0 = rb * ntiles + t0;
  if ((int)threadIdx.x <= t1 - t0) table[threadIdx.x] = toff[u0 + threadIdx.x] / 4;
  // Pull the unit's chunks (contiguous, row-block-major) towards this XCD's
  // L2 with one load per 64-byte line, so the stage copies of the later
  // tiles do not each wait on HBM.
  unsigned sink = 0;
  {
    const int a0 = toff[u0], a1 = toff[u0 + (t1 - t0)];
    for (int i = a0 + (int)threadIdx.x * 16; i < a1; i += NT * 16) sink += (unsigned)timg[i];
  }
  __syncthreads();
  if (t0 < t1) {
    fetch(t0);
    put(0, t0);
  }
  __syncthreads();
  TileArgs args;
  for (int t = t0; t < t1; ++t) {
    const int stage = (t - t0) & 1;
    const bool more = t + 1 < t1;
    if (more) fetch(t + 1);
    if (has_panel) {
      const lds_float4 *st = lds4 + stage * stage_q;
      const lds_int *a = (const lds_int *)(st + TQ);
      args.tile = (const lds_float *)st + lane * V;
      args.cols = a + uniform(a[kTileHdrCols]);
      args.vals = (const lds_float *)(a + uniform(a[kTileHdrVals]));
      D::template run_tile<KM, V>((const lds_int4 *)(a + kTileChunkHeader), uniform(a[w]), uniform(a[w + 1]),
                                  acc, args);
    }
    if (more) put(stage ^ 1, t + 1);
    __syncthreads();
  }
  asm volatile("" ::"v"(sink));  // keeps the prefetch loads (long complete by now)

  const int row0 = panel * KM;
  const int c0 = n0 + lane * V;
  if (nks == 1) {
    if (has_panel) {
#pragma unroll
      for (int r = 0; r < KM; ++r)
        if (row0 + r < M) store_c<V>(C + (size_t)(row0 + r) * N + c0, acc[r], accumulate);
    }
    return;
  }
  // Partial sums go out as agent-scope atomic stores and come back as
  // agent-scope atomic loads: both bypass the per-XCD L2 copies, so the hand
  // over needs no L2 write-back or invalidate (which a release / acquire
  // fence would issue, for the whole cache), only completed stores before
  // the counter is bumped.
  if (has_panel) {
#pragma unroll
    for (int r = 0; r < KM; ++r)
      if (row0 + r < M) {
        float *dst = work + ((size_t)ks * M + row0 + r) * N + c0;
#pragma unroll
        for (int e = 0; e < V; ++e) __hip_atomic_store(dst + e, acc[r][e], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
  }
  __builtin_amdgcn_s_waitcnt(0);  // this thread's partial stores have completed
  __syncthreads();
  int *flag = (int *)smem4;  // the B buffers are free after the last barrier
  unsigned *cnt = counters + rb * gridDim.y + blockIdx.y;
  if (threadIdx.x == 0) {
    const unsigned old = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *flag = old == (unsigned)(nks - 1);
  }
  __syncthreads();
  if (!*flag) return;
  // The row block's chunk of C = the nks partials summed in K-range order,
  // spread over the whole workgroup with every partial load in flight.
  const int rbase = rb * kTilePanels * KM;
  const int rows = min(kTilePanels * KM, M - rbase);
  const size_t kstride = (size_t)M * N * sizeof(float);
  const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
      work, (short)0, (int)0x7fffffff, kBufferWord3);
  for (int i = threadIdx.x; i < rows * Q4; i += NT) {
    const int r = i / Q4;
    const int c = i - r * Q4;
    // byte offsets: lane part in voffset, K range in soffset (the whole
    // workspace is below 2^31 bytes, checked at launch)
    const unsigned off = (unsigned)(((size_t)(rbase + r) * N + n0 + c * 4) * sizeof(float));
    vec4f sum;
#pragma unroll 8
    for (int k = 0; k < nks; ++k) {
      // sc1: read the partial where it was written through, not a stale
      // copy in this XCD's L2
      const vec4f p = __builtin_bit_cast(vec4f, __builtin_amdgcn_raw_buffer_load_b128(
                                                      wr, off, (unsigned)(k * kstride), kCachePolicySc1));
      sum = k == 0 ? p : sum + p;
    }
    float *dst = C + (size_t)(rbase + r) * N + n0 + c * 4;
    if (accumulate) sum += *reinterpret_cast<const vec4f *>(dst);
    *reinterpret_cast<vec4f *>(dst) = sum;
  }
  if (threadIdx.x == 0) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

constexpr size_t kLdsBytes = 160 * 1024;  // LDS per workgroup on gfx950

struct TileGeometry {
  bool use = false;
  int V = 0;        // floats per lane (64 * V columns per chunk)
  int chunks = 0;   // N chunks
  int nks = 1;      // K ranges per row block (units per row block and chunk)
  int tpu = 0;      // K tiles per unit
  int chunk_dw = 0; // stream dwords per stage (multiple of 4)
  size_t lds = 0;   // two stages
  long long work_floats = 0;  // partial sums (nks > 1)
  long long counters = 0;     // one per (row block, chunk) when nks > 1
};

// Split-K workspace of a plan (allocated with the plan, so no launch
// allocates): partial sums and arrival counters.  The tiled and band kernels
// size their K split to fit it.
constexpr size_t kSplitWorkFloats = (size_t)256 * 128 * 64;  // 8 MiB
constexpr size_t kSplitCounters = 4096;

// work_cap / counter_cap: the workspace the launch will pass (floats,
// counters); the K split shrinks until its partial sums fit.
inline TileGeometry tile_geometry(const DevView &v, int N, size_t work_cap = kSplitWorkFloats,
                                  size_t counter_cap = kSplitCounters) {
  TileGeometry t;
  if (!v.timg || v.kblock_kind != 1 || v.tkb != kTileRows || v.tppb != kTilePanels || N % 64 != 0 ||
      v.npanels <= 0 || v.tnkb <= 0 || v.tchunk_dw > 4 * 64 * kTilePanels)
    return t;
  t.use = true;
  t.V = (N % 256 == 0) ? 4 : (N % 128 == 0) ? 2 : 1;
  t.chunks = N / (64 * t.V);
  t.chunk_dw = (v.tchunk_dw + 3) / 4 * 4;
  t.lds = 2 * ((size_t)kTileRows * 64 * t.V + t.chunk_dw) * sizeof(float) + kTileTableBytes;
  if (t.lds > kLdsBytes) {
    t.use = false;
    return t;
  }
  // about two workgroups per CU in flight (one when the buffers take more
  // than half the LDS), split over the K ranges of each (row block, chunk)
  const long long target = t.lds * 2 <= kLdsBytes ? 512 : 256;
  const long long rbc = (long long)v.tnrb * t.chunks;
  int nks = (int)std::max<long long>(1, std::min<long long>(v.tnkb, (target + rbc / 2) / rbc));
  const int nks_min = (v.tnkb + kTileMaxPerUnit - 1) / kTileMaxPerUnit;
  while (nks > std::max(1, nks_min) && (size_t)nks * v.M * N > work_cap) --nks;
  nks = std::max(nks, nks_min);
  t.tpu = (v.tnkb + nks - 1) / nks;
  t.nks = (v.tnkb + t.tpu - 1) / t.tpu;
  t.work_floats = t.nks > 1 ? (long long)t.nks * v.M * N : 0;
  t.counters = t.nks > 1 ? rbc : 0;
  if (t.work_floats * (long long)sizeof(float) >= (1ll << 31)) t.use = false;  // buffer offsets
  if ((size_t)t.work_floats > work_cap || (size_t)t.counters > counter_cap) t.use = false;
  return t;
}
// Floats per lane of the wide path for N columns, 0 if N does not fit it.
inline int wide_v(int N, long long K = 0) {
  if ((long long)K * N * 4 >= (1LL << 32)) return 0;
  if (N % 256 == 0) return 4;
  if (N == 128) return 2;
  if (N == 64) return 1;
  return 0;
}

// Launch geometry for N columns: V floats per lane, L lanes per slot
// (a power of two <= 64), LDS bytes for the cross-wave reduction.
struct Geometry {
  int V, L;
  int ny = 1;         // lanes-over-slots kernel: workgroups per panel, one N chunk of L * V columns each
  bool wide;
  bool stage;         // wide path stages the panel stream in LDS
  int stage_cols;     // floats reserved for column indices in LDS
  size_t lds;
};

constexpr size_t kStageLimit = 64 * 1024;
// The wide and narrow kernels stage a panel's stream in LDS only when the
// plan's streams are at least this large: such a plan comes from HBM, where
// one batched copy per panel beats a load round trip per batch of slots
// (4096^2 at 10 %, N=128: 31.3 vs 33.6 us).  Smaller plans stay in L2 and run
// faster unstaged (FFN 2048x512 at 50 %: 11.4 vs 12.7 us; 512^2 at 10 %,
// N=32: 7.3 vs 7.9 us).
constexpr long long kStageMinBytes = 8ll << 20;
// Panels with at least this many slots on average amortize the staging copy
// even when the plan is L2-resident (lanes-over-slots kernel).
constexpr long long kLongPanelSlots = 1000;

inline Geometry geometry(int km, int N, int W, long long K = 0, int max_pslots = -1,
                         int max_pvals = -1, long long a_bytes = -1, long long avg_pslots = -1,
                         long long npanels = -1) {
  Geometry g;
  g.stage = false;
  g.stage_cols = 0;
  int wv = wide_v(N, K);
  // A plan streamed from HBM, or one with long panels, at N = 64 or 128: the
  // staged lanes-over-slots kernel with 16-byte B loads (two or four slots per
  // wave) beats the wide kernel's 8- or 4-byte ones.  Its B-row gathers are
  // bound by the number of requests in flight, not by bytes: 4096^2 at 10 %,
  // N = 128: 22.2 us against 30.9; FFN 512x2048 at 50 % (1900 slots a panel):
  // 13.8 against 17.0.  Other L2-resident plans stay wide (FFN 2048x512 at
  // 50 %, 480 slots a panel: 11.0 us against 14.3; 512x2048 at 90 %, 700
  // slots a panel: 9.1 against 9.5).
  const bool long_panels = avg_pslots >= kLongPanelSlots;
  const bool stage_fits = max_pslots >= 0 && ((size_t)(max_pslots + 3) / 4 * 4 + (size_t)max_pvals) * 4 <= kStageLimit;
  if ((wv == 1 || wv == 2) && stage_fits && (a_bytes >= kStageMinBytes || long_panels)) wv = 0;
  if (wv) {
    g.wide = true;
    g.V = wv;
    g.L = 64;
    const size_t red = W > 1 ? (size_t)W * km * 64 * wv * sizeof(float) : 0;
    g.lds = red;
    if (max_pslots >= 0 && (a_bytes < 0 || a_bytes >= kStageMinBytes)) {
      const int sc = (max_pslots + 3) / 4 * 4;
      const size_t st = ((size_t)sc + (size_t)max_pvals) * 4;
      if (st <= kStageLimit) {
        g.stage = true;
        g.stage_cols = sc;
        g.lds = st > red ? st : red;
      }
    }
    return g;
  }
  g.wide = false;
  g.V = (N % 4 == 0) ? 4 : (N % 2 == 0) ? 2 : 1;
  const int groups = (N + g.V - 1) / g.V;
  g.L = 1;
  while (g.L < groups && g.L < 64) g.L <<= 1;
  // Fewer panels than CUs and one N chunk a panel (FFN 512 x 2048: 128
  // panels, N = 128): the chunk's halves go to two workgroups, each with half
  // the lanes per slot and twice the slots in flight, so the grid covers the
  // chip; each stages the panel's stream itself.  Measured on MI355X: FFN
  // 512 x 2048 at 50 / 70 % sparsity 13.1 -> 10.0 us and 10.8 -> 8.8; four
  // workgroups a panel ran 15.9 and 14.5.
  if (npanels > 0 && npanels <= 256 && g.L >= 16 && g.L * g.V >= N) {
    g.L >>= 1;
    g.ny = 2;
  }
  const size_t red = W > 1 ? (size_t)W * km * g.L * g.V * sizeof(float) : 0;
  g.lds = red;
  if (max_pslots >= 0 && (a_bytes < 0 || a_bytes >= kStageMinBytes || long_panels)) {
    const int sc = (max_pslots + 3) / 4 * 4;
    const size_t st = ((size_t)sc + (size_t)max_pvals) * 4;
    if (st <= kStageLimit) {
      g.stage = true;
      g.stage_cols = sc;
      g.lds = st + red;  // reduction area first, then the stream (panel_kernel)
    }
  }
  return g;
}

// SpMV / narrow SpMM (N = 1, 2, 4) on one-row panels (km = 1): one wave per
// row, four rows per workgroup.  A lane reads four consecutive slots' columns
// and values with one 16-byte load each (every panel starts on a 16-byte
// boundary), gathers their four B rows (N floats each, one 4-, 8- or 16-byte
// load) and accumulates; slots past the row's last one are masked, never read
// from B; the wave reduces into lane 0 with lane swaps and DPP row shifts.  The shortest
// dependent chain a row has: its offsets, its stream, B, the store.
// Measured on MI355X against the lanes-over-slots kernel (graph replay): SpMV
// 512^2 at 70 % sparsity 2.92 -> 2.23 us, small-B 512^2 N = 1 (rows of km 4)
// 2.79 -> 2.16, structured 4096^2 N = 1 7.63 -> 7.03; non-temporal stream
// loads then took the structured case from 6.99 to 6.20 us (2.20 -> 2.07 on
// the 512^2 SpMV).
constexpr int kRowSpmvRows = 4;  // rows (waves) per workgroup
template <int V>
__device__ __forceinline__ vec4f row_of(const float *__restrict__ B, int col) {
  if constexpr (V == 4) return *reinterpret_cast<const vec4f *>(B + (size_t)col * 4);
  else if constexpr (V == 2) {
    const vec2f t = *reinterpret_cast<const vec2f *>(B + (size_t)col * 2);
    return vec4f{t.x, t.y, 0.f, 0.f};
  } else {
    return vec4f{B[col], 0.f, 0.f, 0.f};
  }
}
template <int V>
__device__ __forceinline__ vec4f row_of_lds(const lds_float *xs, int col) {
  if constexpr (V == 4) return *(const lds_float4 *)(xs + col * 4);
  else if constexpr (V == 2) {
    const vec2f t = *(const lds_float2 *)(xs + col * 2);
    return vec4f{t.x, t.y, 0.f, 0.f};
  } else {
    return vec4f{xs[col], 0.f, 0.f, 0.f};
  }
}
// STAGE: the workgroup first copies all of B (K x V floats) into LDS and the
// rows gather from there (kRowStagedRows rows a workgroup, so that a CU
// copies B about once): on a plan with many entries per B row the gathers
// then cost LDS reads instead of one L2 request each.
template <int ROWS, int V, bool STAGE>
__global__ void __launch_bounds__(64 * ROWS)
    row_spmv_kernel(const int *__restrict__ panel_slot, const int *__restrict__ panel_val,
                    const int *__restrict__ row_len, const int *__restrict__ cols,
                    const float *__restrict__ vals, const float *__restrict__ B, float *__restrict__ C, int M,
                    int K, int accumulate) {
  extern __shared__ float4 xs4[];
  lds_float *xs = (lds_float *)xs4;
  if constexpr (STAGE) {
    const int nf = K * V;
    for (int i = threadIdx.x; i < nf; i += 64 * ROWS) xs[i] = B[i];
    __syncthreads();
  }
  auto b_row = [&](int col) __attribute__((always_inline)) {
    if constexpr (STAGE) return row_of_lds<V>(xs, col);
    else return row_of<V>(B, col);
  };
  const int row = blockIdx.x * ROWS + (int)(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= M) return;
  const vec4i *c4 = reinterpret_cast<const vec4i *>(cols + panel_slot[row]);
  const vec4f *v4 = reinterpret_cast<const vec4f *>(vals + panel_val[row]);
  const int n = row_len[row];
  const int nq = (n + 3) >> 2;
  float acc[V];
#pragma unroll
  for (int k = 0; k < V; ++k) acc[k] = 0.f;
  // the stream is read once: non-temporal loads keep it from displacing B
  // and the neighbouring rows' lines in the caches
  if constexpr (V == 1) {
    // scalar B values
    auto quad = [&](const vec4i &c, const vec4f &v, int q) __attribute__((always_inline)) {
      const int e = q * 4;
      const float x0 = b_row(c.x)[0];  // e < n for every q < nq
      const float x1 = e + 1 < n ? b_row(c.y)[0] : 0.f;
      const float x2 = e + 2 < n ? b_row(c.z)[0] : 0.f;
      const float x3 = e + 3 < n ? b_row(c.w)[0] : 0.f;
      acc[0] = __builtin_fmaf(v.x, x0, acc[0]);
      if (e + 1 < n) acc[0] = __builtin_fmaf(v.y, x1, acc[0]);
      if (e + 2 < n) acc[0] = __builtin_fmaf(v.z, x2, acc[0]);
      if (e + 3 < n) acc[0] = __builtin_fmaf(v.w, x3, acc[0]);
    };
    if constexpr (STAGE) {
      // two of the lane's quads in flight together (the second clamped into the row)
      for (int q = lane; q < nq; q += 128) {
        const int q2 = min(q + 64, nq - 1);
        const vec4i c = __builtin_nontemporal_load(c4 + q);
        const vec4f v = __builtin_nontemporal_load(v4 + q);
        const vec4i c2 = __builtin_nontemporal_load(c4 + q2);
        const vec4f v2 = __builtin_nontemporal_load(v4 + q2);
        quad(c, v, q);
        if (q + 64 < nq) quad(c2, v2, q + 64);
      }
    } else {
      for (int q = lane; q < nq; q += 64) {
        const vec4i c = __builtin_nontemporal_load(c4 + q);
        const vec4f v = __builtin_nontemporal_load(v4 + q);
        quad(c, v, q);
      }
    }
  } else
  for (int q = lane; q < nq; q += 64) {
    const vec4i c = __builtin_nontemporal_load(c4 + q);
    const vec4f v = __builtin_nontemporal_load(v4 + q);
    const int e = q * 4;
    const vec4f zero = {0.f, 0.f, 0.f, 0.f};
    const vec4f b0 = b_row(c.x);  // e < n for every q < nq
    const vec4f b1 = e + 1 < n ? b_row(c.y) : zero;
    const vec4f b2 = e + 2 < n ? b_row(c.z) : zero;
    const vec4f b3 = e + 3 < n ? b_row(c.w) : zero;
#pragma unroll
    for (int k = 0; k < V; ++k) {
      acc[k] = __builtin_fmaf(v.x, b0[k], acc[k]);
      if (e + 1 < n) acc[k] = __builtin_fmaf(v.y, b1[k], acc[k]);
      if (e + 2 < n) acc[k] = __builtin_fmaf(v.z, b2[k], acc[k]);
      if (e + 3 < n) acc[k] = __builtin_fmaf(v.w, b3[k], acc[k]);
    }
  }
  // the wave's sum into lane 0 (same pairings as a butterfly of offsets 32 .. 1)
#pragma unroll
  for (int k = 0; k < V; ++k) {
    acc[k] += lane_down<32>(acc[k]);
    acc[k] += lane_down<16>(acc[k]);
    acc[k] += lane_down<8>(acc[k]);
    acc[k] += lane_down<4>(acc[k]);
    acc[k] += lane_down<2>(acc[k]);
    acc[k] += lane_down<1>(acc[k]);
  }
  if (lane == 0) {
    float *dst = C + (size_t)row * V;
    // a branch, not a select: C is read only when accumulating (a select
    // made the compiler load C on every launch, +0.3 us at 512^2)
    if (accumulate) {
#pragma unroll
      for (int k = 0; k < V; ++k) dst[k] += acc[k];
    } else {
#pragma unroll
      for (int k = 0; k < V; ++k) dst[k] = acc[k];
    }
  }
}

// The launches row_spmv_kernel takes: km = 1, N = 1, 2 or 4, one wave per row.
inline bool use_row_spmv(const DevView &v, int km, int N, int W) {
  return km == 1 && (N == 1 || N == 2 || N == 4) && W == 1 && v.row_len != nullptr;
}

// ... and with B staged in LDS: B fits 32 KiB, the rows fill at least 256
// workgroups of kRowStagedRows, and every B row serves at least 64 entries.
constexpr int kRowStagedRows = 16;
inline bool row_spmv_staged(const DevView &v, int N) {
  return (long long)v.K * N * (long long)sizeof(float) <= 32768 && v.M >= 256 * kRowStagedRows &&
         v.nslots >= 64ll * v.K;
}

// The buffer-descriptor form of the lanes-over-slots kernel forms a B-row
// offset as __umul24(row, N * 4) + lane bytes: every operand of the 24-bit
// multiply must fit 24 bits (K below 2^24 rows, N * 4 below 2^24 bytes) and
// the offsets the descriptor's 31-bit range (B below 2 GiB).  Other shapes
// take the 64-bit pointer form.
constexpr bool buffer_offsets_fit(long long K, long long N) {
  return K * N * (long long)sizeof(float) < (1ll << 31) && K < (1ll << 24) && N * (long long)sizeof(float) < (1ll << 24);
}
static_assert(buffer_offsets_fit(4096, 128) && buffer_offsets_fit((1 << 24) - 1, 1) &&
                  buffer_offsets_fit(127, (1 << 22) - 1),
              "shapes inside the 24-bit multiply take the buffer path");
static_assert(!buffer_offsets_fit(127, 1 << 22) && !buffer_offsets_fit(1 << 24, 1) &&
                  !buffer_offsets_fit(1 << 15, 1 << 14),
              "row bytes of 2^24, 2^24 rows or 2 GiB of B take the pointer path");

template <int KM, class D>
hipError_t launch_panels(const DevView &v, const float *B, float *C, int N, int accumulate, int W,
                         int pack, hipStream_t stream) {
  if (v.npanels <= 0 || N <= 0) return hipSuccess;
  if (use_row_spmv(v, KM, N, W)) {
    const bool st = row_spmv_staged(v, N);
    const int rows = st ? kRowStagedRows : kRowSpmvRows;
    const size_t lds = st ? (size_t)v.K * N * sizeof(float) : 0;
    const dim3 rgrid((unsigned)((v.M + rows - 1) / rows)), rblock(64u * rows);
#define SC_ROW(RR, VV, SS)                                                                              \
  hipLaunchKernelGGL((row_spmv_kernel<RR, VV, SS>), rgrid, rblock, lds, stream, v.panel_slot,         \
                     v.panel_val, v.row_len, v.cols, v.vals, B, C, v.M, v.K, accumulate)
    if (st) {
      if (N == 4) SC_ROW(kRowStagedRows, 4, true);
      else if (N == 2) SC_ROW(kRowStagedRows, 2, true);
      else SC_ROW(kRowStagedRows, 1, true);
    } else {
      if (N == 4) SC_ROW(kRowSpmvRows, 4, false);
      else if (N == 2) SC_ROW(kRowSpmvRows, 2, false);
      else SC_ROW(kRowSpmvRows, 1, false);
    }
#undef SC_ROW
    return hipGetLastError();
  }
  const TileGeometry tg = tile_geometry(v, N);
  if (tg.use && (tg.nks == 1 || (v.work && v.work_floats >= tg.work_floats && v.tcount &&
                                 v.tcount_n >= tg.counters))) {
    dim3 tgrid((unsigned)(v.tnrb * tg.nks), (unsigned)tg.chunks), tblock(64u * kTilePanels);
#define SC_TILED(VV)                                                                                  \
  hipLaunchKernelGGL((tiled_kernel<KM, VV, D>), tgrid, tblock, tg.lds, stream, v.timg, v.toff, B, C,  \
                     v.work, v.tcount, v.M, v.K, N, v.npanels, v.tnkb, tg.nks, tg.tpu, tg.chunk_dw,   \
                     accumulate)
    if (tg.V == 4) SC_TILED(4);
    else if (tg.V == 2) SC_TILED(2);
    else SC_TILED(1);
#undef SC_TILED
    return hipGetLastError();
  }
  if (pack == 1) {
    const ChunkGeometry cg = chunk_geometry(v, N);
    if (cg.use) {
      hipLaunchKernelGGL((chunk_kernel<KM, 4, D>), dim3(cg.grid), dim3((unsigned)(64 * cg.W)), cg.lds,
                         stream, v.tseg, v.kp_seg, v.kp_slot, v.kp_val, v.tcols, v.tvals, B, C, v.M,
                         v.K, N, v.npanels, v.tppb, cg.ngroups, cg.nchunks, cg.KT, v.tnkb,
                         v.tstage_cols, accumulate);
      return hipGetLastError();
    }
  }
  const Geometry g = geometry(KM, N, W, v.K, v.max_pslots, v.max_pvals, v.a_bytes, v.nslots / v.npanels,
                              v.npanels);
  dim3 grid((unsigned)v.npanels), block((unsigned)(64 * W));
  if (g.wide) {
#define SC_WIDE(VV, ST)                                                                           \
  hipLaunchKernelGGL((wide_kernel<KM, VV, ST, D>), grid, block, g.lds, stream, v.seg,                  \
                     reinterpret_cast<const PanelLaunch *>(v.launch), v.cols, v.vals, B, C, v.M, v.K, N,  \
                     accumulate, pack, g.stage_cols)
    if (g.stage) {
      if (g.V == 4) SC_WIDE(4, true);
      else if (g.V == 2) SC_WIDE(2, true);
      else SC_WIDE(1, true);
    } else {
      if (g.V == 4) SC_WIDE(4, false);
      else if (g.V == 2) SC_WIDE(2, false);
      else SC_WIDE(1, false);
    }
#undef SC_WIDE
    return hipGetLastError();
  }
  if (const size_t glds = gather_lds_f32(N, W, KM, v.max_pslots, v.max_pvals)) {
    const int sv = (v.max_pvals + 3) / 4 * 4;
#define SC_GATHER(VV)                                                                                   \
  hipLaunchKernelGGL((gather_kernel<KM, VV, false, D>), grid, block, glds, stream, v.seg, v.panel_seg,      \
                     v.panel_slot, v.panel_val, v.cols, v.vals, B, C, v.M, accumulate, pack, sv)
    if (N == 4) SC_GATHER(4);
    else if (N == 2) SC_GATHER(2);
    else SC_GATHER(1);
#undef SC_GATHER
    return hipGetLastError();
  }
  const dim3 ngrid((unsigned)v.npanels, (unsigned)g.ny);
#define SC_NARROW(VV, ST, AA)                                                                          \
  hipLaunchKernelGGL((panel_kernel<KM, VV, ST, D, AA>), ngrid, block, g.lds, stream, v.seg,                \
                     reinterpret_cast<const PanelLaunch *>(v.launch), v.cols, v.vals, B, C, v.M, v.K, N, g.L,  \
                     accumulate, pack, g.stage_cols)
  if (buffer_offsets_fit(v.K, N)) {
    if (g.stage) {
      if (g.V == 4) SC_NARROW(4, true, SegArgsBuf);
      else if (g.V == 2) SC_NARROW(2, true, SegArgsBuf);
      else SC_NARROW(1, true, SegArgsBuf);
    } else {
      if (g.V == 4) SC_NARROW(4, false, SegArgsBuf);
      else if (g.V == 2) SC_NARROW(2, false, SegArgsBuf);
      else SC_NARROW(1, false, SegArgsBuf);
    }
  } else {
    if (g.stage) {
      if (g.V == 4) SC_NARROW(4, true, SegArgs);
      else if (g.V == 2) SC_NARROW(2, true, SegArgs);
      else SC_NARROW(1, true, SegArgs);
    } else {
      if (g.V == 4) SC_NARROW(4, false, SegArgs);
      else if (g.V == 2) SC_NARROW(2, false, SegArgs);
      else SC_NARROW(1, false, SegArgs);
    }
  }
#undef SC_NARROW
  return hipGetLastError();
}

// binary16 values, B and C (N = 1, 2 or 4): the small-N gather kernel with
// fp32 accumulation.  The counterpart of the reference's fp16 small-B bodies
// (PatternWith{pop}NNZByRowPanelFullHALF), which accumulate in binary16.
template <int KM, class D>
hipError_t launch_panels_f16(const DevView &v, const void *B, void *C, int N, int accumulate, int W,
                             int pack, hipStream_t stream) {
  if (!v.vals16 || !(N == 1 || N == 2 || N == 4)) return hipErrorInvalidValue;
  if (v.npanels <= 0) return hipSuccess;
  const size_t glds = gather_lds(N, W, KM, v.max_pslots, v.max_pvals);
  if (!glds) return hipErrorInvalidValue;
  const int sv = (v.max_pvals + 3) / 4 * 4;
  dim3 grid((unsigned)v.npanels), block((unsigned)(64 * W));
#define SC_GATHER16(VV)                                                                                 \
  hipLaunchKernelGGL((gather_kernel<KM, VV, true, D>), grid, block, glds, stream, v.seg, v.panel_seg,       \
                     v.panel_slot, v.panel_val, v.cols, v.vals16, B, C, v.M, accumulate, pack, sv)
  if (N == 4) SC_GATHER16(4);
  else if (N == 2) SC_GATHER16(2);
  else SC_GATHER16(1);
#undef SC_GATHER16
  return hipGetLastError();
}

}  // namespace sc
