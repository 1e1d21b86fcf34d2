// sc_band.hpp -- the band kernel: kernel_m 4 plans at N a multiple of 64,
// with B staged in LDS once per (band of panels, K range) and every stored
// entry on the matrix cores.
//
// Why.  The panel kernels gather one B row per slot from L2 (a 512-byte row
// at N = 128); on a 4096 x 4096 matrix at 10 % density that is 415 MB per
// launch through the L2 -> L1 path, which serves such rows at 30 to 33 TB/s
// on MI355X (measured) and the panel kernel drives at about 25 TB/s.
// A band of 64 panels touches almost every column of a K range, so staging
// the range's B rows in LDS once per band replaces the per-slot L2 gathers
// with LDS reads, and the L2 -> CU traffic falls to the B ranges (one copy
// per band), the stream, and the split-K partial sums.
//
// Work decomposition.  A unit (workgroup of 16 waves) owns one band, one N
// chunk of 64 columns and one K range of up to 512 B rows.  It stages
// B[range rows, chunk] (256 bytes a row) in LDS by LDS DMA, waits once, and
// then its waves run on their own: no barrier couples them.  The plan
// assigns the band's panels to the 16 waves per K range, balancing their
// items (longest first onto the least loaded wave); a wave runs its panels
// one after another, accumulating each in registers, and keeps the finished
// tiles in registers until its last panel.  The unit count is bands x K
// ranges x N chunks; consecutive units take consecutive K ranges, so with 8
// K ranges every XCD holds one range of B and the two chunks of a (band,
// range) share the stream in one L2.
//
// Items on the matrix cores.  An item is a window of four consecutive
// columns of A (four consecutive B rows, aligned to 4 in the range) inside
// one panel: its 16 values, row i and column t at A(i, t), 0 where no entry
// is stored.  It runs as four v_mfma_f32_4x4x1f32, instruction t taking
// window column t: all 16 blocks take its four row values (cbsz 4, abid the
// lane block holding them) and block b columns 4b .. 4b + 3 of B row
// (window + t), so lane l reads the one float at column l of each of the
// four rows (ds_read_b32 at offsets 0, 256, 512, 768 from one address), and
// instruction t accumulates into the 4 x 64 tile D[t]: lane l holds rows
// 0..3 of column l.  The four tiles are added in the lane when the panel
// ends; there is no cross-lane reduction.  A wave's items,
// all its panels one after another, come in blocks of 16 items (four groups
// of four), 272 dwords each:
//   * 256 values: lane l loads the 16 bytes at 4l, whose dword G is
//     A(i, t) of item 4G + u for l = 16u + 4t + i;
//   * 16 window byte offsets into the stage (item x at x), which lane
//     16r + x loads, and item x's reaches the whole row of 16 lanes by a DPP
//     row broadcast (row_newbcast x) fused with the add of the lane's column.
// That one add is the only vector ALU work of an item: on gfx950 each VALU
// instruction among 4x4x1 MFMAs costs about 1.5 MFMA issue slots (measured),
// so the loop keeps them to one per four MFMAs.  Four blocks are in
// registers at a time: three load while one runs.
//
// Numerics.  A window's zero values multiply B rows the panel's row does not
// use, as the format's own padding slots do in the reference's kernels: with
// finite B the sums equal the pattern bodies' to rounding, while an Inf or
// NaN in a B row can reach a row of C that has no entry in that column
// (0 * Inf = NaN).
//
// Split K.  With more than one K range, a wave writes each panel's partial
// tile (4 rows x 64 columns) to the workspace with write-through stores and,
// after all its panels, bumps each panel's (panel, chunk) counter; the wave
// that arrives last for a panel adds the nks partials in K-range order (so
// the result does not depend on arrival order), writes C and resets the
// counter.  Launches that share a workspace must be stream ordered.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "sc_kernels.hpp"

namespace sc {

constexpr int kBandWaves = 16;                // waves per unit
constexpr int kBandCols = 64;                 // columns of B and C per N chunk
constexpr int kBandRowBytes = 4 * kBandCols;  // bytes of one staged B row
constexpr int kBandMaxRange = 512;            // most B rows of one K range
constexpr int kBandMaxRanges = 16;            // most K ranges (K up to 8192)
constexpr int kBandBlockDw = 272;             // dwords of a block of 16 items (4 groups)
constexpr int kBandRecHeader = 4;             // dwords of a wave record's header
constexpr int kBandWavePanels = 8;            // most panels of one wave per K range
constexpr int kBandBlocksInFlight = 4;        // stream blocks a wave holds in registers
constexpr int kBandMaxChunks = 4;             // the plan's workspace covers N <= 256
constexpr size_t kBandLdsBytes = 160 * 1024;
// units per (band, K range) pair the plan aims for at N = 128 (two chunks):
// one unit per CU
constexpr int kBandTargetPairs = 128;

// Wave record (dwords), one per (band, K range, wave), stored in that order
// and 16-byte aligned:
//   [0] panels of this wave (np), [1] groups of all of them, [2] blocks
//   (at least one), [3] 0;
//   then np (panel, groups) pairs, padded to a multiple of 4 dwords;
//   then the blocks (layout above), the panels' groups one after another.
//   A panel's last group is padded with items of value 0 on window 0, the
//   last block with such groups; a panel with no entry in the range has one
//   such group, and a wave without panels one block of them.
struct BandView {
  const int *img;   // wave records
  const int *woff;  // first dword of record (band * nks + ks) * 16 + w, + end
  int nbands;
  int nks;          // K ranges
  int KR;           // B rows per K range (a multiple of 4)
  int npanels;
};

// Launch shape of the band kernel for N columns.
struct BandGeometry {
  bool use = false;
  int nch = 0;  // N chunks of 64 columns
  unsigned grid = 0;
  size_t lds = 0;
  size_t work_floats = 0;  // partial sums needed (nks > 1)
  int counters = 0;        // arrival counters needed (nks > 1)
};

__host__ __device__ inline size_t band_lds_bytes(int KR) { return (size_t)KR * kBandRowBytes; }

// Partial tile (4 x 64 floats) of (K range k, panel q, chunk c).
__host__ __device__ inline size_t band_partial_floats(int nks, int npanels, int nch) {
  return nks > 1 ? (size_t)nks * npanels * nch * 4 * kBandCols : 0;
}

// work_cap / counter_cap: the workspace the launch will pass.
inline BandGeometry band_geometry(const BandView &b, int N, size_t work_cap, size_t counter_cap) {
  BandGeometry g;
  if (!b.img || N <= 0 || N % kBandCols != 0 || b.nbands <= 0 || b.nks <= 0) return g;
  g.nch = N / kBandCols;
  g.lds = band_lds_bytes(b.KR);
  if (g.lds > kBandLdsBytes) return g;
  g.work_floats = band_partial_floats(b.nks, b.npanels, g.nch);
  g.counters = b.nks > 1 ? b.npanels * g.nch : 0;
  // byte offsets into the workspace are 32-bit
  if (g.work_floats > work_cap || (size_t)g.counters > counter_cap || g.work_floats * 4 > 0x7fffffffu) return g;
  const long long grid = (long long)b.nbands * b.nks * g.nch;
  if (grid <= 0 || grid > 0x7fffffffLL) return g;
  g.grid = (unsigned)grid;
  g.use = true;
  return g;
}

typedef float vec4f_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) char lds_char;

// The four B values of one item for this lane: column `lane` of the
// window's rows (window offset W broadcast from lane 16r + X of every row,
// plus the lane's column bytes `lc`).
struct BandRows {
  float x[4];
};

template <int X>
__device__ __forceinline__ BandRows band_read(const lds_char *lds, int W, int lc) {
  const int a = __builtin_amdgcn_update_dpp(0, W, 0x150 + X, 0xf, 0xf, false) + lc;
  const lds_char *p = lds + a;
  BandRows r;
  r.x[0] = *(const lds_float *)(p);
  r.x[1] = *(const lds_float *)(p + kBandRowBytes);
  r.x[2] = *(const lds_float *)(p + 2 * kBandRowBytes);
  r.x[3] = *(const lds_float *)(p + 3 * kBandRowBytes);
  return r;
}

// Item 4G + U: its four instructions; window column t's row values sit in
// lane block 4U + t of values dword G.
// Window column t accumulates into D[t], so consecutive instructions do not
// wait on each other's results; the four are added when the panel ends.
template <int U>
__device__ __forceinline__ void band_mfma(vec4f_t (&D)[4], float a, const BandRows &r) {
  D[0] = __builtin_amdgcn_mfma_f32_4x4x1f32(a, r.x[0], D[0], 4, 4 * U + 0, 0);
  D[1] = __builtin_amdgcn_mfma_f32_4x4x1f32(a, r.x[1], D[1], 4, 4 * U + 1, 0);
  D[2] = __builtin_amdgcn_mfma_f32_4x4x1f32(a, r.x[2], D[2], 4, 4 * U + 2, 0);
  D[3] = __builtin_amdgcn_mfma_f32_4x4x1f32(a, r.x[3], D[3], 4, 4 * U + 3, 0);
}

// The B values of one group's four items.
struct BandGroupRows {
  BandRows it[4];
};

// The band kernel (kernel_m 4).  blockDim.x = 64 * kBandWaves.  Unit u of
// the grid: ks = u % nks, chunk = (u / nks) % nch, band = u / (nks * nch).
__global__ void __launch_bounds__(64 * kBandWaves)
    band_kernel(const int *__restrict__ img, const int *__restrict__ woff, const float *__restrict__ B,
                float *__restrict__ C, float *__restrict__ work, unsigned *__restrict__ counters, int M, int K,
                int N, int npanels, int nks, int KR, int nch, int accumulate) {
  extern __shared__ float4 smem4[];
  const int u = blockIdx.x;
  const int ks = u % nks;
  const int chunk = (u / nks) % nch;
  const int band = u / (nks * nch);
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int n0 = chunk * kBandCols;
  const int k0 = ks * KR;
  const int rows = min(KR, K - k0);
  lds_char *lds = (lds_char *)smem4;

  // B[k0 .. k0 + rows, n0 .. n0 + 64) into LDS by LDS DMA: one wave
  // instruction moves four B rows (lane l: row l / 16 of the four, 16 bytes
  // of column group l % 16), wave w the groups w, w + 16, ...; rows past the
  // range re-read its last row into rows below KR (read by windows that
  // reach past the range, whose values there are 0)
  {
    const int groups = (rows + 3) >> 2;
    const float *src = B + n0 + (lane & 15) * 4;
    for (int i = w; i < groups; i += kBandWaves) {
      const int r = min(4 * i + (lane >> 4), rows - 1);
      __builtin_amdgcn_global_load_lds(src + (size_t)(k0 + r) * N,
                                       (__attribute__((address_space(3))) void *)(lds + i * 4 * kBandRowBytes), 16,
                                       0, 0);
    }
  }

  // this wave's record; its panel table in lanes (lane k: panel k's id and
  // groups), read back with readlane, so the loop below holds no memory
  // access but the stream's block loads
  const int *rec = img + woff[(band * nks + ks) * kBandWaves + w];
  const int npan = rec[0];
  const int *ptab = rec + kBandRecHeader;
  const int *blk = ptab + ((2 * npan + 3) & ~3);
  const int nblk = rec[2];
  int pidv = 0, ngv = 0;
  if (lane < npan) {
    pidv = ptab[2 * lane];
    ngv = ptab[2 * lane + 1];
  }
  // the blocks through a buffer descriptor: the block's byte offset is a
  // scalar, the lane's part a constant, so a block load costs no vector
  // address arithmetic (non-temporal: the stream is read once)
  const __amdgpu_buffer_rsrc_t brs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<int *>(blk), (short)0, (int)0x7fffffff, kBufferWord3);
  const unsigned vofs = 16u * (unsigned)lane;
  const unsigned wofs = 4u * (256u + (unsigned)(lane & 15));
  auto load_block = [&](int nb, vec4f &Vv, int &Wv) __attribute__((always_inline)) {
    const unsigned so = (unsigned)__builtin_amdgcn_readfirstlane(nb * kBandBlockDw * 4);
    Vv = __builtin_bit_cast(vec4f, __builtin_amdgcn_raw_buffer_load_b128(brs, vofs, so, kCachePolicyNt));
    Wv = (int)__builtin_amdgcn_raw_buffer_load_b32(brs, wofs, so, kCachePolicyNt);
  };
  // blocks b .. b + 3 in registers (the stream comes from HBM: three blocks
  // of lead time cover its latency under load).  Every record holds at least
  // one block, so the four loads are issued on every path (past the end they
  // re-read the last block), and the barrier waits for the DMA and the panel
  // table only: the blocks keep arriving while the first groups run.
  vec4f V[kBandBlocksInFlight];
  int W[kBandBlocksInFlight];
#pragma unroll
  for (int i = 0; i < kBandBlocksInFlight; ++i) {
    const int nb = min(i, nblk - 1);
    load_block(nb, V[i], W[i]);
  }
  // vmcnt(8): everything but the eight block loads (the DMA, the panel
  // table); expcnt and lgkmcnt at their maximum (no wait)
  static_assert(kBandBlocksInFlight * 2 == 8, "the wait below counts eight block loads");
  __builtin_amdgcn_s_waitcnt(0x0F78);
  // a bare barrier: __syncthreads() would also wait for the block loads
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");

  // this lane's column of a staged row; the windows' offsets add to it
  const int lc = 4 * lane;
  vec4f_t D[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) D[t] = vec4f_t{0.f, 0.f, 0.f, 0.f};
  // the wave's finished panel tiles (panel k in T[k]), stored after the loop:
  // a store pending beside the block loads would make every wait for a block
  // a wait for everything
  vec4f T[kBandWavePanels];
#pragma unroll
  for (int k = 0; k < kBandWavePanels; ++k) T[k] = vec4f{0.f, 0.f, 0.f, 0.f};

  // Panel p's tile is done: lane l holds rows 0..3 of its column l.
  int p = 0;
  auto flush = [&]() __attribute__((always_inline)) {
    const vec4f_t d = (D[0] + D[1]) + (D[2] + D[3]);
    const vec4f r = vec4f{d[0], d[1], d[2], d[3]};
#pragma unroll
    for (int t = 0; t < 4; ++t) D[t] = vec4f_t{0.f, 0.f, 0.f, 0.f};
    switch (p) {
#define SC_BAND_KEEP(k) \
  case k:               \
    T[k] = r;           \
    break;
      SC_BAND_KEEP(0) SC_BAND_KEEP(1) SC_BAND_KEEP(2) SC_BAND_KEEP(3)
      SC_BAND_KEEP(4) SC_BAND_KEEP(5) SC_BAND_KEEP(6) SC_BAND_KEEP(7)
#undef SC_BAND_KEEP
      default:
        break;
    }
  };
  static_assert(kBandWavePanels == 8, "flush keeps eight tiles");
  // the current panel and the groups it has left (every panel has at least
  // one group in every range: the plan gives an empty one a group of zeros)
  int left = npan > 0 ? __builtin_amdgcn_readfirstlane(ngv) : 0;
  auto next_panel = [&]() __attribute__((always_inline)) {
    ++p;
    if (p < npan) left = __builtin_amdgcn_readlane(ngv, p);
  };
  // Group G of a block: the B values of its items 4G .. 4G + 3 (windows in
  // W), then their instructions (values dword G of V).  The reads of the
  // next group are issued before a group's instructions, so a wave always
  // has B values in flight while its instructions issue.
  auto reads = [&](auto GC, int Wb) __attribute__((always_inline)) {
    constexpr int G = decltype(GC)::value;
    BandGroupRows x;
    x.it[0] = band_read<4 * G + 0>(lds, Wb, lc);
    x.it[1] = band_read<4 * G + 1>(lds, Wb, lc);
    x.it[2] = band_read<4 * G + 2>(lds, Wb, lc);
    x.it[3] = band_read<4 * G + 3>(lds, Wb, lc);
    return x;
  };
  auto compute = [&](auto GC, const vec4f &V, const BandGroupRows &x) __attribute__((always_inline)) {
    constexpr int G = decltype(GC)::value;
    if (p >= npan) return;  // past the last panel: padding groups
    const float a = V[G];
    band_mfma<0>(D, a, x.it[0]);
    band_mfma<1>(D, a, x.it[1]);
    band_mfma<2>(D, a, x.it[2]);
    band_mfma<3>(D, a, x.it[3]);
    if (--left == 0) {
      flush();
      next_panel();
    }
  };
  using G0 = std::integral_constant<int, 0>;
  using G1 = std::integral_constant<int, 1>;
  using G2 = std::integral_constant<int, 2>;
  using G3 = std::integral_constant<int, 3>;
  // The next loads are issued on every path (past the end they re-read the
  // last block), so that every wait for a block counts the same loads after
  // it; a load issued on one path only makes the compiler wait for
  // everything.  Blocks past the last one run no group (p == npan).
  BandGroupRows x = reads(G0{}, W[0]);
  for (int b = 0; b < nblk; b += kBandBlocksInFlight) {
#pragma unroll
    for (int i = 0; i < kBandBlocksInFlight; ++i) {
      BandGroupRows y = reads(G1{}, W[i]);
      __builtin_amdgcn_sched_barrier(0);
      compute(G0{}, V[i], x);
      x = reads(G2{}, W[i]);
      __builtin_amdgcn_sched_barrier(0);
      compute(G1{}, V[i], y);
      y = reads(G3{}, W[i]);
      __builtin_amdgcn_sched_barrier(0);
      compute(G2{}, V[i], x);
      // the next block's first group (block b + 4 when i = 3: refilled at i = 0)
      x = reads(G0{}, W[(i + 1) % kBandBlocksInFlight]);
      __builtin_amdgcn_sched_barrier(0);
      compute(G3{}, V[i], y);
      const int nb = min(b + i + kBandBlocksInFlight, nblk - 1);
      load_block(nb, V[i], W[i]);
    }
  }

  // the tiles to C (one K range) or as this range's partials to the
  // workspace (written through, sc1, 16 bytes a lane: whole 128-byte lines);
  // lane l holds rows 0..3 of column n0 + l of its panel
  const int my_col = n0 + lane;
  const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(work, (short)0, (int)0x7fffffff, kBufferWord3);
  auto to_c = [&](int pid, vec4f r) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = 4 * pid + i;
      if (row < M) {
        float *dst = C + (size_t)row * N + my_col;
        *dst = accumulate ? *dst + r[i] : r[i];
      }
    }
  };
#pragma unroll
  for (int k = 0; k < kBandWavePanels; ++k) {
    if (k >= npan) break;
    const int pid = __builtin_amdgcn_readlane(pidv, k);
    if (nks == 1) {
      to_c(pid, T[k]);
    } else {
      const unsigned off = (unsigned)((((size_t)ks * npanels + pid) * nch + chunk) * (4 * kBandCols) * sizeof(float)) +
                           16u * (unsigned)lane;
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(vec4i, T[k]), wr, off, 0, kCachePolicySc1);
    }
  }
  if (nks == 1) return;

  // split-K hand-over: once this wave's partial stores have completed, one
  // counter bump per panel (lane k: the wave's panel k); the last of the nks
  // arrivals adds the partials in K-range order
  __builtin_amdgcn_s_waitcnt(0);
  const size_t kstride = (size_t)npanels * nch * (4 * kBandCols) * sizeof(float);
  {
    const int pid = pidv;
    bool last = false;
    if (lane < npan) {
      const unsigned old =
          __hip_atomic_fetch_add(counters + (size_t)pid * nch + chunk, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      last = old == (unsigned)(nks - 1);
    }
    uint64_t mask = __ballot(last);
    while (mask) {
      const int i = __builtin_ctzll(mask);
      mask &= mask - 1;
      const int q = __builtin_amdgcn_readlane(pid, i);
      const unsigned off = (unsigned)(((size_t)q * nch + chunk) * (4 * kBandCols) * sizeof(float) + 16 * lane);
      vec4f sum = vec4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll 8
      for (int k = 0; k < nks; ++k) {
        // sc1: read the partial where it was written through, not a stale
        // copy in this XCD's L2
        sum += __builtin_bit_cast(vec4f, __builtin_amdgcn_raw_buffer_load_b128(wr, off, (unsigned)(k * kstride),
                                                                               kCachePolicySc1));
      }
      to_c(q, sum);
      if (lane == 0)
        __hip_atomic_store(counters + (size_t)q * nch + chunk, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

inline hipError_t launch_band(const BandView &b, const BandGeometry &g, const float *B, float *C, float *work,
                              unsigned *counters, int M, int K, int N, int accumulate, hipStream_t stream) {
  if (!g.use) return hipErrorInvalidValue;
  if (g.grid == 0) return hipSuccess;
  hipLaunchKernelGGL(band_kernel, dim3(g.grid), dim3(64 * kBandWaves), g.lds, stream, b.img, b.woff, B, C, work,
                     counters, M, K, N, b.npanels, b.nks, b.KR, g.nch, accumulate);
  return hipGetLastError();
}

}  // namespace sc
