// sc_band.hpp -- the band kernel: kernel_m 4 plans at N a multiple of 64,
// with B staged in LDS once per (band of panels, K range) and every slot on
// the matrix cores.
//
// Why.  The panel kernels gather one B row per slot from L2 (a 512-byte row
// at N = 128); on a 4096 x 4096 matrix at 10 % density that is 415 MB per
// launch through the L2 -> L1 path, which runs at about 19 TB/s on MI355X.
// A band of 64 panels touches almost every column of a K range, so staging
// the range's B rows in LDS once per band replaces the per-slot L2 gathers
// with LDS reads, and the L2 -> CU traffic falls to the B ranges (one copy
// per band), the stream, and the split-K partial sums.
//
// Work decomposition.  A unit (workgroup of 16 waves) owns one band, one N
// chunk of 64 columns and one K range of up to 512 B rows.  It stages
// B[range rows, chunk] (256 bytes a row, then one row of zeros for padding
// slots) in LDS by LDS DMA, waits once, and then its waves run on their own:
// no barrier couples them.  The plan assigns the band's panels to the 16
// waves per K range, balancing their items (longest first onto the least
// loaded wave); a wave runs its panels one after another, accumulating each
// in registers, and hands it over when its items end.  The unit count is
// bands x K ranges x N chunks; consecutive units take consecutive K ranges,
// so with 8 K ranges every XCD holds one range of B and the two chunks of a
// (band, range) share the stream in one L2.
//
// Items on the matrix cores.  A panel's slots in the range, in column order,
// come four to an item, whatever their patterns (rows a pattern lacks carry
// value 0), and every item runs on v_mfma_f32_4x4x1f32: 16 blocks of a 4-row
// by 4-column outer product; block b = 4s + c takes slot s and columns
// 16c + 4j + q (j the block's column, q = 0..3 over four instructions).
// Lane 16s + 4c + j reads 16 bytes at column 16c + 4j of slot s's staged B
// row (one LDS read feeds the four instructions).  A wave's items, all its
// panels one after another, come in blocks of 16 items (four groups of
// four), 320 dwords each:
//   * 256 values: lane l loads the 16 bytes at 4l, whose dword G is
//     value (item 4G + t, slot s, row i) for l = 16s + 4t + i; item 4G + t's
//     instructions take their A operand from dword G with cbsz 2 / abid t
//     (each group of four blocks reads block 4s + t's lanes), so no lane
//     holds a copy;
//   * 64 B-row byte offsets into the stage, (item x, slot s) at 16s + x:
//     lane l loads dword l, and item x's offset reaches the whole row of 16
//     lanes by a DPP row broadcast (row_newbcast x).
// Four blocks are in registers at a time: three load while one runs.
// The four slot positions' sums are added once per panel with the gfx950
// lane swaps (a reduce-scatter: lane 16s + x ends with row s).
//
// Numerics.  Rows a slot's pattern lacks are multiplied by 0 here, as the
// format's own padding slots are in the reference's kernels: with finite B
// the sums equal the pattern bodies' to rounding, while an Inf or NaN in a B
// row can reach a row of C that has no entry in that column (0 * Inf = NaN).
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
constexpr int kBandBlockDw = 320;             // dwords of a block of 16 items (4 groups)
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
//   A panel's last group is padded with items of value 0 on the zero row, the
//   last block with such groups; a panel with no slot in the range has one
//   such group, and a wave without panels one block of them.
struct BandView {
  const int *img;   // wave records
  const int *woff;  // first dword of record (band * nks + ks) * 16 + w, + end
  int nbands;
  int nks;          // K ranges
  int KR;           // B rows per K range (a multiple of 4; the zero row follows)
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

__host__ __device__ inline size_t band_lds_bytes(int KR) { return (size_t)(KR + 1) * kBandRowBytes; }

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

// Swap halves between two registers: x's lanes 32..63 with y's lanes 0..31
// (v_permlane32_swap_b32), and x's rows 1 and 3 with y's rows 0 and 2
// (v_permlane16_swap_b32).  Inline asm for the reason given at lane_down;
// the s_nop covers the VALU-write hazard.
__device__ __forceinline__ void swap_halves32(float &x, float &y) {
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(x), "+v"(y));
}
__device__ __forceinline__ void swap_rows16(float &x, float &y) {
  asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(x), "+v"(y));
}

// Item T of a group: its B rows (offset o, broadcast from lane 16s + T of
// every row), then the four instructions.
template <int T>
__device__ __forceinline__ vec4f band_read(const lds_char *tile, int o) {
  const int off = __builtin_amdgcn_update_dpp(0, o, 0x150 + T, 0xf, 0xf, false);
  return *(const lds_float4 *)(tile + off);
}

template <int T>
__device__ __forceinline__ void band_mfma(vec4f_t (&D)[4], float a, const vec4f &x) {
  D[0] = __builtin_amdgcn_mfma_f32_4x4x1f32(a, x.x, D[0], 2, T, 0);
  D[1] = __builtin_amdgcn_mfma_f32_4x4x1f32(a, x.y, D[1], 2, T, 0);
  D[2] = __builtin_amdgcn_mfma_f32_4x4x1f32(a, x.z, D[2], 2, T, 0);
  D[3] = __builtin_amdgcn_mfma_f32_4x4x1f32(a, x.w, D[3], 2, T, 0);
}

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

  // the zero row (row KR): padding slots read it
  if (threadIdx.x < kBandCols / 4) ((lds_float4 *)(lds + KR * kBandRowBytes))[threadIdx.x] = vec4f{0.f, 0.f, 0.f, 0.f};
  // B[k0 .. k0 + rows, n0 .. n0 + 64) into LDS by LDS DMA: one wave
  // instruction moves four B rows (lane l: row l / 16 of the four, 16 bytes
  // of column group l % 16), wave w the groups w, w + 16, ...; rows past the
  // range re-read its last row into rows below KR (never referenced)
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
  const int ngroups = rec[1];
  const int *ptab = rec + kBandRecHeader;
  const int *blk = ptab + ((2 * npan + 3) & ~3);
  const int nblk = rec[2];
  int pidv = 0, ngv = 0;
  if (lane < npan) {
    pidv = ptab[2 * lane];
    ngv = ptab[2 * lane + 1];
  }
  const vec4f *bval = reinterpret_cast<const vec4f *>(blk) + lane;
  const int *boff = blk + 256 + lane;
  // blocks b .. b + 3 in registers (the stream comes from HBM: three blocks
  // of lead time cover its latency under load).  Every record holds at least
  // one block, so the four loads are issued on every path (past the end they
  // re-read the last block), and the barrier waits for the DMA and the panel
  // table only: the blocks keep arriving while the first groups run.
  vec4f V[kBandBlocksInFlight];
  int O[kBandBlocksInFlight];
#pragma unroll
  for (int i = 0; i < kBandBlocksInFlight; ++i) {
    const int nb = min(i, nblk - 1);
    V[i] = __builtin_nontemporal_load(bval + (size_t)nb * (kBandBlockDw / 4));
    O[i] = __builtin_nontemporal_load(boff + (size_t)nb * kBandBlockDw);
  }
  // vmcnt(8): everything but the eight block loads (the DMA, the panel
  // table); expcnt and lgkmcnt at their maximum (no wait; the barrier below
  // waits for the LDS writes of the zero row)
  static_assert(kBandBlocksInFlight * 2 == 8, "the wait below counts eight block loads");
  __builtin_amdgcn_s_waitcnt(0x0F78);
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the zero row is written
  // a bare barrier: __syncthreads() would also wait for the block loads
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");

  // this lane's 16 bytes (columns 16c + 4j .. + 3) of a staged row; the
  // offsets in the stream add to it
  const lds_char *tile = lds + 16 * (lane & 15);
  vec4f_t D[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) D[q] = vec4f_t{0.f, 0.f, 0.f, 0.f};
  // the wave's finished panel tiles (panel k in T[k]), stored after the loop:
  // a store pending beside the block loads would make every wait for a block
  // a wait for everything
  vec4f T[kBandWavePanels];
#pragma unroll
  for (int k = 0; k < kBandWavePanels; ++k) T[k] = vec4f{0.f, 0.f, 0.f, 0.f};

  // Panel p's tile is done: its four slot positions' sums (rows 0, 1 to
  // lanes 0..31 and 2, 3 to lanes 32..63, then row 2 (s / 2) to the even
  // rows of 16 lanes and 2 (s / 2) + 1 to the odd ones: lane 16s + x ends
  // with row s) into T[p]
  int p = 0;
  auto flush = [&]() __attribute__((always_inline)) {
    vec4f r;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      float x0 = D[q][0], x2 = D[q][2], x1 = D[q][1], x3 = D[q][3];
      swap_halves32(x0, x2);
      swap_halves32(x1, x3);
      float a = x0 + x2, b = x1 + x3;
      swap_rows16(a, b);
      r[q] = a + b;
      D[q] = vec4f_t{0.f, 0.f, 0.f, 0.f};
    }
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
  // group G of a block (values dword G, offsets of items 4G .. 4G + 3)
  auto group = [&](auto GC, const vec4f &V, int O) __attribute__((always_inline)) {
    constexpr int G = decltype(GC)::value;
    if (p >= npan) return;  // past the last panel: padding groups
    const float v = V[G];
    const vec4f x0 = band_read<4 * G + 0>(tile, O);
    const vec4f x1 = band_read<4 * G + 1>(tile, O);
    const vec4f x2 = band_read<4 * G + 2>(tile, O);
    const vec4f x3 = band_read<4 * G + 3>(tile, O);
    __builtin_amdgcn_sched_barrier(0);  // the four reads in flight together
    band_mfma<0>(D, v, x0);
    band_mfma<1>(D, v, x1);
    band_mfma<2>(D, v, x2);
    band_mfma<3>(D, v, x3);
    if (--left == 0) {
      flush();
      next_panel();
    }
  };
  auto run_block = [&](const vec4f &V, int O) __attribute__((always_inline)) {
    group(std::integral_constant<int, 0>{}, V, O);
    group(std::integral_constant<int, 1>{}, V, O);
    group(std::integral_constant<int, 2>{}, V, O);
    group(std::integral_constant<int, 3>{}, V, O);
  };
  // The next loads are issued on every path (past the end they re-read the
  // last block), so that every wait for a block counts the same loads after
  // it; a load issued on one path only makes the compiler wait for
  // everything.  Blocks past the last one run no group (p == npan).
  for (int b = 0; b < nblk; b += kBandBlocksInFlight) {
#pragma unroll
    for (int i = 0; i < kBandBlocksInFlight; ++i) {
      run_block(V[i], O[i]);
      const int nb = min(b + i + kBandBlocksInFlight, nblk - 1);
      V[i] = __builtin_nontemporal_load(bval + (size_t)nb * (kBandBlockDw / 4));
      O[i] = __builtin_nontemporal_load(boff + (size_t)nb * kBandBlockDw);
    }
  }

  // the tiles to C (one K range) or as this range's partials to the
  // workspace (written through, sc1); lane 16s + x holds row s, columns
  // n0 + 4x .. + 3 of its panel
  const int my_row = lane >> 4;
  const int my_col = n0 + 4 * (lane & 15);
  const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(work, (short)0, (int)0x7fffffff, kBufferWord3);
#pragma unroll
  for (int k = 0; k < kBandWavePanels; ++k) {
    if (k >= npan) break;
    const int pid = __builtin_amdgcn_readlane(pidv, k);
    vec4f r = T[k];
    if (nks == 1) {
      const int row = 4 * pid + my_row;
      if (row < M) {
        vec4f *dst = reinterpret_cast<vec4f *>(C + (size_t)row * N + my_col);
        if (accumulate) r += *dst;
        *dst = r;
      }
    } else {
      // 16 bytes a lane, so the wave writes whole 128-byte lines
      const unsigned off = (unsigned)((((size_t)ks * npanels + pid) * nch + chunk) * (4 * kBandCols) * sizeof(float)) +
                           16u * (unsigned)lane;
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(vec4i, r), wr, off, 0, kCachePolicySc1);
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
      const int row = 4 * q + my_row;
      if (row < M) {
        vec4f *dst = reinterpret_cast<vec4f *>(C + (size_t)row * N + my_col);
        if (accumulate) sum += *dst;
        *dst = sum;
      }
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
