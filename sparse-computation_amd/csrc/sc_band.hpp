// sc_band.hpp -- the band kernel: km = 4 plans at N a multiple of 64, with
// B staged in LDS once per band of 32 panels (128 rows) and K tile.
//
// Why.  The panel kernels gather one B row per slot from L2 (a 512-byte row
// at N = 128); on a 4096 x 4096 matrix at 10 % density that is 415 MB per
// launch through the L2 -> L1 path, which runs at about 19 TB/s on MI355X.
// A band of 32 panels touches almost every column of a K tile, so staging the
// tile's B rows in LDS once per band replaces the per-slot L2 gathers with
// LDS reads, and the L2 -> CU traffic falls to the B tiles (one copy per
// band), the stream, and the split-K partial sums.
//
// Work decomposition.  A unit (workgroup of 16 waves) owns one band, one N
// chunk of 64 columns and one range of K tiles (split K, so that the grid
// covers the 256 CUs).  Per tile it stages B[tile rows, chunk] (256 bytes a
// row, one extra row of zeros for padding) and each wave its own part of the
// tile's stream (the wave image) in LDS, double-buffered for B, while the
// waves compute the previous tile.  Wave w owns panels 2w and 2w + 1 of the
// band.  A panel's slots in a tile come as two kinds of items:
//   * dense items: four slots of the all-ones pattern (the 4 x 4 blocks of a
//     km = 4 format), run on the matrix cores: v_mfma_f32_4x4x1f32 with 16
//     blocks covers one slot's four rows times the chunk's 64 columns, lane l
//     holding column l and register i row i of the panel;
//   * single items: four (row, column, value) entries of one panel row, the
//     slots of every other pattern split into their rows (a pop-2 slot gives
//     two entries), run on the VALU with 16 lanes of 4 columns per entry.
// Items are padded to four slots with value 0 on the zero row.
//
// Split K.  With more than one K range per (band, chunk), every unit writes
// its partial tile to the workspace (write-through stores) and bumps the
// (band, chunk) counter; the unit that arrives last adds the partials in
// K-range order (so the result does not depend on arrival order), writes C
// and resets the counter.  Launches that share a workspace must be stream
// ordered.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "sc_kernels.hpp"

namespace sc {

constexpr int kBandPanels = 32;               // panels (km = 4) per band
constexpr int kBandWaves = 16;                // waves per unit, two panels each
constexpr int kBandRows = 4 * kBandPanels;    // rows of C per band
constexpr int kBandCols = 64;                 // columns of B and C per N chunk
constexpr int kBandRowBytes = 4 * kBandCols;  // bytes of one staged B row
constexpr int kBandImgHeader = 16;            // dwords of a wave image header
constexpr int kBandImgMaxDw = 512;            // most dwords of one wave image
constexpr size_t kBandLdsBytes = 160 * 1024;
// The workspace of a plan with a band layout: partial tiles of at most
// kBandTargetUnits units (every geometry keeps units * chunks * bands under
// it when K is split) and one counter per (band, chunk).
constexpr int kBandTargetUnits = 256;
constexpr size_t kBandWorkFloats = (size_t)kBandTargetUnits * kBandRows * kBandCols;
constexpr size_t kBandCounters = kBandTargetUnits;
static_assert(kBandWorkFloats == kSplitWorkFloats && kBandCounters <= kSplitCounters,
              "the band kernel's split K fits the plan workspace");

// Wave image (dwords), one per (band, K tile, wave), 16-byte aligned:
//   [0], [1]  dense items of panels 0 and 1 (nd0, nd1)
//   [2]       single items (a multiple of 4)
//   [3], [4]  dword offsets of the dense and the single item areas
//   [5]       max(nd0, nd1)
//   [6..15]   0
// Dense area: item 0 is a zero item (the zero row, values 0), then panel 0's
// items, then panel 1's; a wave runs the two panels' lists in lockstep and
// the shorter list reads the zero item.  Single area: the single items of the
// eight lists k = 4p + r (panel p, row r) one list after another, padded to a
// multiple of four items with zero items of list 0.
//   dense item (20 dwords): the byte offsets of its four slots' rows in the
//     staged B tile (row * 256), then its 16 values laid out [panel row i]
//     [slot k], so that lane l reads its row's four values (l % 4) at once;
//   single item (8 dwords): the byte offsets of its four entries' rows, the
//     first one with the item's list k in its low bits (offsets are
//     multiples of 256), then the four values.
constexpr int kBandDenseDw = 20;
constexpr int kBandSingleDw = 8;
struct BandView {
  const int *img;   // wave images, 16-byte aligned each
  const int *woff;  // first dword of image (band * ntiles + tile) * 16 + wave, + end
  int nbands;
  int ntiles;
  int KT;           // B rows per K tile
  int wimg_dw;      // dwords reserved per wave image in LDS (multiple of 4)
};

// Launch shape of the band kernel for N columns.
struct BandGeometry {
  bool use = false;
  int nch = 0;   // N chunks of 64 columns
  int nks = 1;   // K ranges per (band, chunk)
  int tpu = 0;   // K tiles per unit
  unsigned grid = 0;
  size_t lds = 0;
  size_t work_floats = 0;  // partial sums needed (nks > 1)
  int counters = 0;
};

inline size_t band_stage_bytes(int KT) { return (size_t)(KT + 1) * kBandRowBytes; }

// The epilogue reuses the LDS for the single items' partial sums: 8 KiB per
// wave ([panel][row][slot group][64 columns]) and one flag.
constexpr size_t kBandRedBytes = (size_t)kBandWaves * 2 * 4 * 4 * kBandCols * sizeof(float) + 16;

inline size_t band_lds_bytes(int KT, int wimg_dw) {
  return std::max(2 * band_stage_bytes(KT) + (size_t)kBandWaves * wimg_dw * 4, kBandRedBytes);
}

// units: the most units the grid may hold (kBandTargetUnits for the plan's
// own workspace); work_cap: floats of workspace available.
inline BandGeometry band_geometry(const BandView &b, int N, int units = kBandTargetUnits,
                                  size_t work_cap = kBandWorkFloats) {
  BandGeometry g;
  if (!b.img || N <= 0 || N % kBandCols != 0 || b.nbands <= 0 || b.ntiles <= 0) return g;
  g.nch = N / kBandCols;
  g.lds = band_lds_bytes(b.KT, b.wimg_dw);
  if (g.lds > kBandLdsBytes) return g;
  const long long bc = (long long)b.nbands * g.nch;
  int nks = (int)std::max<long long>(1, std::min<long long>(b.ntiles, units / std::max<long long>(1, bc)));
  // the partial tiles must fit the workspace
  while (nks > 1 && (size_t)nks * bc * kBandRows * kBandCols > work_cap) --nks;
  g.tpu = (b.ntiles + nks - 1) / nks;
  g.nks = (b.ntiles + g.tpu - 1) / g.tpu;
  g.grid = (unsigned)(bc * g.nks);
  g.work_floats = g.nks > 1 ? (size_t)g.nks * bc * kBandRows * kBandCols : 0;
  g.counters = g.nks > 1 ? (int)bc : 0;
  if (g.nks > 1 && (bc > (long long)kBandCounters || g.work_floats > work_cap)) return g;
  g.use = true;
  return g;
}

typedef float vec4f_t __attribute__((ext_vector_type(4)));
typedef int vec2i __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) vec2i lds_int2;
typedef __attribute__((address_space(3))) char lds_char;

// The dense items of one lockstep step: item ja of panel 0 and jb of panel
// 1 (item 0 is the zero item), 16 MFMA blocks per slot.  tileb: this
// lane's column in the staged B tile (lane l -> column l).
__device__ __forceinline__ void band_dense_step(const lds_int *dense, int ja, int jb, const lds_char *tileb, int lane,
                                                vec4f_t (&D)[2][2]) {
  const vec4i ca = *(const lds_int4 *)(dense + kBandDenseDw * ja);
  const vec4i cb = *(const lds_int4 *)(dense + kBandDenseDw * jb);
  const vec4f a = *(const lds_float4 *)(dense + kBandDenseDw * ja + 4 + 4 * (lane & 3));
  const vec4f b = *(const lds_float4 *)(dense + kBandDenseDw * jb + 4 + 4 * (lane & 3));
  const float a0 = *(const lds_float *)(tileb + ca.x);
  const float a1 = *(const lds_float *)(tileb + ca.y);
  const float a2 = *(const lds_float *)(tileb + ca.z);
  const float a3 = *(const lds_float *)(tileb + ca.w);
  const float b0 = *(const lds_float *)(tileb + cb.x);
  const float b1 = *(const lds_float *)(tileb + cb.y);
  const float b2 = *(const lds_float *)(tileb + cb.z);
  const float b3 = *(const lds_float *)(tileb + cb.w);
  D[0][0] = __builtin_amdgcn_mfma_f32_4x4x1f32(a.x, a0, D[0][0], 0, 0, 0);
  D[1][0] = __builtin_amdgcn_mfma_f32_4x4x1f32(b.x, b0, D[1][0], 0, 0, 0);
  D[0][1] = __builtin_amdgcn_mfma_f32_4x4x1f32(a.y, a1, D[0][1], 0, 0, 0);
  D[1][1] = __builtin_amdgcn_mfma_f32_4x4x1f32(b.y, b1, D[1][1], 0, 0, 0);
  D[0][0] = __builtin_amdgcn_mfma_f32_4x4x1f32(a.z, a2, D[0][0], 0, 0, 0);
  D[1][0] = __builtin_amdgcn_mfma_f32_4x4x1f32(b.z, b2, D[1][0], 0, 0, 0);
  D[0][1] = __builtin_amdgcn_mfma_f32_4x4x1f32(a.w, a3, D[0][1], 0, 0, 0);
  D[1][1] = __builtin_amdgcn_mfma_f32_4x4x1f32(b.w, b3, D[1][1], 0, 0, 0);
}

// acc[0..3] += v * x[0..3] as four v_fmac_f32.  Volatile asm: the eight
// lists' cases of a switch stay apart, so the compiler cannot merge them into
// one update through a dynamic (scratch memory) index of the accumulators.
#define SC_BAND_FMA4(a, v, x)                                                                          \
  asm volatile("v_fmac_f32 %0, %4, %5\n\tv_fmac_f32 %1, %4, %6\n\tv_fmac_f32 %2, %4, %7\n\tv_fmac_f32 %3, %4, %8" \
               : "+v"(a[0]), "+v"(a[1]), "+v"(a[2]), "+v"(a[3])                                         \
               : "v"(v), "v"(x.x), "v"(x.y), "v"(x.z), "v"(x.w))

__device__ __forceinline__ void band_single_acc(int k, float v, const vec4f &x, float (&acc)[2][4][4]) {
  switch (k) {  // uniform: scalar branches
    case 0: SC_BAND_FMA4(acc[0][0], v, x); break;
    case 1: SC_BAND_FMA4(acc[0][1], v, x); break;
    case 2: SC_BAND_FMA4(acc[0][2], v, x); break;
    case 3: SC_BAND_FMA4(acc[0][3], v, x); break;
    case 4: SC_BAND_FMA4(acc[1][0], v, x); break;
    case 5: SC_BAND_FMA4(acc[1][1], v, x); break;
    case 6: SC_BAND_FMA4(acc[1][2], v, x); break;
    default: SC_BAND_FMA4(acc[1][3], v, x); break;
  }
}

// Four single items from item j on: lane (s, g) takes entry s = lane / 16 of
// each and columns 4g .. 4g+3.  All loads first, then the updates.  tileg:
// column group g in the staged B tile.
__device__ __forceinline__ void band_single_group(const lds_int *single, int j, int s, const lds_char *tileg,
                                                  float (&acc)[2][4][4]) {
  int o[4];
  float v[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    o[u] = single[kBandSingleDw * (j + u) + s];
    v[u] = *(const lds_float *)(single + kBandSingleDw * (j + u) + 4 + s);
  }
  int k[4];
  vec4f x[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    k[u] = uniform(o[u]) & 7;  // lane 0 holds entry 0, whose low bits carry the list
    x[u] = *(const lds_float4 *)(tileg + (o[u] & ~255));
  }
#pragma unroll
  for (int u = 0; u < 4; ++u) band_single_acc(k[u], v[u], x[u], acc);
}

// The band kernel (km = 4).  blockDim.x = 64 * kBandWaves.  Unit u of the
// grid: chunk = u % nch, ks = (u / nch) % nks, band = u / (nch * nks).
__global__ void __launch_bounds__(64 * kBandWaves)
    band_kernel(const int *__restrict__ img, const int *__restrict__ woff, const float *__restrict__ B,
                float *__restrict__ C, float *__restrict__ work, unsigned *__restrict__ counters, int M, int K,
                int N, int nbands, int ntiles, int KT, int wimg_dw, int nch, int nks, int tpu, int accumulate) {
  extern __shared__ float4 smem4[];
  constexpr int Q4 = kBandCols / 4;  // float4 per staged B row
  const int u = blockIdx.x;
  const int chunk = u % nch;
  const int ks = (u / nch) % nks;
  const int band = u / (nch * nks);
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int n0 = chunk * kBandCols;
  const int t0 = ks * tpu;
  const int t1 = min(ntiles, t0 + tpu);
  const size_t stage_bytes = (size_t)(KT + 1) * kBandRowBytes;
  char *lds = (char *)smem4;
  // stage st at lds + st * stage_bytes
  auto stage = [&](int st) { return (lds_float4 *)(lds + (size_t)st * stage_bytes); };
  lds_int *wimg = (lds_int *)(lds + 2 * stage_bytes) + w * wimg_dw;

  // the zero row (row KT) of both stages: padding slots read it
  if (threadIdx.x < 2 * Q4) stage(threadIdx.x / Q4)[KT * Q4 + (threadIdx.x % Q4)] = vec4f{0.f, 0.f, 0.f, 0.f};

  // B tile t into stage st by LDS DMA: one wave instruction moves four B
  // rows (lane l: row l / 16 of the four, 16 bytes of column group l % 16),
  // wave w the groups w, w + 16, ...; rows past the tile re-read its last row
  // (never referenced)
  auto dma = [&](int st, int t) {
    const int k0 = t * KT;
    const int rows = min(KT, K - k0);
    const int groups = (rows + 3) >> 2;
    const float *src = B + n0 + (lane & 15) * 4;
    for (int i = w; i < groups; i += kBandWaves) {
      const int r = min(4 * i + (lane >> 4), rows - 1);
      __builtin_amdgcn_global_load_lds(src + (size_t)(k0 + r) * N,
                                       (__attribute__((address_space(3))) void *)(stage(st) + 4 * i * Q4), 16, 0,
                                       0);
    }
  };
  // the wave's image of tile t: at most 2 float4 per lane, in registers until
  // the wave is done with the previous image
  vec4i prei[2];
  int nimg = 0;
  auto fetch_img = [&](int t) {
    const int a0 = woff[(band * ntiles + t) * kBandWaves + w];
    nimg = woff[(band * ntiles + t) * kBandWaves + w + 1] - a0;  // dwords, a multiple of 4
    const vec4i *src = reinterpret_cast<const vec4i *>(img + a0);
#pragma unroll
    for (int q = 0; q < 2; ++q)
      if (4 * (lane + 64 * q) < nimg) prei[q] = __builtin_nontemporal_load(src + lane + 64 * q);
  };
  auto put_img = [&]() {
    lds_int4 *dst = (lds_int4 *)wimg;
#pragma unroll
    for (int q = 0; q < 2; ++q)
      if (4 * (lane + 64 * q) < nimg) dst[lane + 64 * q] = prei[q];
  };

  vec4f_t D[2][2];
  float acc[2][4][4];
#pragma unroll
  for (int p = 0; p < 2; ++p) {
#pragma unroll
    for (int i = 0; i < 2; ++i) D[p][i] = vec4f_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[p][r][e] = 0.f;
  }

  if (t0 < t1) {
    dma(0, t0);
    fetch_img(t0);
    put_img();
  }
  __builtin_amdgcn_s_waitcnt(0);  // the DMA of the first tile has landed
  __syncthreads();
  for (int t = t0; t < t1; ++t) {
    const int st = (t - t0) & 1;
    const bool more = t + 1 < t1;
    if (more) {
      dma(st ^ 1, t + 1);
      fetch_img(t + 1);
    }
    {
      // the wave image header, as scalars
      const lds_int4 *h4 = (const lds_int4 *)wimg;
      const vec4i h0 = uniform4(h4[0]), h1 = uniform4(h4[1]);
      const lds_int *dense = wimg + h0.w;
      const lds_int *single = wimg + h1.x;
      // the stage; the byte offsets in the image add to it
      const lds_char *tbase = (const lds_char *)lds + (size_t)st * stage_bytes;
      const lds_char *tileb = tbase + 4 * lane;
      const lds_char *tileg = tbase + 16 * (lane & 15);
      // dense items: the two panels' lists in lockstep
      const int nd0 = h0.x, nd1 = h0.y;
      for (int i = 0; i < h1.y; ++i)
        band_dense_step(dense, i < nd0 ? 1 + i : 0, i < nd1 ? 1 + nd0 + i : 0, tileb, lane, D);
      // single items: four at a time
      const int s = lane >> 4;
      for (int j = 0; j < h0.z; j += 4) band_single_group(single, j, s, tileg, acc);
    }
    if (more) put_img();  // the wave is done with its previous image
    __builtin_amdgcn_s_waitcnt(0);  // this wave's DMA of the next tile has landed
    __syncthreads();
  }

  // single-item sums: every slot group s writes its partial row sums (4
  // columns per lane) to LDS, then lane l adds the four groups' values of
  // column l to its MFMA tiles.  The stages are free after the loop's last
  // barrier; each wave uses its own 8 KiB.
  const int s = lane >> 4;
  const int g = lane & 15;
  lds_float *red = (lds_float *)lds + w * (2 * 4 * 4 * kBandCols);  // [p][r][s][64]
#pragma unroll
  for (int p = 0; p < 2; ++p)
#pragma unroll
    for (int r = 0; r < 4; ++r)
      *(lds_float4 *)(red + ((p * 4 + r) * 4 + s) * kBandCols + 4 * g) =
          vec4f{acc[p][r][0], acc[p][r][1], acc[p][r][2], acc[p][r][3]};
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the wave's LDS writes are done
  __builtin_amdgcn_wave_barrier();
  float out[2][4];
#pragma unroll
  for (int p = 0; p < 2; ++p)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const lds_float *q = red + (p * 4 + i) * 4 * kBandCols + lane;
      out[p][i] = D[p][0][i] + D[p][1][i] + ((q[0] + q[kBandCols]) + (q[2 * kBandCols] + q[3 * kBandCols]));
    }

  // rows of this wave: band * 128 + (2w + p) * 4 + i, column n0 + lane
  const int rbase = band * kBandRows + 8 * w;
  if (nks == 1) {
#pragma unroll
    for (int p = 0; p < 2; ++p)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = rbase + 4 * p + i;
        if (row < M) {
          float *dst = C + (size_t)row * N + n0 + lane;
          *dst = accumulate ? *dst + out[p][i] : out[p][i];
        }
      }
    return;
  }
  // split K: this unit's partial tile (128 x 64, row-major) in the workspace
  const size_t tile_floats = (size_t)kBandRows * kBandCols;
  const size_t bc = (size_t)band * nch + chunk;
  float *mine = work + ((size_t)ks * nbands * nch + bc) * tile_floats;
#pragma unroll
  for (int p = 0; p < 2; ++p)
#pragma unroll
    for (int i = 0; i < 4; ++i)
      __hip_atomic_store(mine + (size_t)(8 * w + 4 * p + i) * kBandCols + lane, out[p][i], __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
  __builtin_amdgcn_s_waitcnt(0);  // this thread's partial stores have completed
  __syncthreads();
  int *flag = (int *)lds + kBandWaves * 2 * 4 * 4 * kBandCols;  // past the reduction area
  unsigned *cnt = counters + bc;
  if (threadIdx.x == 0) {
    const unsigned old = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *flag = old == (unsigned)(nks - 1);
  }
  __syncthreads();
  if (!*flag) return;
  // last unit of (band, chunk): the partials summed in K-range order
  const __amdgpu_buffer_rsrc_t wr =
      __builtin_amdgcn_make_buffer_rsrc(work, (short)0, (int)0x7fffffff, kBufferWord3);
  const size_t kstride = (size_t)nbands * nch * tile_floats;
  const unsigned off0 = (unsigned)((bc * tile_floats + (size_t)(8 * w) * kBandCols + lane) * 4);
  float sum[8];
  for (int k = 0; k < nks; ++k) {
    // the eight partials of range k, all loads in flight (sc1: read where
    // they were written through, not a stale copy in this XCD's L2)
    float x[8];
    if (k == ks) {
#pragma unroll
      for (int q = 0; q < 8; ++q) x[q] = out[q >> 2][q & 3];
    } else {
#pragma unroll
      for (int q = 0; q < 8; ++q)
        x[q] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                              wr, off0 + (unsigned)(q * kBandCols * 4), (unsigned)(k * kstride * 4),
                                              kCachePolicySc1));
    }
#pragma unroll
    for (int q = 0; q < 8; ++q) sum[q] = k == 0 ? x[q] : sum[q] + x[q];
  }
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const int row = rbase + q;
    if (row < M) {
      float *dst = C + (size_t)row * N + n0 + lane;
      *dst = accumulate ? *dst + sum[q] : sum[q];
    }
  }
  if (threadIdx.x == 0) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

inline hipError_t launch_band(const BandView &b, const BandGeometry &g, const float *B, float *C, float *work,
                              unsigned *counters, int M, int K, int N, int accumulate, hipStream_t stream) {
  if (!g.use) return hipErrorInvalidValue;
  if (g.grid == 0) return hipSuccess;
  hipLaunchKernelGGL(band_kernel, dim3(g.grid), dim3(64 * kBandWaves), g.lds, stream, b.img, b.woff, B, C, work,
                     counters, M, K, N, b.nbands, b.ntiles, b.KT, b.wimg_dw, g.nch, g.nks, g.tpu, accumulate);
  return hipGetLastError();
}

}  // namespace sc
