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
// Measured on MI355X (structured 4096 x 4096 at 10 % density, N = 128):
// 33.3 us per launch against the panel kernel's 21.8, with 0.89 M L2 read
// requests against 3.29 M.  The item loop waits on one LDS round trip per
// step, and the split-K epilogue plus the first tile cost about 16 k cycles
// of the unit's 64 k.  So plans build the band layout only when asked
// (SC_PLAN_BANDS).
//
// Work decomposition.  A unit (workgroup of 16 waves) owns one band, one N
// chunk of 64 columns and one range of K tiles (split K, so that the grid
// covers the 256 CUs).  Per tile it stages B[tile rows, chunk] (256 bytes a
// row, one extra row of zeros for padding) and each wave its own part of the
// tile's stream (the wave image) in LDS, double-buffered for B, while the
// waves compute the previous tile.  Wave w owns panels 2w and 2w + 1 of the
// band.  A panel's slots in a tile, in column order, come four to an item
// and every item runs on the matrix cores, whatever its slots' patterns
// (rows a pattern lacks carry value 0): v_mfma_f32_4x4x1f32 has 16 blocks of
// a 4-row by 4-column product; block b = 4s + c of an item takes slot s and
// columns 16c + 4j + q (j the block's column, q = 0..3 over four
// instructions), so lane 16s + 4c + j reads its slot's value for row j (the A
// operand) with one 4-byte LDS read and the 16 bytes at column 16c + 4j of
// the slot's B row with one 16-byte read that feeds the four instructions.
// Each block accumulates its slot's products; the four slots' partial sums
// (lanes 16s + x, s = 0..3) are added once, after the last tile.  A wave
// runs its two panels' item lists in lockstep and reads the next step's
// values and offsets together with the current step's B rows.  Items are
// padded to four slots with value 0 on the zero row.
//
// Numerics.  Rows a slot's pattern lacks are multiplied by 0 here, as the
// format's own padding slots are in the reference's kernels: with finite B
// the sums equal the pattern bodies' to rounding, while an Inf or NaN in a B
// row can reach a row of C that has no entry in that column (0 * Inf = NaN).
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
constexpr int kBandImgHeader = 4;             // dwords of a wave image header
constexpr int kBandImgMaxDw = 768;            // most dwords of one wave image (3 x 16 bytes a lane)
constexpr size_t kBandLdsBytes = 160 * 1024;
// The workspace of a plan with a band layout: partial tiles of at most
// kBandTargetUnits units (every geometry keeps units * chunks * bands under
// it when K is split) and one counter per (band, chunk).
constexpr int kBandTargetUnits = 256;
constexpr size_t kBandWorkFloats = (size_t)kBandTargetUnits * kBandRows * kBandCols;
constexpr size_t kBandCounters = kBandTargetUnits;
static_assert(kBandWorkFloats == kSplitWorkFloats && kBandCounters <= kSplitCounters,
              "the band kernel's split K fits the plan workspace");

// Wave image (dwords), one per (band, wave, K tile) and stored in that
// order (a wave's tiles one after another), 16-byte aligned:
//   [0], [1]  items of panels 0 and 1 (n0, n1)
//   [2]       max(n0, n1)
//   [3]       0
// then the items: item 0 is the zero item (the zero row, values 0), then
// panel 0's n0 items, then panel 1's n1.  A wave runs the two panels' lists in
// lockstep and the shorter list reads the zero item.
//   item (20 dwords): its 16 values laid out [slot k][panel row i] (0 where
//     slot k's pattern lacks row i), then the byte offsets of its four slots'
//     rows in the staged B tile (row * 256; the zero row for padding slots).
constexpr int kBandItemDw = 20;
struct BandView {
  const int *img;   // wave images, 16-byte aligned each
  const int *woff;  // first dword of image (band * 16 + wave) * ntiles + tile, + end
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

__host__ __device__ inline size_t band_stage_bytes(int KT) { return (size_t)(KT + 1) * kBandRowBytes; }

// After the last tile the LDS holds each wave's sums, one column per lane:
// 2 KiB a wave ([panel][row][64 columns]); the split-K flag follows both.
constexpr size_t kBandRedBytes = (size_t)kBandWaves * 2 * 4 * kBandCols * sizeof(float);

__host__ __device__ inline size_t band_flag_offset(int KT, int wimg_dw) {
  const size_t a = 2 * band_stage_bytes(KT) + (size_t)kBandWaves * wimg_dw * 4;
  return a > kBandRedBytes ? a : kBandRedBytes;
}

inline size_t band_lds_bytes(int KT, int wimg_dw) { return band_flag_offset(KT, wimg_dw) + 16; }

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
  if (g.tpu + 1 > 64) return g;  // a unit's image offsets sit in one register, a lane per tile
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

// One lockstep step: item ja of panel 0 and jb of panel 1 (item 0 is the
// zero item), this lane's A value and B-row offset of each.  aoff: byte
// offset of the lane's value in an item (slot s = lane / 16, row lane % 4);
// ooff: byte offset of slot s's B-row offset.
struct BandStep {
  float a, b;
  int oa, ob;
};

__device__ __forceinline__ BandStep band_load_step(const lds_char *items, int ja, int jb, int aoff, int ooff) {
  BandStep s;
  const lds_char *ia = items + kBandItemDw * 4 * ja;
  const lds_char *ib = items + kBandItemDw * 4 * jb;
  s.a = *(const lds_float *)(ia + aoff);
  s.b = *(const lds_float *)(ib + aoff);
  s.oa = *(const lds_int *)(ia + ooff);
  s.ob = *(const lds_int *)(ib + ooff);
  return s;
}

// The band kernel (km = 4).  blockDim.x = 64 * kBandWaves.  Unit u of the
// grid: chunk = u % nch, ks = (u / nch) % nks, band = u / (nch * nks).
__global__ void __launch_bounds__(64 * kBandWaves)
    band_kernel(const int *__restrict__ img, const int *__restrict__ woff, const float *__restrict__ B,
                float *__restrict__ C, float *__restrict__ work, unsigned *__restrict__ counters, int M, int K,
                int N, int nbands, int ntiles, int KT, int wimg_dw, int nch, int nks, int tpu, int accumulate) {
  extern __shared__ float4 smem4[];
  constexpr int Q4 = kBandCols / 4;  // float4 per staged B row
  constexpr int IQ = kBandImgMaxDw / 256;  // float4 of a wave image per lane
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
  // the offsets of this wave's images of tiles t0 .. t1 (and the end of the
  // last), lane t - t0 holding tile t's: read once, so that no tile waits
  // for a scalar load of its image's place
  const int *wo = woff + (size_t)(band * kBandWaves + w) * ntiles + t0;
  const int woffv = lane <= t1 - t0 ? wo[lane] : 0;
  // the wave's image of tile t: at most IQ float4 per lane, in registers
  // until the wave is done with the previous image; its header goes to
  // scalar registers when it is put to LDS
  vec4i prei[IQ];
  int nimg = 0;
  vec4i hdr = vec4i{0, 0, 0, 0};
  auto fetch_img = [&](int t) {
    const int a0 = __builtin_amdgcn_readlane(woffv, t - t0);
    nimg = __builtin_amdgcn_readlane(woffv, t - t0 + 1) - a0;  // dwords, a multiple of 4
    const vec4i *src = reinterpret_cast<const vec4i *>(img + a0);
#pragma unroll
    for (int q = 0; q < IQ; ++q)
      if (4 * (lane + 64 * q) < nimg) prei[q] = __builtin_nontemporal_load(src + lane + 64 * q);
  };
  auto put_img = [&]() {
    lds_int4 *dst = (lds_int4 *)wimg;
#pragma unroll
    for (int q = 0; q < IQ; ++q)
      if (4 * (lane + 64 * q) < nimg) dst[lane + 64 * q] = prei[q];
    hdr = uniform4(prei[0]);  // lane 0: the image's first four dwords
  };

  // D[p][q]: panel p, column 4x + q of slot s's partial sum in lane
  // 16s + x (x = lane % 16), register i row i of the panel
  vec4f_t D[2][4];
#pragma unroll
  for (int p = 0; p < 2; ++p)
#pragma unroll
    for (int q = 0; q < 4; ++q) D[p][q] = vec4f_t{0.f, 0.f, 0.f, 0.f};

  if (t0 < t1) {
    dma(0, t0);
    fetch_img(t0);
    put_img();
  }
  __builtin_amdgcn_s_waitcnt(0);  // the DMA of the first tile has landed
  __syncthreads();
  const int aoff = 4 * (4 * (lane >> 4) + (lane & 3));
  const int ooff = 64 + 4 * (lane >> 4);
  for (int t = t0; t < t1; ++t) {
    const int st = (t - t0) & 1;
    const bool more = t + 1 < t1;
    if (more) {
      dma(st ^ 1, t + 1);
      fetch_img(t + 1);
    }
    {
      const vec4i h = hdr;
      const lds_char *items = (const lds_char *)(wimg + kBandImgHeader);
      // this lane's 16 bytes (columns 4x .. 4x+3) of a staged row; the byte
      // offsets in the items add to it
      const lds_char *tileb = (const lds_char *)lds + (size_t)st * stage_bytes + 16 * (lane & 15);
      const int na = h.x, nb = h.y, nmax = h.z;
      BandStep cur = band_load_step(items, na > 0 ? 1 : 0, nb > 0 ? 1 + na : 0, aoff, ooff);
      for (int i = 0; i < nmax; ++i) {
        // the next step's values and offsets first (past the lists' ends:
        // the zero item), then this step's B rows: LDS reads return in
        // order, so the one wait for the B rows also covers the next step,
        // and both round trips overlap
        const lds_char *pa = tileb + cur.oa, *pb = tileb + cur.ob;
        __builtin_amdgcn_sched_barrier(0);
        const int j = i + 1;
        const BandStep nxt = band_load_step(items, j < na ? 1 + j : 0, j < nb ? 1 + na + j : 0, aoff, ooff);
        __builtin_amdgcn_sched_barrier(0);
        const vec4f xa = *(const lds_float4 *)pa;
        const vec4f xb = *(const lds_float4 *)pb;
        __builtin_amdgcn_sched_barrier(0);
        D[0][0] = __builtin_amdgcn_mfma_f32_4x4x1f32(cur.a, xa.x, D[0][0], 0, 0, 0);
        D[1][0] = __builtin_amdgcn_mfma_f32_4x4x1f32(cur.b, xb.x, D[1][0], 0, 0, 0);
        D[0][1] = __builtin_amdgcn_mfma_f32_4x4x1f32(cur.a, xa.y, D[0][1], 0, 0, 0);
        D[1][1] = __builtin_amdgcn_mfma_f32_4x4x1f32(cur.b, xb.y, D[1][1], 0, 0, 0);
        D[0][2] = __builtin_amdgcn_mfma_f32_4x4x1f32(cur.a, xa.z, D[0][2], 0, 0, 0);
        D[1][2] = __builtin_amdgcn_mfma_f32_4x4x1f32(cur.b, xb.z, D[1][2], 0, 0, 0);
        D[0][3] = __builtin_amdgcn_mfma_f32_4x4x1f32(cur.a, xa.w, D[0][3], 0, 0, 0);
        D[1][3] = __builtin_amdgcn_mfma_f32_4x4x1f32(cur.b, xb.w, D[1][3], 0, 0, 0);
        cur = nxt;
      }
    }
    if (more) put_img();  // the wave is done with its previous image
    __builtin_amdgcn_s_waitcnt(0);  // this wave's DMA of the next tile has landed
    __syncthreads();
  }

  // the four slots' partial sums: lanes x, 16 + x, 32 + x, 48 + x into lane x
#pragma unroll
  for (int p = 0; p < 2; ++p)
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float v = D[p][q][i];
        v += lane_down<32>(v);
        v += lane_down<16>(v);
        D[p][q][i] = v;
      }
  // to one column per lane through LDS (the stages are free after the
  // loop's last barrier; each wave its own 2 KiB, [p][row][64 columns])
  lds_float *red = (lds_float *)lds + w * (2 * 4 * kBandCols);
  if (lane < 16) {
#pragma unroll
    for (int p = 0; p < 2; ++p)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        *(lds_float4 *)(red + (p * 4 + i) * kBandCols + 4 * lane) =
            vec4f{D[p][0][i], D[p][1][i], D[p][2][i], D[p][3][i]};
  }
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the wave's LDS writes are done
  __builtin_amdgcn_wave_barrier();
  float out[2][4];
#pragma unroll
  for (int p = 0; p < 2; ++p)
#pragma unroll
    for (int i = 0; i < 4; ++i) out[p][i] = red[(p * 4 + i) * kBandCols + lane];

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
  int *flag = (int *)(lds + band_flag_offset(KT, wimg_dw));
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
