// ubench_memory.hip -- ceilings of the data paths the pattern kernels use on
// gfx950: random 512-byte row gathers from an L2-resident table (the B-row
// gathers of the wide kernel), contiguous streaming reads from L2, the
// strided K x Nc column-chunk reads that stage a B chunk in LDS, LDS read
// bandwidth (b64/b128), LDS b128 reads of random rows (lanes over slots),
// L1-hit reads, and the issue rate of the fp32 MFMA shapes a km = 4 slot
// maps to (v_mfma_f32_4x4x1f32: one 4x1 column block times 64 columns of B).
// All indices are masked into their buffers; every loop has a fixed trip count.
//   hipcc --offload-arch=gfx950 -O3 -Xclang -target-feature -Xclang -packed-fp32-ops \
//         ubench_memory.hip -o ../../lib/ubench_memory
#include <hip/hip_runtime.h>
#include <cstdio>
#include <cstdint>
#include <vector>

#define CK(x) do { hipError_t e_ = (x); if (e_ != hipSuccess) { printf("HIP error %s at %d\n", hipGetErrorString(e_), __LINE__); return 1; } } while (0)

// Random 512-byte row gathers (float2 per lane, 64 lanes) from a table of
// `rows` rows; row index from a xorshift per wave (uniform).  U loads in flight.
template <int U>
__global__ void gather_rows(const float2 *__restrict__ tab, int rows_mask, int iters, float *out) {
  const int lane = threadIdx.x & 63;
  unsigned st = 0x9E3779B9u * (blockIdx.x * 16 + (threadIdx.x >> 6) + 1);
  st = __builtin_amdgcn_readfirstlane(st);
  float acc = 0.f;
  for (int it = 0; it < iters; ++it) {
    float2 b[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      st ^= st << 13; st ^= st >> 17; st ^= st << 5;
      const int r = (int)(st & (unsigned)rows_mask);
      b[u] = tab[(size_t)r * 64 + lane];
    }
#pragma unroll
    for (int u = 0; u < U; ++u) acc += b[u].x * b[u].y;
  }
  if (acc == 1234.5f) out[0] = acc;
}

// LDS reads: each lane reads float2 (b64) or float4 (b128) at a lane-strided
// address; `iters` rounds over a 32 KiB array.
template <int VEC>
__global__ void lds_read(int iters, float *out) {
  __shared__ float s[8192];
  for (int t = threadIdx.x; t < 8192; t += blockDim.x) s[t] = (float)t;
  __syncthreads();
  const int lane = threadIdx.x & 63;
  float acc = 0.f;
  int base = (threadIdx.x >> 6) * 512;
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int off = ((base + u * 64 * VEC + lane * VEC) & (8192 - VEC));
      if constexpr (VEC == 4) {
        float4 v = *reinterpret_cast<const float4 *>(&s[off]);
        acc += v.x + v.y + v.z + v.w;
      } else {
        float2 v = *reinterpret_cast<const float2 *>(&s[off]);
        acc += v.x + v.y;
      }
    }
    base += 256;
  }
  if (acc == 1234.5f) out[0] = acc;
}

// Contiguous runs from an L2-resident buffer: per iteration each wave reads
// U consecutive 1 KiB pieces (float4 per lane) starting at a random piece
// (scalar xorshift), wrapping in `mask64`.
template <int U>
__global__ void stream_l2(const float4 *__restrict__ buf, int mask64, int iters, float *out) {
  const int lane = threadIdx.x & 63;
  unsigned st = 0x9E3779B9u * (blockIdx.x * 16 + (threadIdx.x >> 6) + 1);
  st = __builtin_amdgcn_readfirstlane(st);
  float acc = 0.f;
  for (int it = 0; it < iters; ++it) {
    st ^= st << 13; st ^= st >> 17; st ^= st << 5;
    const int piece = (int)st;
    float4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = buf[(size_t)((piece + u) & mask64) * 64 + lane];
#pragma unroll
    for (int u = 0; u < U; ++u) acc += v[u].x + v[u].w;
  }
  if (acc == 1234.5f) out[0] = acc;
}

// Column-chunk staging: block b copies rows 0..K-1, columns [c0, c0+NC) of a
// row-major K x 128 fp32 matrix into LDS (NC/4 lanes per row, float4 each),
// the load pattern of a B chunk staged for lanes-over-slots kernels.
template <int NC>
__global__ void chunk_stage(const float4 *__restrict__ B, int K, int reps, float *out) {
  extern __shared__ float4 lds4[];
  const int per_row = NC / 4;
  const int c0 = (blockIdx.x % (128 / NC)) * NC;
  float acc = 0.f;
  for (int r = 0; r < reps; ++r) {
    for (int t = threadIdx.x; t < K * per_row; t += blockDim.x) {
      const int row = t / per_row, q = t % per_row;
      lds4[t] = B[(size_t)row * 32 + c0 / 4 + q];
    }
    __syncthreads();
    acc += lds4[(threadIdx.x * 7 + r) % (K * per_row)].x;
    __syncthreads();
  }
  if (acc == 1234.5f) out[0] = acc;
}

// LDS b128 reads of rows: lanes are (slot, part) with LPS lanes per slot;
// lane q of a slot reads bytes [16q, 16q+16) of its row (row stride
// STRIDE_F4 float4) in a 128 KiB array.  Per iteration each slot draws a
// random start row r0 < NROWS/2 (RANDOM) or takes r0 = its slot number
// (consecutive rows, the conflict-free control), then reads rows
// r0 + u*NROWS/32 for u < 16 (immediate offsets, so the loop is LDS-bound).
template <int LPS, int STRIDE_F4, int NROWS, bool RANDOM>
__global__ void lds_rows(int iters, float *out) {
  extern __shared__ float4 lds4[];
  for (int t = threadIdx.x; t < NROWS * STRIDE_F4; t += blockDim.x) lds4[t] = make_float4(t, 0, 0, 0);
  __syncthreads();
  const int lane = threadIdx.x & 63;
  const int q = lane % LPS;
  const int slot = lane / LPS;
  unsigned st = 0x9E3779B9u * (blockIdx.x * 1024 + threadIdx.x / LPS + 1);
  constexpr int D = NROWS / 32;
  float acc = 0.f;
  for (int it = 0; it < iters; ++it) {
    int r0;
    if constexpr (RANDOM) {
      st ^= st << 13; st ^= st >> 17; st ^= st << 5;
      r0 = (int)(st & (NROWS / 2 - 1));
    } else {
      r0 = (slot + it) & (NROWS / 2 - 1);
    }
    const float4 *p = lds4 + r0 * STRIDE_F4 + q;
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      float4 v = p[u * D * STRIDE_F4];
      // keep all four dwords live without spending VALU on them
      asm volatile("" : : "v"(v.x), "v"(v.y), "v"(v.z), "v"(v.w));
    }
    acc += (float)r0;
  }
  if (acc == 1234.5f) out[0] = acc;
}

// L1-resident reads: each wave re-reads the same 8 KiB window.
__global__ void l1_read(const float4 *__restrict__ buf, int iters, float *out) {
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  float acc = 0.f;
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      float4 v = buf[(size_t)((w * 8 + u) & 7) * 64 + lane];  // 8 x 1 KiB = 8 KiB per block
      acc += v.x + v.y + v.z + v.w;
    }
  }
  if (acc == 1234.5f) out[0] = acc;
}

// fp32 MFMA issue rate: 8 independent accumulator chains per wave, `iters`
// steps each.  KIND 0: v_mfma_f32_4x4x1f32 (16 blocks of 4x4x1), KIND 1:
// v_mfma_f32_16x16x4f32.
typedef float v4f_t __attribute__((ext_vector_type(4)));
template <int KIND>
__global__ void __launch_bounds__(256) mfma_rate(float a, float b, int iters, float *out) {
  v4f_t acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = (v4f_t){0.f, 0.f, 0.f, 0.f};
  const float x = a + (float)threadIdx.x;
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (KIND == 0) acc[i] = __builtin_amdgcn_mfma_f32_4x4x1f32(x, b, acc[i], 0, 0, 0);
      else acc[i] = __builtin_amdgcn_mfma_f32_16x16x4f32(x, b, acc[i], 0, 0, 0);
    }
  }
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) s += acc[i][0] + acc[i][1] + acc[i][2] + acc[i][3];
  if (s == 1234.5f) out[0] = s;
}

int main() {
  hipDeviceProp_t prop;
  CK(hipGetDeviceProperties(&prop, 0));
  printf("device %s CUs %d clock %d kHz L2 %d bytes LDS/block %zu\n", prop.gcnArchName,
         prop.multiProcessorCount, prop.clockRate, prop.l2CacheSize, prop.sharedMemPerBlock);
  const int CUs = prop.multiProcessorCount;
  float *out;
  CK(hipMalloc(&out, 4));
  hipEvent_t e0, e1;
  CK(hipEventCreate(&e0));
  CK(hipEventCreate(&e1));
  // gather table: 4096 rows x 512 B = 2 MiB (L2 resident per XCD)
  const int rows = 4096;
  float2 *tab;
  CK(hipMalloc(&tab, (size_t)rows * 512));
  CK(hipMemset(tab, 0, (size_t)rows * 512));
  for (int wpb : {4, 8, 16}) {
    const int blocks = CUs * 4;
    const int iters = 64;
    hipLaunchKernelGGL(gather_rows<8>, dim3(blocks), dim3(64 * wpb), 0, 0, tab, rows - 1, iters, out);
    CK(hipDeviceSynchronize());
    CK(hipEventRecord(e0));
    for (int rep = 0; rep < 10; ++rep)
      hipLaunchKernelGGL(gather_rows<8>, dim3(blocks), dim3(64 * wpb), 0, 0, tab, rows - 1, iters, out);
    CK(hipEventRecord(e1));
    CK(hipEventSynchronize(e1));
    float ms;
    CK(hipEventElapsedTime(&ms, e0, e1));
    double bytes = 10.0 * blocks * wpb * iters * 8 * 512.0;
    printf("gather U=8 waves/block=%d blocks=%d: %.2f TB/s (%.1f B/clk/CU)\n", wpb, blocks,
           bytes / (ms * 1e-3) / 1e12, bytes / (ms * 1e-3) / CUs / (prop.clockRate * 1e3));
  }
  for (int wpb : {4, 8, 16}) {
    const int blocks = CUs * 4;
    const int iters = 64;
    hipLaunchKernelGGL(gather_rows<16>, dim3(blocks), dim3(64 * wpb), 0, 0, tab, rows - 1, iters, out);
    CK(hipDeviceSynchronize());
    CK(hipEventRecord(e0));
    for (int rep = 0; rep < 10; ++rep)
      hipLaunchKernelGGL(gather_rows<16>, dim3(blocks), dim3(64 * wpb), 0, 0, tab, rows - 1, iters, out);
    CK(hipEventRecord(e1));
    CK(hipEventSynchronize(e1));
    float ms;
    CK(hipEventElapsedTime(&ms, e0, e1));
    double bytes = 10.0 * blocks * wpb * iters * 16 * 512.0;
    printf("gather U=16 waves/block=%d blocks=%d: %.2f TB/s (%.1f B/clk/CU)\n", wpb, blocks,
           bytes / (ms * 1e-3) / 1e12, bytes / (ms * 1e-3) / CUs / (prop.clockRate * 1e3));
  }
  {
    const int blocks = CUs * 2, wpb = 16, iters = 256;
    for (int vec : {2, 4}) {
      auto k = vec == 2 ? lds_read<2> : lds_read<4>;
      hipLaunchKernelGGL(k, dim3(blocks), dim3(64 * wpb), 0, 0, iters, out);
      CK(hipDeviceSynchronize());
      CK(hipEventRecord(e0));
      for (int rep = 0; rep < 10; ++rep) hipLaunchKernelGGL(k, dim3(blocks), dim3(64 * wpb), 0, 0, iters, out);
      CK(hipEventRecord(e1));
      CK(hipEventSynchronize(e1));
      float ms;
      CK(hipEventElapsedTime(&ms, e0, e1));
      double bytes = 10.0 * blocks * wpb * iters * 8 * 64.0 * vec * 4;
      printf("lds b%d: %.2f TB/s (%.1f B/clk/CU)\n", vec * 32, bytes / (ms * 1e-3) / 1e12,
             bytes / (ms * 1e-3) / CUs / (prop.clockRate * 1e3));
    }
  }
  {
    // contiguous reads of the 2 MiB table (L2 resident)
    const int blocks = CUs * 4, wpb = 8, iters = 64;  // runs of 8 KiB
    for (int rep = -1; rep < 10; ++rep) {
      if (rep == 0) CK(hipEventRecord(e0));
      hipLaunchKernelGGL(stream_l2<8>, dim3(blocks), dim3(64 * wpb), 0, 0, (const float4 *)tab,
                         (rows * 512 / 1024) - 1, iters, out);
    }
    CK(hipEventRecord(e1));
    CK(hipEventSynchronize(e1));
    float ms;
    CK(hipEventElapsedTime(&ms, e0, e1));
    double bytes = 10.0 * blocks * wpb * iters * 8 * 1024.0;
    printf("contiguous 8 KiB runs from l2: %.2f TB/s (%.1f B/clk/CU)\n", bytes / (ms * 1e-3) / 1e12,
           bytes / (ms * 1e-3) / CUs / (prop.clockRate * 1e3));
  }
  {
    // column-chunk staging: K = 4096 rows of the 4096 x 128 table, NC = 8 / 16 / 32 columns
    const int K = 4096, blocks = CUs, reps = 8;
    struct { int nc, lds; void (*k)(const float4 *, int, int, float *); } cfgs[] = {
        {8, 4096 * 32, chunk_stage<8>}, {16, 2048 * 64, chunk_stage<16>}, {32, 1024 * 128, chunk_stage<32>}};
    for (auto &c : cfgs) {
      const int Kc = c.lds / (c.nc * 4);
      CK(hipFuncSetAttribute((const void *)c.k, hipFuncAttributeMaxDynamicSharedMemorySize, c.lds));
      for (int rep = -1; rep < 10; ++rep) {
        if (rep == 0) CK(hipEventRecord(e0));
        hipLaunchKernelGGL(c.k, dim3(blocks), dim3(1024), c.lds, 0, (const float4 *)tab, Kc, reps, out);
      }
      CK(hipEventRecord(e1));
      CK(hipEventSynchronize(e1));
      float ms;
      CK(hipEventElapsedTime(&ms, e0, e1));
      double bytes = 10.0 * blocks * reps * (double)c.lds;
      printf("chunk stage NC=%d (%d rows): %.2f TB/s (%.1f B/clk/CU)\n", c.nc, Kc,
             bytes / (ms * 1e-3) / 1e12, bytes / (ms * 1e-3) / CUs / (prop.clockRate * 1e3));
    }
    (void)K;
  }
  {
    // LDS b128 reads of random rows: 64-byte rows (NC=16, 4 lanes per slot) and
    // 128-byte rows (NC=32, 8 lanes per slot), dense or padded by 16 bytes
    const int blocks = CUs, wpb = 16, iters = 256;
    struct { const char *name; int lps, stride; void (*k)(int, float *); } cfgs[] = {
        {"64B rows, 4 lanes/slot, consecutive", 4, 4, lds_rows<4, 4, 2048, false>},
        {"64B rows, 4 lanes/slot, random", 4, 4, lds_rows<4, 4, 2048, true>},
        {"64B rows +16B pad, 4 lanes/slot, random", 4, 5, lds_rows<4, 5, 1024, true>},
        {"128B rows, 8 lanes/slot, consecutive", 8, 8, lds_rows<8, 8, 1024, false>},
        {"128B rows, 8 lanes/slot, random", 8, 8, lds_rows<8, 8, 1024, true>},
        {"128B rows +16B pad, 8 lanes/slot, random", 8, 9, lds_rows<8, 9, 512, true>},
        {"256B rows, 16 lanes/slot, random", 16, 16, lds_rows<16, 16, 512, true>}};
    for (auto &c : cfgs) {
      const int lds = 131072;
      CK(hipFuncSetAttribute((const void *)c.k, hipFuncAttributeMaxDynamicSharedMemorySize, lds));
      for (int rep = -1; rep < 10; ++rep) {
        if (rep == 0) CK(hipEventRecord(e0));
        hipLaunchKernelGGL(c.k, dim3(blocks), dim3(64 * wpb), lds, 0, iters, out);
      }
      CK(hipEventRecord(e1));
      CK(hipEventSynchronize(e1));
      float ms;
      CK(hipEventElapsedTime(&ms, e0, e1));
      double bytes = 10.0 * blocks * wpb * iters * 16 * 64.0 * 16;
      printf("lds rows b128 (%s): %.2f TB/s (%.1f B/clk/CU)\n", c.name,
             bytes / (ms * 1e-3) / 1e12, bytes / (ms * 1e-3) / CUs / (prop.clockRate * 1e3));
    }
  }
  {
    const int blocks = CUs * 2, wpb = 16, iters = 256;
    hipLaunchKernelGGL(l1_read, dim3(blocks), dim3(64 * wpb), 0, 0, (const float4 *)tab, iters, out);
    CK(hipDeviceSynchronize());
    CK(hipEventRecord(e0));
    for (int rep = 0; rep < 10; ++rep)
      hipLaunchKernelGGL(l1_read, dim3(blocks), dim3(64 * wpb), 0, 0, (const float4 *)tab, iters, out);
    CK(hipEventRecord(e1));
    CK(hipEventSynchronize(e1));
    float ms;
    CK(hipEventElapsedTime(&ms, e0, e1));
    double bytes = 10.0 * blocks * wpb * iters * 8 * 1024.0;
    printf("l1 read dwordx4: %.2f TB/s (%.1f B/clk/CU)\n", bytes / (ms * 1e-3) / 1e12,
           bytes / (ms * 1e-3) / CUs / (prop.clockRate * 1e3));
  }
  {
    // 4 waves per SIMD; cycles per MFMA per SIMD at the reported clock
    const int blocks = 4 * CUs, iters = 2000;
    for (int kind = 0; kind < 2; ++kind) {
      float ms = 0.f;
      for (int rep = 0; rep < 2; ++rep) {  // first launch warms up
        CK(hipEventRecord(e0));
        if (kind == 0) hipLaunchKernelGGL(mfma_rate<0>, dim3(blocks), dim3(256), 0, 0, 1.f, 2.f, iters, out);
        else hipLaunchKernelGGL(mfma_rate<1>, dim3(blocks), dim3(256), 0, 0, 1.f, 2.f, iters, out);
        CK(hipEventRecord(e1));
        CK(hipEventSynchronize(e1));
        CK(hipEventElapsedTime(&ms, e0, e1));
      }
      const double per_simd = (double)blocks * 4 * iters * 8 / (4.0 * CUs);
      const double fmas = kind == 0 ? 256.0 : 1024.0;
      printf("mfma %s: %.1f cycles per instruction per SIMD, %.1f fp32 TFLOP/s\n",
             kind == 0 ? "f32_4x4x1 (16 blocks)" : "f32_16x16x4", ms * 1e-3 * prop.clockRate * 1e3 / per_simd,
             2.0 * fmas * per_simd * 4 * CUs / (ms * 1e-3) / 1e12);
    }
  }
  return 0;
}
