// ubench_memory.hip -- ceilings of the data paths the pattern kernels use on
// gfx950: random 512-byte row gathers from an L2-resident table (the B-row
// gathers of the wide kernel), LDS read bandwidth (b64/b128) and L1-hit reads.
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
  return 0;
}
