// L1 access-pattern microbenchmark (gfx950): the cost of a wave's 16-byte global accesses in
// the lane orders the expert kernels use, each wave reading or writing 8 KiB-apart blocks
// of an L2-resident window in a loop.  Prints, per pattern, the kernel time and the cycles
// per wave access per CU (time x 2.4 GHz / accesses per CU).  The patterns, for a 16-row
// block of a row-major operand with 512-byte rows:
//   contiguous   lane l: bytes 16 l of one 1 KiB block (a packed MFMA fragment)
//   quad-major   lane 4 r + q: row r, 16-byte chunk q (each lane quad one row's 64 bytes)
//   mfma-order   lane 16 q + r: row r, chunk q (the MFMA operand / accumulator order:
//                a lane quad spans four rows)
//   8 rows x 128 B, 4 rows x 256 B: wider row segments per lane group
// as loads, stores and LDS-DMA copies (global_load_lds_dwordx4), plus ds_bpermute.
// Build and run: hipcc --offload-arch=gfx950 -O3 -std=c++17 -o l1_access l1_access.hip
// (not part of libnsmoe.so: nanospeaker_amd/build.py compiles csrc/*.hip only).
#include <hip/hip_runtime.h>
#include <cstdio>
#include <cstdint>
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4;
constexpr int WIN = 1 << 20;  // bytes of source window (L2-resident, shared by all WGs)
__device__ __forceinline__ int off_of(int pat, int l) {
  switch (pat) {
    case 0: return 16 * l;                                   // contiguous 1 KiB
    case 1: return (l >> 2) * 512 + (l & 3) * 16;            // quad-major: 16 rows x 64 B
    case 2: return (l & 15) * 512 + (l >> 4) * 16;           // mfma order: 16 rows x 64 B
    case 3: return (l >> 3) * 512 + (l & 7) * 16;            // 8 rows x 128 B
    case 4: return (l >> 4) * 512 + (l & 15) * 16;           // 4 rows x 256 B
    default: return 16 * l;
  }
}
template <int PAT>
__global__ void __launch_bounds__(256) ld_kernel(const char* __restrict__ src, uint32_t* out, int iters) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int o = off_of(PAT, lane);
  u32x4 acc = {0, 0, 0, 0};
  uint32_t base = (blockIdx.x * 4 + wave) * 8192u;
  for (int it = 0; it < iters; ++it) {
    u32x4 v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const uint32_t b = (base + (it * 4 + u) * 8192u) & (WIN - 1);
      v[u] = *(const u32x4*)(src + b + o);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) acc ^= v[u];
  }
  if ((acc[0] ^ acc[1] ^ acc[2] ^ acc[3]) == 0x12345678u) out[blockIdx.x] = 1;
}
template <int PAT>
__global__ void __launch_bounds__(256) st_kernel(char* __restrict__ dst, int iters) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int o = off_of(PAT, lane);
  const uint32_t base = (blockIdx.x * 4 + wave) * 8192u;
  u32x4 v = {(uint32_t)lane, 1u, 2u, 3u};
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const uint32_t b = (base + (it * 4 + u) * 8192u) & (8 * WIN - 1);
      *(u32x4*)(dst + b + o) = v;
    }
    v[1] += 1u;
  }
}
__global__ void __launch_bounds__(256) bperm_kernel(uint32_t* out, int iters) {
  const int lane = threadIdx.x & 63;
  const int a = (4 * (lane & 15) + (lane >> 4)) << 2;
  uint32_t v0 = lane, v1 = lane * 3, v2 = lane * 5, v3 = lane * 7;
  for (int it = 0; it < iters; ++it) {
    v0 = __builtin_amdgcn_ds_bpermute(a, v0) + 1;
    v1 = __builtin_amdgcn_ds_bpermute(a, v1) + 1;
    v2 = __builtin_amdgcn_ds_bpermute(a, v2) + 1;
    v3 = __builtin_amdgcn_ds_bpermute(a, v3) + 1;
  }
  if ((v0 ^ v1 ^ v2 ^ v3) == 0x12345678u) out[blockIdx.x] = 1;
}
__device__ __forceinline__ void async_copy16(const void* gsrc, char* lds_wave_base) {
  const uint32_t lds = __builtin_amdgcn_readfirstlane(
      (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)lds_wave_base);
  uint32_t saved;
  asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off\n\ts_mov_b32 m0, %0"
               : "=&s"(saved) : "v"(gsrc), "s"(lds) : "memory");
}
template <int PAT>
__global__ void __launch_bounds__(256) dma_kernel(const char* __restrict__ src, uint32_t* out, int iters) {
  __shared__ __attribute__((aligned(1024))) char s[4][4][1024];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int o = off_of(PAT, lane);
  uint32_t base = (blockIdx.x * 4 + wave) * 8192u;
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const uint32_t b = (base + (it * 4 + u) * 8192u) & (WIN - 1);
      async_copy16(src + b + o, s[wave][u]);
    }
    asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (*(const uint32_t*)&s[0][0][lane * 4] == 0x12345678u) out[blockIdx.x] = 1;
}
int main() {
  char *src, *dst; uint32_t* out;
  if (hipMalloc(&src, 8 * WIN) != hipSuccess || hipMalloc(&dst, 8 * WIN) != hipSuccess ||
      hipMalloc(&out, 1 << 16) != hipSuccess || hipMemset(src, 1, 8 * WIN) != hipSuccess ||
      hipMemset(out, 0, 1 << 16) != hipSuccess) {
    printf("allocation failed\n");
    return 1;
  }
  const int grid = 768, iters = 256;
  hipEvent_t a, b;
  (void)hipEventCreate(&a);
  (void)hipEventCreate(&b);
  auto timeit = [&](const char* name, auto launch, double instrs_per_wave) {
    launch();
    (void)hipDeviceSynchronize();
    (void)hipEventRecord(a);
    for (int r = 0; r < 5; ++r) launch();
    (void)hipEventRecord(b);
    (void)hipEventSynchronize(b);
    float ms = 0.0f;
    (void)hipEventElapsedTime(&ms, a, b);
    ms /= 5;
    const double waves_per_cu = grid * 4 / 256.0;
    const double cyc = ms * 1e-3 * 2.4e9;
    printf("%-22s %8.2f us  %7.1f cycles per wave-instr per CU (at 2.4 GHz)\n", name, ms * 1e3, cyc / (waves_per_cu * instrs_per_wave));
  };
  const double n = 4.0 * iters;
  timeit("load contiguous", [&] { ld_kernel<0><<<grid, 256>>>(src, out, iters); }, n);
  timeit("load quad-major", [&] { ld_kernel<1><<<grid, 256>>>(src, out, iters); }, n);
  timeit("load mfma-order", [&] { ld_kernel<2><<<grid, 256>>>(src, out, iters); }, n);
  timeit("load 8rows x128B", [&] { ld_kernel<3><<<grid, 256>>>(src, out, iters); }, n);
  timeit("load 4rows x256B", [&] { ld_kernel<4><<<grid, 256>>>(src, out, iters); }, n);
  timeit("store contiguous", [&] { st_kernel<0><<<grid, 256>>>(dst, iters); }, n);
  timeit("store quad-major", [&] { st_kernel<1><<<grid, 256>>>(dst, iters); }, n);
  timeit("store mfma-order", [&] { st_kernel<2><<<grid, 256>>>(dst, iters); }, n);
  timeit("store 8rows x128B", [&] { st_kernel<3><<<grid, 256>>>(dst, iters); }, n);
  timeit("dma contiguous", [&] { dma_kernel<0><<<grid, 256>>>(src, out, iters); }, n);
  timeit("dma quad-major", [&] { dma_kernel<1><<<grid, 256>>>(src, out, iters); }, n);
  timeit("dma mfma-order", [&] { dma_kernel<2><<<grid, 256>>>(src, out, iters); }, n);
  timeit("bpermute", [&] { bperm_kernel<<<grid, 256>>>(out, iters * 4); }, 4.0 * iters * 4);
  printf("status: %s\n", hipGetErrorString(hipGetLastError()));
  return 0;
}
