// LDS atomic throughput on gfx950: ds_add_f32 vs ds_add_u32 vs a plain
// read-add-write, random and conflict-free addresses.  Every address is masked
// into the workgroup's own 64 KiB allocation.
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <stdint.h>
constexpr int SLOTS = 16384;  // 64 KiB of 4-byte slots
template <int MODE>
__global__ void __launch_bounds__(1024) k(float *out, int iters, int stride_mode) {
  __shared__ float accf[SLOTS];
  uint32_t *accu = reinterpret_cast<uint32_t *>(accf);
  for (int i = threadIdx.x; i < SLOTS; i += blockDim.x) accf[i] = 0.f;
  __syncthreads();
  uint32_t h = (blockIdx.x * 1024 + threadIdx.x) * 2654435761u + 12345u;
  for (int it = 0; it < iters; ++it) {
    h ^= h << 13; h ^= h >> 17; h ^= h << 5;
    uint32_t a = stride_mode ? ((threadIdx.x & 63) + 64 * ((h >> 20) & 255)) & (SLOTS - 1) : (h & (SLOTS - 1));
    if (MODE == 0) __hip_atomic_fetch_add(&accf[a], 1.0f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    if (MODE == 1) __hip_atomic_fetch_add(&accu[a], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    if (MODE == 2) { accf[a] = accf[a] + 1.0f; }
  }
  __syncthreads();
  if (threadIdx.x == 0) out[blockIdx.x] = accf[blockIdx.x & (SLOTS - 1)];
}
int main() {
  float *out;
  if (hipMalloc(&out, 4096 * 4) != hipSuccess) return 1;
  hipEvent_t e0, e1;
  (void)hipEventCreate(&e0);
  (void)hipEventCreate(&e1);
  const int blocks = 2048, iters = 4096;
  const char *names[] = {"ds_add_f32 (atomic)", "ds_add_u32 (atomic)", "ds_read+add+ds_write"};
  for (int sm = 0; sm < 2; ++sm)
  for (int mode = 0; mode < 3; ++mode) {
    for (int rep = 0; rep < 2; ++rep) {
      (void)hipEventRecord(e0);
      if (mode == 0) k<0><<<blocks, 1024>>>(out, iters, sm);
      if (mode == 1) k<1><<<blocks, 1024>>>(out, iters, sm);
      if (mode == 2) k<2><<<blocks, 1024>>>(out, iters, sm);
      (void)hipEventRecord(e1);
      (void)hipEventSynchronize(e1);
      float ms = 0;
      (void)hipEventElapsedTime(&ms, e0, e1);
      double ops = (double)blocks * 1024 * iters;
      if (rep) printf("%-24s %s: %8.3f ms  %.2f lane-ops/clk/CU (2.4 GHz, 256 CU)\n", names[mode],
                      sm ? "conflict-free" : "random     ", ms, ops / (ms * 1e-3) / 2.4e9 / 256);
    }
  }
  hipError_t e = hipDeviceSynchronize(); printf("status %s\n", hipGetErrorString(e));
  return 0;
}
