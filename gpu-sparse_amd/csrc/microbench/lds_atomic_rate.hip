// LDS atomic throughput on gfx950: ds_add_f32 vs ds_add_u32 vs ds_add_u64 vs a
// plain read-add-write, on random and conflict-free addresses.  Prints a table and
// one line "JSON {...}" with the rates in lane-ops/s over the whole GPU (and
// 32-bit slot adds/s: two per ds_add_u64).  Each lane keeps
// 16 fixed random word indices and xors them with a wave-uniform value per
// round, so one VALU op precedes each LDS op and the LDS pipe is the limit.
// Every address stays inside the workgroup's own 64 KiB allocation.
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <stdint.h>
constexpr int SLOTS = 16384;  // 64 KiB of 4-byte slots
constexpr int U = 16;
template <int MODE>
__global__ void __launch_bounds__(1024) k(float *out, int iters, int conflict_free) {
  __shared__ float accf[SLOTS];
  uint32_t *accu = reinterpret_cast<uint32_t *>(accf);
  unsigned long long *acc64 = reinterpret_cast<unsigned long long *>(accf);
  for (int i = threadIdx.x; i < SLOTS; i += blockDim.x) accf[i] = 0.f;
  __syncthreads();
  const int lane = threadIdx.x & 63;
  uint32_t h = (blockIdx.x * 1024 + threadIdx.x) * 2654435761u + 12345u;
  const uint32_t words = MODE == 3 ? SLOTS / 2 : SLOTS;  // elements of the accessed type
  uint32_t r[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    h ^= h << 13; h ^= h >> 17; h ^= h << 5;
    // conflict-free: lane l -> element l of a 64-element row (consecutive banks)
    r[u] = conflict_free ? (uint32_t)lane + 64u * ((h >> 20) % (words / 64)) : h % words;
  }
  for (int it = 0; it < iters; ++it) {
    const uint32_t s = (uint32_t)__builtin_amdgcn_readfirstlane((int)((it * 64u * 7u) % words)) & ~63u;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t a = r[u] ^ s;  // stays below `words` (a power of two)
      if (MODE == 0) __hip_atomic_fetch_add(&accf[a], 1.0f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      if (MODE == 1) __hip_atomic_fetch_add(&accu[a], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      if (MODE == 2) accu[a] = accu[a] + 1u;
      if (MODE == 3) __hip_atomic_fetch_add(&acc64[a], 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
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
  const int blocks = 2048, iters = 256;
  const char *names[] = {"ds_add_f32 (atomic)", "ds_add_u32 (atomic)", "ds_read+add+ds_write", "ds_add_u64 (atomic)"};
  const char *keys[] = {"ds_add_f32", "ds_add_u32", "ds_read_add_write", "ds_add_u64"};
  char json[2048];
  int jn = snprintf(json, sizeof json, "{");
  for (int cf = 0; cf < 2; ++cf)
    for (int mode = 0; mode < 4; ++mode) {
      for (int rep = 0; rep < 2; ++rep) {
        (void)hipEventRecord(e0);
        if (mode == 0) k<0><<<blocks, 1024>>>(out, iters, cf);
        if (mode == 1) k<1><<<blocks, 1024>>>(out, iters, cf);
        if (mode == 2) k<2><<<blocks, 1024>>>(out, iters, cf);
        if (mode == 3) k<3><<<blocks, 1024>>>(out, iters, cf);
        (void)hipEventRecord(e1);
        (void)hipEventSynchronize(e1);
        float ms = 0;
        (void)hipEventElapsedTime(&ms, e0, e1);
        const double ops = (double)blocks * 1024 * iters * U;
        if (rep) {
          const double rate = ops / (ms * 1e-3);  // lane-ops per second over the whole GPU
          printf("%-22s %s: %8.3f ms  %.3e lane-ops/s  %.2f lane-ops/clk/CU (2.4 GHz, 256 CU)\n", names[mode],
                 cf ? "conflict-free" : "random       ", ms, rate, rate / 2.4e9 / 256);
          // 32-bit slots added per second: a ds_add_u64 adds two
          jn += snprintf(json + jn, sizeof json - jn,
                         "%s\"%s_%s\": {\"ms\": %.4f, \"lane_ops_per_s\": %.4e, \"slot_adds_per_s\": %.4e}",
                         jn > 1 ? ", " : "", keys[mode], cf ? "conflict_free" : "random", ms, rate,
                         rate * (mode == 3 ? 2.0 : 1.0));
        }
      }
    }
  hipError_t e = hipDeviceSynchronize();
  printf("status %s\n", hipGetErrorString(e));
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, 0) == hipSuccess)
    jn += snprintf(json + jn, sizeof json - jn, ", \"device\": \"%s\", \"cus\": %d, \"clock_khz\": %d",
                   prop.gcnArchName, prop.multiProcessorCount, prop.clockRate);
  snprintf(json + jn, sizeof json - jn, ", \"ops_per_lane\": %d, \"blocks\": %d, \"threads\": 1024}", iters * U, blocks);
  printf("JSON %s\n", json);
  return 0;
}
