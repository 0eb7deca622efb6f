// fp32 atomic-add throughput probe for gfx950 (a measurement tool, not part of the library):
// each of 4096 workgroups adds a 64x64 fp32 tile partial per step into a rotating target tile
// (the dQ accumulation a fused dK/dV' + dQ sweep would need), 128 steps, with
// global_atomic_add_f32 (unsafeAtomicAdd); the same pattern with plain stores for comparison.
// Targets stay inside the 128 MB buffer (tile index mod NT, offsets below 4096 per tile).
// Build: hipcc --offload-arch=gfx950 -O3 -o atomic_add_probe lucid_amd/csrc/atomic_add_probe.hip
#include <hip/hip_runtime.h>
#include <cstdio>
constexpr int NT = 8192;            // target tiles (64x64 fp32 = 16 KB each): 128 MB
constexpr int STEPS = 128;
__global__ __launch_bounds__(256) void k_atomic(float* buf, int spread) {
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  float v = 1.0f + 1e-3f * (float)tid;
  for (int st = 0; st < STEPS; ++st) {
    const int tile = (blockIdx.x * spread + st) % NT;
    float* t = buf + (size_t)tile * 4096 + w * 1024;
#pragma unroll
    for (int i = 0; i < 16; ++i) unsafeAtomicAdd(t + i * 64 + lane, v);
  }
}
__global__ __launch_bounds__(256) void k_store(float* buf, int spread) {
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  float v = 1.0f + 1e-3f * (float)tid;
  for (int st = 0; st < STEPS; ++st) {
    const int tile = (blockIdx.x * spread + st) % NT;
    float* t = buf + (size_t)tile * 4096 + w * 1024;
#pragma unroll
    for (int i = 0; i < 16; ++i) t[i * 64 + lane] = v + (float)st;
  }
}
int main() {
  float* buf;
  if (hipMalloc(&buf, (size_t)NT * 4096 * 4)) return 1;
  if (hipMemset(buf, 0, (size_t)NT * 4096 * 4)) return 1;
  hipEvent_t a, b;
  if (hipEventCreate(&a) || hipEventCreate(&b)) return 1;
  const int grid = 4096;
  for (int spread : {1, 2, 7}) {
    for (int rep = 0; rep < 3; ++rep) {
      float ms1 = 0, ms2 = 0;
      if (hipEventRecord(a)) return 2;
      k_atomic<<<grid, 256>>>(buf, spread);
      if (hipEventRecord(b) || hipEventSynchronize(b) || hipEventElapsedTime(&ms1, a, b)) return 2;
      if (hipEventRecord(a)) return 2;
      k_store<<<grid, 256>>>(buf, spread);
      if (hipEventRecord(b) || hipEventSynchronize(b) || hipEventElapsedTime(&ms2, a, b)) return 2;
      const double n = (double)grid * STEPS * 4096;
      printf("spread %d: atomic %.3f ms (%.2f T adds/s, %.0f GB/s), store %.3f ms (%.0f GB/s)\n", spread, ms1,
             n / ms1 / 1e9, n * 4 / ms1 / 1e6, ms2, n * 4 / ms2 / 1e6);
      fflush(stdout);
    }
  }
  return 0;
}
