// LDS bank-conflict calibration for gfx950 (a measurement tool, not part of the library):
// one kernel per access pattern, each reading LDS 512 times per wave, so that
// rocprofv3 SQ_LDS_BANK_CONFLICT / (waves x 512) gives the conflict cycles of one read.
// Patterns: contiguous 16/8/4-byte reads (no conflicts by construction), one bank per
// wave (the worst case), a 32-byte lane stride (two lanes per bank group), and the
// operand reads of the LUCID kernels on a swizzled 128-byte-row tile: 16-byte reads of
// one chunk by 32 consecutive rows and the transposing read ds_read_b64_tr_b16, with the
// shipped swizzle (chunk c of row r at c ^ (r & 7)), without a swizzle, and with the
// conflict-free alternative c ^ bitrev3((r >> 1) & 7).  Every address stays inside the
// 64 KB LDS array (tile index masked, offsets below the tile size).
// Build: hipcc --offload-arch=gfx950 -O3 -o lds_bank_probe lucid_amd/csrc/lds_bank_probe.hip
#include <hip/hip_runtime.h>
#include <cstdio>
typedef __bf16 bf16;
typedef bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
constexpr int NIT = 512;
constexpr int LDS_BYTES = 65536;

#define PROLOGUE \
  __shared__ __attribute__((aligned(16))) unsigned char lds[LDS_BYTES]; \
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6; \
  for (int i = tid; i < LDS_BYTES / 4; i += 256) reinterpret_cast<float*>(lds)[i] = (float)(i & 255); \
  __syncthreads(); \
  float acc = 0.f;

#define EPILOGUE out[blockIdx.x * 256 + tid] = acc;

// A: 16-byte reads, 64 lanes read 1 KB contiguous
__global__ __launch_bounds__(256) void k_b128_linear(float* out) {
  PROLOGUE
  _Pragma("unroll 1") for (int it = 0; it < NIT; ++it) {
    const int off = ((it * 4 + w) * 1024 + lane * 16) & (LDS_BYTES - 1);
    const f32x4 v = *reinterpret_cast<const f32x4*>(lds + off);
    acc += v[0] + v[1] + v[2] + v[3];
  }
  EPILOGUE
}
// B: the MFMA A-operand read of a swizzled row tile (8 chunks of 16 B per row, chunk c of
// row r at c ^ (r & 7)): lane reads row lane%32, chunk kb + lane/32
__global__ __launch_bounds__(256) void k_b128_swz(float* out) {
  PROLOGUE
  _Pragma("unroll 1") for (int it = 0; it < NIT; ++it) {
    const int r = lane & 31, c = ((2 * (it & 3) + (lane >> 5)) ^ (r & 7));
    const int tile = ((it >> 2) * 4 + w) & 15;  // 16 tiles of 4 KB (32 rows x 128 B)
    const int off = tile * 4096 + r * 128 + c * 16;
    const f32x4 v = *reinterpret_cast<const f32x4*>(lds + off);
    acc += v[0] + v[1] + v[2] + v[3];
  }
  EPILOGUE
}
// C: the same operand without the swizzle (row stride 128 B: every 8 rows share banks)
__global__ __launch_bounds__(256) void k_b128_noswz(float* out) {
  PROLOGUE
  _Pragma("unroll 1") for (int it = 0; it < NIT; ++it) {
    const int r = lane & 31, c = 2 * (it & 3) + (lane >> 5);
    const int tile = ((it >> 2) * 4 + w) & 15;
    const int off = tile * 4096 + r * 128 + c * 16;
    const f32x4 v = *reinterpret_cast<const f32x4*>(lds + off);
    acc += v[0] + v[1] + v[2] + v[3];
  }
  EPILOGUE
}
// D: 8-byte reads, contiguous
__global__ __launch_bounds__(256) void k_b64_linear(float* out) {
  PROLOGUE
  _Pragma("unroll 1") for (int it = 0; it < NIT; ++it) {
    const int off = ((it * 4 + w) * 512 + lane * 8) & (LDS_BYTES - 1);
    const float2 v = *reinterpret_cast<const float2*>(lds + off);
    acc += v.x + v.y;
  }
  EPILOGUE
}
// E: 4-byte reads, contiguous
__global__ __launch_bounds__(256) void k_b32_linear(float* out) {
  PROLOGUE
  _Pragma("unroll 1") for (int it = 0; it < NIT; ++it) {
    const int off = ((it * 4 + w) * 256 + lane * 4) & (LDS_BYTES - 1);
    acc += *reinterpret_cast<const float*>(lds + off);
  }
  EPILOGUE
}
// F: the transposing read (ds_read_b64_tr_b16) of a swizzled 8-chunk row tile, as the
// kernels issue it for an A operand at row0 (multiple of 16), column block col0
__global__ __launch_bounds__(256) void k_tr_swz(float* out) {
  PROLOGUE
  typedef __attribute__((address_space(3))) bf16x4 lds_bf16x4;
  const bf16* tileb = reinterpret_cast<const bf16*>(lds);
  _Pragma("unroll 1") for (int it = 0; it < NIT; ++it) {
    const int s = lane & 15, col0 = 32 * (it & 1), row0 = 16 * ((it >> 1) & 3);
    const int col = col0 + 16 * ((lane >> 4) & 1) + 4 * (s & 3);
    const int r1 = row0 + 4 * (lane >> 5) + (s >> 2);
    const int o = (((col >> 3) ^ (r1 & 7)) << 3) | (col & 7);
    const int tile = ((it >> 3) * 4 + w) & 7;  // 8 tiles of 8 KB (64 rows x 64 bf16)
    const bf16* t = tileb + tile * 4096;
    const bf16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(t + r1 * 64 + o));
    acc += (float)v[0] + (float)v[1] + (float)v[2] + (float)v[3];
  }
  EPILOGUE
}
// G: 16-byte reads with a 32-byte lane stride (two lanes per bank group: 2-way)
__global__ __launch_bounds__(256) void k_b128_stride32(float* out) {
  PROLOGUE
  _Pragma("unroll 1") for (int it = 0; it < NIT; ++it) {
    const int off = ((it * 4 + w) * 2048 + lane * 32) & (LDS_BYTES - 1);
    const f32x4 v = *reinterpret_cast<const f32x4*>(lds + off);
    acc += v[0] + v[1] + v[2] + v[3];
  }
  EPILOGUE
}
// H: 4-byte reads, all 64 lanes of a wave on one bank (128-byte lane stride)
__global__ __launch_bounds__(256) void k_b32_samebank(float* out) {
  PROLOGUE
  _Pragma("unroll 1") for (int it = 0; it < NIT; ++it) {
    const int off = ((it * 4 + w) * 4 + lane * 128) & (LDS_BYTES - 1);
    acc += *reinterpret_cast<const float*>(lds + off);
  }
  EPILOGUE
}
// I: global_load_lds_dwordx4 (direct HBM/L2 -> LDS, 1 KB per instruction), NIT/8 rounds
__global__ __launch_bounds__(256) void k_dma(const bf16* src, float* out) {
  PROLOGUE
  bf16* l = reinterpret_cast<bf16*>(lds);
  for (int it = 0; it < NIT / 8; ++it) {
    const int piece = (it * 4 + w) & 63;  // 64 pieces of 1 KB
    __builtin_amdgcn_global_load_lds(src + (size_t)(blockIdx.x & 63) * 32768 + piece * 512 + lane * 8, l + piece * 512, 16, 0, 0);
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  acc += reinterpret_cast<const float*>(lds)[tid];
  EPILOGUE
}


// bitrev3((r >> 1) & 7)
__device__ __forceinline__ int fnew8(int r) { const int x = (r >> 1) & 7; return ((x & 1) << 2) | (x & 2) | (x >> 2); }
// B2: the operand read with the new CPR-8 swizzle
__global__ __launch_bounds__(256) void k_b128_swz_new(float* out) {
  PROLOGUE
  _Pragma("unroll 1") for (int it = 0; it < NIT; ++it) {
    const int r = lane & 31, c = ((2 * (it & 3) + (lane >> 5)) ^ fnew8(r));
    const int tile = ((it >> 2) * 4 + w) & 15;
    const int off = tile * 4096 + r * 128 + c * 16;
    const f32x4 v = *reinterpret_cast<const f32x4*>(lds + off);
    acc += v[0] + v[1] + v[2] + v[3];
  }
  EPILOGUE
}
// F2: the transposing read with the new CPR-8 swizzle (rows r1 and r1 + 8 alternate)
__global__ __launch_bounds__(256) void k_tr_swz_new(float* out) {
  PROLOGUE
  typedef __attribute__((address_space(3))) bf16x4 lds_bf16x4;
  const bf16* tileb = reinterpret_cast<const bf16*>(lds);
  _Pragma("unroll 1") for (int it = 0; it < NIT; ++it) {
    const int s = lane & 15, col0 = 32 * (it & 1), row0 = 16 * ((it >> 1) & 3) + 8 * ((it >> 3) & 1);
    const int col = col0 + 16 * ((lane >> 4) & 1) + 4 * (s & 3);
    const int r1 = row0 + 4 * (lane >> 5) + (s >> 2);
    const int o = (((col >> 3) ^ fnew8(r1)) << 3) | (col & 7);
    const int tile = ((it >> 4) * 4 + w) & 7;
    const bf16* t = tileb + tile * 4096;
    const bf16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(t + r1 * 64 + o));
    acc += (float)v[0] + (float)v[1] + (float)v[2] + (float)v[3];
  }
  EPILOGUE
}

int main() {
  const int grid = 1024;
  float* out;
  bf16* src;
  if (hipMalloc(&out, grid * 256 * 4) || hipMalloc(&src, 64 * 32768 * 2)) return 1;
  if (hipMemset(src, 0, 64 * 32768 * 2)) return 1;
  hipEvent_t a, b;
  if (hipEventCreate(&a) || hipEventCreate(&b)) return 1;
#define RUN(NAME, ...)                                                       \
  {                                                                          \
    if (hipEventRecord(a)) return 2;                                         \
    NAME<<<grid, 256>>>(__VA_ARGS__);                                        \
    if (hipEventRecord(b) || hipEventSynchronize(b)) return 2;               \
    float ms = 0.f;                                                          \
    if (hipEventElapsedTime(&ms, a, b)) return 2;                            \
    printf("%-18s %.4f ms\n", #NAME, ms); fflush(stdout);                   \
  }
  for (int rep = 0; rep < 2; ++rep) {
    RUN(k_b128_linear, out) RUN(k_b128_swz, out) RUN(k_b128_noswz, out) RUN(k_b64_linear, out)
    RUN(k_b32_linear, out) RUN(k_tr_swz, out) RUN(k_b128_stride32, out) RUN(k_b32_samebank, out)
    RUN(k_dma, src, out) RUN(k_b128_swz_new, out) RUN(k_tr_swz_new, out)
  }
  printf("done\n");
  return 0;
}
