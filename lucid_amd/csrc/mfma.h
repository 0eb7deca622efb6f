// CDNA4 (gfx950) MFMA helpers shared by the LUCID kernels.
//
// All contractions use v_mfma_f32_32x32x16_bf16 (one wave64, 32x32 fp32 tile,
// 16-deep bf16 reduction).  Lane layouts (checked on an MI355X):
//   A operand [m][k]: lane l holds A[l%32][8*(l/32) + e], e = 0..7
//   B operand [k][n]: lane l holds B[8*(l/32) + e][l%32], e = 0..7
//   C/D       [m][n]: lane l holds D[8*(e/4) + 4*(l/32) + e%4][l%32], e = 0..15
//
// "Transposed" tiles: a score tile is computed as D[m = key j][n = row i] so
// that lane <-> row i and the 16 fp32 values of a lane run over keys j.  That
// D tile, converted to bf16, is directly the B operand [k = j][n = i] of the
// next MFMA, provided the A operand of that MFMA stores its k index (j) in
// the order the D layout produces: within every aligned group of 16, logical
// k slot kappa holds position jmap(kappa), where jmap swaps bits 2 and 3.
// Operand matrices that are consumed this way are kept in HBM as "T-perm"
// tiles: [head][d][T] with the T index permuted by jmap inside each 16-group.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

#define LOG2E_F 1.4426950408889634f

// Two waves per SIMD: caps a kernel at 256 VGPR+AGPR per lane so that the MFMA
// work of one wave overlaps the exp/VALU work of the other (one wave per SIMD
// leaves the matrix core idle while its own softmax-style VALU code runs).
#define LUCID_TWO_WAVES_IF(COND) __attribute__((amdgpu_waves_per_eu((COND) ? 2 : 1)))

__device__ __forceinline__ f32x16 mfma32(const bf16x8& a, const bf16x8& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int e = 0; e < 16; ++e) z[e] = 0.f;
  return z;
}

// accumulator with every element x (an MFMA then adds its product to x)
__device__ __forceinline__ f32x16 splat16(float x) {
  f32x16 z;
#pragma unroll
  for (int e = 0; e < 16; ++e) z[e] = x;
  return z;
}

// position of sequence index j inside a T-perm row (involution on the low 4 bits)
__host__ __device__ __forceinline__ int jmap(int j) {
  return (j & ~0xC) | ((j & 4) << 1) | ((j & 8) >> 1);
}

// D-layout row (m) of element e for lane group g = lane/32
__device__ __forceinline__ int drow(int e, int g) { return 8 * (e >> 2) + 4 * g + (e & 3); }

__device__ __forceinline__ bf16x8 ld8(const bf16* p) { return *reinterpret_cast<const bf16x8*>(p); }

// acc + the sum of eight bf16 values (four v_dot2 against (1, 1)): the row sums of a
// softmax taken from the same bf16 values that enter its P V product
__device__ __forceinline__ float add_sum8(const bf16x8& p, float acc) {
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  const bf16x2 ones = {(bf16)1.0f, (bf16)1.0f};
#pragma unroll
  for (int k = 0; k < 4; ++k)
    acc = __builtin_amdgcn_fdot2_f32_bf16(bf16x2{p[2 * k], p[2 * k + 1]}, ones, acc, false);
  return acc;
}

// eight bf16 values times a in fp32, rounded once to bf16
__device__ __forceinline__ bf16x8 scale8(const bf16x8& x, float a) {
  bf16x8 r;
#pragma unroll
  for (int e = 0; e < 8; ++e) r[e] = (bf16)(a * (float)x[e]);
  return r;
}

// Pack D-layout fp32 values e = 8h .. 8h+7 into a bf16 B operand (k-step h of the tile)
__device__ __forceinline__ bf16x8 pack_b(const f32x16& x, int h) {
  bf16x8 r;
#pragma unroll
  for (int e = 0; e < 8; ++e) r[e] = (bf16)x[8 * h + e];
  return r;
}

// Reductions of a value over lane pairs (l, l ^ 32), the two halves of a D-layout row.
// v_permlane32_swap exchanges the lane halves in the VALU (no LDS round trip): of the
// two results, one holds this lane's value and the other its partner's, so the
// symmetric reduction of the pair is the same on both lanes.
__device__ __forceinline__ float wave_max32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, v), __builtin_bit_cast(unsigned, v),
                                                  false, false);
  return fmaxf(__builtin_bit_cast(float, (unsigned)r[0]), __builtin_bit_cast(float, (unsigned)r[1]));
}
__device__ __forceinline__ float wave_sum32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, v), __builtin_bit_cast(unsigned, v),
                                                  false, false);
  return __builtin_bit_cast(float, (unsigned)r[0]) + __builtin_bit_cast(float, (unsigned)r[1]);
}

// Chain progress counters.  A producer writes a finished block, makes it
// visible at agent scope (release fence: the L2 of its XCD is written back) and
// then stores its progress counter.  Consumers poll the counter with relaxed
// agent-scope loads (they read the coherent value without cache maintenance).
//
// Once the awaited progress has been seen a consumer needs only an ordering
// fence, not an agent-scope acquire (which would invalidate the whole L2 of the
// XCD for every other workgroup on it): the chain operands are laid out so that
// one 64-row block fills whole 128-byte cache lines, no line of a block is read
// by anyone before the block is published within the kernel, and the caches
// are invalidated at kernel start, so neither this CU's L1 nor this XCD's L2 can
// hold a stale copy of the lines read after the wait.  Workspaces must
// therefore be 256-byte aligned (checked at the C ABI).
__device__ __forceinline__ int poll_counter(const int* cnt) {
  return __hip_atomic_load(cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void chain_acquire() { __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup"); }

// Bounded waits.  In-order dispatch makes every wait end (a workgroup waits only on
// blocks of lower ids, which are running or done), so a wait that lasts longer than
// chain_wait_ticks of the constant-rate wall clock means that the protocol broke: it
// stores 1 to *chain_error (pinned host memory set up by the library's C ABI, which
// reports it on the next call) and returns, so that every wave of the kernel still
// finishes -- the results of that launch are then invalid.  Each library (translation
// unit) has its own pair, set per device by chain_guard.h.
static __device__ long long chain_wait_ticks = 200000000LL;  // 2 s at the 100 MHz wall clock
static __device__ int* chain_error = nullptr;

// Wait until *cnt > target (or the bound above); returns the value seen.
__device__ __forceinline__ int wait_counter_gt(const int* cnt, int target) {
  int v = poll_counter(cnt);
  if (v <= target) {
    const long long t0 = wall_clock64();
    const long long limit = chain_wait_ticks;
    while (v <= target) {
      __builtin_amdgcn_s_sleep(1);
      v = poll_counter(cnt);
      if (v <= target && wall_clock64() - t0 > limit) {
        int* err = chain_error;
        if (err) __hip_atomic_store(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        break;
      }
    }
  }
  chain_acquire();
  return v;
}
