// Shared device helpers for the LUCID kernels (chain counters, triangular
// inverse of a 64x64 diagonal block, fp32 -> bf16 hi/lo split).
#pragma once
#include "mfma.h"

namespace lucid {

// element strides of a [B, H, T, d] (or [B, T, H, d]) tensor; d is contiguous
struct Strides {
  int64_t b, h, t;
};

// Precision of the preconditioner chains, chosen per head.  The off-diagonal products
// P_ij V'_j (forward), P_ij dV_i (transposed solve) and the M = (dV V'^T) * P sums of the
// backward accumulate over every earlier (later) key of a row, and with bf16 operands
// their rounding error grows like 2^-8 |V'| sqrt(m_i), m_i = sum_{j<i} P_ij^2 (measured
// on CPU emulations of the kernels: ~1e-3 sqrt(m) relative for V' and dV).  A head whose
// largest row mass exceeds kExactMass runs the exact chain kernels, which carry V' and
// dV as bf16 hi/lo pairs and split every such product into hi*hi + hi*lo + lo*hi (~fp32
// accuracy); the others run the bf16 kernels.  Keys with no common direction
// (N(0,1)-like) give m ~ 1e-2; keys along a shared direction give m ~ T.
constexpr float kExactMass = 4.0f;

// Staged tiles in flight in the backward sweeps: three buffers (the tile in use, the next
// one landed, the one after in flight), two for the fp32-input instances at head dim 128,
// whose hi and lo tiles would not fit three deep in the 160 KB of LDS (the next tile is
// then waited for at the end of each step).
constexpr int stage_bufs(int D, bool F32) { return (F32 && D == 128) ? 2 : 3; }

// fp32 inputs (F32 kernel instances): each fp32 input X reaches the kernels as two bf16
// tensors, X ~= X_hi + X_lo (lucid_split_kernel: 16 significant bits), and every product
// with an input operand takes three MFMAs (hi*hi + hi*lo + lo*hi).  The score products
// (K.K of P, Q.K of the softmax) take the fourth, lo*lo, as well: where the two operands
// share a direction (a key with itself or its neighbours, keys along a common direction)
// the lo parts are correlated and the dropped lo*lo terms add up instead of cancelling,
// a bias of ~2^-18 |k|^2 in the exponent's argument (a 2e-4 relative V' error at
// correlated keys, T = 1024, against 1.5e-5 with it).  The hi copies are passed in
// the kernels' ordinary bf16 arguments; this struct carries the lo copies (same layouts,
// same strides) and the fp32 values themselves where a kernel reads them directly.
// Null members in the bf16 instances.
struct Lo {
  const bf16* q;     // query lo, strides as the kernel's q
  const bf16* k;     // key lo, strides as the kernel's k
  const bf16* dout;  // dO lo, strides as the kernel's dout
  const bf16* kt;    // K^T lo, T-perm [bh][D][T]
  const float* v;    // fp32 V [B, H, T, D], strides vs (the chain's right-hand side)
  const float* o;    // fp32 O, strides as the kernel's o (delta of the backward)
  const float* dof;  // fp32 dO, strides as the kernel's dout (delta of the backward)
};

// bf16 of the residual x - hi for D-layout values e = 8h .. 8h+7 (hi = pack_b(x, h)):
// the lo term of a two-term bf16 split (x ~= hi + lo to ~2^-17 relative)
__device__ __forceinline__ bf16x8 pack_lo(const f32x16& x, int h, const bf16x8& hi) {
  bf16x8 r;
#pragma unroll
  for (int e = 0; e < 8; ++e) r[e] = (bf16)(x[8 * h + e] - (float)hi[e]);
  return r;
}

// X = P^-1 for a 64x64 lower-triangular fp32 block held in LDS (row-major,
// row stride 68).  Called by ONE wave: lane c solves column c by forward
// substitution, x_r = (delta_rc - sum_{k<r} P_rk x_k) / P_rr.  The diagonal of
// P is exp(s K^_r.K^_r - 1/s) in (0, 1], the off-diagonal entries lie in (0, 1],
// so plain substitution (no series) is used.  X overwrites P in LDS and is
// also written to gout[r*64 + c].
__device__ __forceinline__ void invert_lower64(float (*Ps)[68], int c, float* __restrict__ gout) {
  float x[64];
#pragma unroll
  for (int r = 0; r < 64; ++r) {
    float acc = (r == c) ? 1.f : 0.f;
#pragma unroll
    for (int kk = 0; kk < (r & ~3); kk += 4) {
      const f32x4 p = *reinterpret_cast<const f32x4*>(&Ps[r][kk]);
      acc = fmaf(-p[0], x[kk], acc);
      acc = fmaf(-p[1], x[kk + 1], acc);
      acc = fmaf(-p[2], x[kk + 2], acc);
      acc = fmaf(-p[3], x[kk + 3], acc);
    }
#pragma unroll
    for (int kk = (r & ~3); kk < r; ++kk) acc = fmaf(-Ps[r][kk], x[kk], acc);
    x[r] = acc / Ps[r][r];
  }
#pragma unroll
  for (int r = 0; r < 64; ++r) {
    Ps[r][c] = x[r];
    gout[r * 64 + c] = x[r];
  }
}

// 8 consecutive fp32 values -> bf16 hi + bf16 lo (x ~= hi + lo to ~2^-17 relative)
__device__ __forceinline__ void split8(const float* p, bf16x8& hi, bf16x8& lo) {
  const f32x4 a = *reinterpret_cast<const f32x4*>(p);
  const f32x4 b = *reinterpret_cast<const f32x4*>(p + 4);
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const bf16 ha = (bf16)a[e], hb = (bf16)b[e];
    hi[e] = ha;
    hi[e + 4] = hb;
    lo[e] = (bf16)(a[e] - (float)ha);
    lo[e + 4] = (bf16)(b[e] - (float)hb);
  }
}

// Per-row seed of an MFMA accumulator: mfma32(seed_a(x_m, g), seed_ones(g), 0) gives
// D[m][n] = x_m for every column n (m = the lane's row, lane % 32).  x is split into
// three bf16 terms at k = 0, 1, 2 (exact to ~2^-24 relative); the other k are zero.
__device__ __forceinline__ bf16x8 seed_a(float x, int g) {
  bf16x8 a;
#pragma unroll
  for (int e = 0; e < 8; ++e) a[e] = (bf16)0.f;
  if (g == 0) {
    const bf16 h = (bf16)x;
    const float r1 = x - (float)h;
    const bf16 m = (bf16)r1;
    a[0] = h;
    a[1] = m;
    a[2] = (bf16)(r1 - (float)m);
  }
  return a;
}
__device__ __forceinline__ bf16x8 seed_ones(int g) {
  bf16x8 b;
#pragma unroll
  for (int e = 0; e < 8; ++e) b[e] = (bf16)((g == 0 && e < 3) ? 1.f : 0.f);
  return b;
}

// one element of a T-perm matrix [bh][D][T]
__device__ __forceinline__ void vpth_w(bf16* base, int bh, int D, int T, int d, int slot, bf16 val) {
  base[((int64_t)bh * D + d) * T + slot] = val;
}

// Make this workgroup's global writes visible at agent scope, then advance the
// head's chain counter to val.  Every wave first waits until its own stores
// have reached the L2 (s_waitcnt 0), the barrier orders that before wave 0,
// whose agent-scope release writes the XCD's L2 back once for the whole
// workgroup before the counter store.  Every thread must call it.
__device__ __forceinline__ void publish_counter(int* cnt, int val) {
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x < 64) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    __builtin_amdgcn_s_waitcnt(0);  // the write-back has completed
    if (threadIdx.x == 0) __hip_atomic_store(cnt, val, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// 16 consecutive-in-D-layout fp32 values of a per-row vector: rows drow(e, g) + base
__device__ __forceinline__ void load_rows16(const float* __restrict__ p, int g, float out[16]) {
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const f32x4 t4 = *reinterpret_cast<const f32x4*>(p + 8 * q + 4 * g);
    out[4 * q] = t4[0];
    out[4 * q + 1] = t4[1];
    out[4 * q + 2] = t4[2];
    out[4 * q + 3] = t4[3];
  }
}

// ---------------------------------------------------------------------------
// Cooperative LDS staging of 64-wide tiles by a 256-thread workgroup with
// coalesced 16-byte global loads (D/32 chunks per thread per tile).
//   row tile:    [64 rows][D]   from rows j0.. of a [T][D]-strided source
//   T-perm tile: [D][64 slots]  from a [D][T] T-perm source (slots j0..)
// g2r_* loads into registers (issued early, overlapping compute), r2l_* stores
// the registers to LDS.
// ---------------------------------------------------------------------------
template <int D>
__device__ __forceinline__ void g2r_rows(const bf16* __restrict__ src, int64_t st, int j0, bf16x8* stg) {
#pragma unroll
  for (int u = 0; u < D / 32; ++u) {
    const int c = threadIdx.x + 256 * u;
    stg[u] = ld8(src + (int64_t)(j0 + c / (D / 8)) * st + (c % (D / 8)) * 8);
  }
}
template <int D>
__device__ __forceinline__ void r2l_rows(bf16 (*dst)[D + 8], const bf16x8* stg) {
#pragma unroll
  for (int u = 0; u < D / 32; ++u) {
    const int c = threadIdx.x + 256 * u;
    *reinterpret_cast<bf16x8*>(&dst[c / (D / 8)][(c % (D / 8)) * 8]) = stg[u];
  }
}
template <int D>
__device__ __forceinline__ void g2r_tp(const bf16* __restrict__ src, int T, int j0, bf16x8* stg) {
#pragma unroll
  for (int u = 0; u < D / 32; ++u) {
    const int c = threadIdx.x + 256 * u;
    stg[u] = ld8(src + (int64_t)(c >> 3) * T + j0 + (c & 7) * 8);
  }
}
template <int D>
__device__ __forceinline__ void r2l_tp(bf16 (*dst)[72], const bf16x8* stg) {
#pragma unroll
  for (int u = 0; u < D / 32; ++u) {
    const int c = threadIdx.x + 256 * u;
    *reinterpret_cast<bf16x8*>(&dst[c >> 3][(c & 7) * 8]) = stg[u];
  }
}
// 16 fp32 values of a staged per-row vector for D-layout rows base + drow(e, g)
__device__ __forceinline__ void lds_rows16(const float* p, int g, float out[16]) {
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const f32x4 t4 = *reinterpret_cast<const f32x4*>(p + 8 * q + 4 * g);
    out[4 * q] = t4[0];
    out[4 * q + 1] = t4[1];
    out[4 * q + 2] = t4[2];
    out[4 * q + 3] = t4[3];
  }
}

// Generalised staging: a [ROWS][D] row tile and a [D][SLOTS] T-perm tile.
template <int D, int ROWS>
__device__ __forceinline__ void g2r_rows_n(const bf16* __restrict__ src, int64_t st, int j0, bf16x8* stg) {
#pragma unroll
  for (int u = 0; u < ROWS * D / 2048; ++u) {
    const int c = threadIdx.x + 256 * u;
    stg[u] = ld8(src + (int64_t)(j0 + c / (D / 8)) * st + (c % (D / 8)) * 8);
  }
}
template <int D, int ROWS>
__device__ __forceinline__ void r2l_rows_n(bf16 (*dst)[D + 8], const bf16x8* stg) {
#pragma unroll
  for (int u = 0; u < ROWS * D / 2048; ++u) {
    const int c = threadIdx.x + 256 * u;
    *reinterpret_cast<bf16x8*>(&dst[c / (D / 8)][(c % (D / 8)) * 8]) = stg[u];
  }
}
template <int D, int SLOTS>
__device__ __forceinline__ void g2r_tp_n(const bf16* __restrict__ src, int T, int j0, bf16x8* stg) {
#pragma unroll
  for (int u = 0; u < D * SLOTS / 2048; ++u) {
    const int c = threadIdx.x + 256 * u;
    stg[u] = ld8(src + (int64_t)(c / (SLOTS / 8)) * T + j0 + (c % (SLOTS / 8)) * 8);
  }
}
template <int D, int SLOTS>
__device__ __forceinline__ void r2l_tp_n(bf16 (*dst)[SLOTS + 8], const bf16x8* stg) {
#pragma unroll
  for (int u = 0; u < D * SLOTS / 2048; ++u) {
    const int c = threadIdx.x + 256 * u;
    *reinterpret_cast<bf16x8*>(&dst[c / (SLOTS / 8)][(c % (SLOTS / 8)) * 8]) = stg[u];
  }
}

// ---------------------------------------------------------------------------
// Direct global -> LDS staging (gfx950 global_load_lds_dwordx4: every lane
// fetches 16 bytes from its own address and the 64 lanes of one instruction
// fill 1 KB of LDS contiguously from a wave-uniform base), so staged tiles
// cost no registers and no LDS store instructions.  Tiles are unpadded; the
// 16-byte chunk c of row r is stored at chunk c ^ (r & 7) of that row, so that
// 16-byte reads of one chunk by 8 consecutive rows hit distinct banks.
// All 256 threads call dma_tile; the data may be read after dma_wait() and a
// barrier.
// ---------------------------------------------------------------------------
template <int ROWS, int CPR>  // CPR: 16-byte chunks per row
__device__ __forceinline__ void dma_tile(const bf16* __restrict__ src, int64_t stride, bf16* lds) {
  constexpr int PER_WAVE = ROWS * CPR / 256;
  static_assert(PER_WAVE * 256 == ROWS * CPR, "tile must be a whole number of 1 KB pieces per wave");
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
#pragma unroll
  for (int i = 0; i < PER_WAVE; ++i) {
    const int q = (w * PER_WAVE + i) * 64 + lane;
    const int r = q / CPR, c = (q % CPR) ^ (r & 7);
    __builtin_amdgcn_global_load_lds(src + (int64_t)r * stride + c * 8, lds + (w * PER_WAVE + i) * 512, 16, 0, 0);
  }
}
// dma_tile split in two: the per-lane element offsets for a fixed row stride
// (dma_plan, once per kernel) and the loads of one tile (dma_stage), by a workgroup of
// NTHR threads.
// Swizzle key of row r: chunk c of row r is stored at chunk c ^ swz_key<SW>(r).
//   SW = 0: r & 7.  With 128-byte rows, rows r and r + 8 of one 16-lane pass of 16-byte
//     reads land on the same banks (2-way), as do rows r and r + 2 of a transposing read.
//   SW = 1: bitrev3((r >> 1) & 7), conflict-free for both reads of 128-byte rows; rows r and
//     r + 8 then differ in the key, so a transposing read needs a second lane offset.
template <int SW>
__device__ __forceinline__ int swz_key(int r) {
  if constexpr (SW == 0) {
    return r & 7;
  } else {
    const int x = (r >> 1) & 7;
    return ((x & 1) << 2) | (x & 2) | (x >> 2);
  }
}
template <int ROWS, int CPR, int NTHR = 256, int SW = 0>
__device__ __forceinline__ void dma_plan(int64_t stride, int* off) {
  constexpr int PER_WAVE = ROWS * CPR / NTHR;
  static_assert(PER_WAVE * NTHR == ROWS * CPR, "tile must be a whole number of 1 KB pieces per wave");
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
#pragma unroll
  for (int i = 0; i < PER_WAVE; ++i) {
    const int q = (w * PER_WAVE + i) * 64 + lane;
    const int r = q / CPR, c = (q % CPR) ^ swz_key<SW>(r);
    off[i] = (int)(r * stride) + c * 8;
  }
}
template <int ROWS, int CPR, int NTHR = 256>
__device__ __forceinline__ void dma_stage(const int* off, const bf16* __restrict__ src, bf16* lds) {
  constexpr int PER_WAVE = ROWS * CPR / NTHR;
  const int w = threadIdx.x >> 6;
#pragma unroll
  for (int i = 0; i < PER_WAVE; ++i)
    __builtin_amdgcn_global_load_lds(src + off[i], lds + (w * PER_WAVE + i) * 512, 16, 0, 0);
}
// 64 consecutive fp32 values into LDS by one wave (call from a single wave)
__device__ __forceinline__ void dma_f32x64(const float* __restrict__ src, float* lds) {
  __builtin_amdgcn_global_load_lds(src + (threadIdx.x & 63), lds, 4, 0, 0);
}
// 1 KB (512 consecutive bf16) into LDS by one wave (call from a single wave)
__device__ __forceinline__ void dma_1k(const bf16* __restrict__ src, bf16* lds) {
  __builtin_amdgcn_global_load_lds(src + 8 * (threadIdx.x & 63), lds, 16, 0, 0);
}
// Wait until this wave's staging loads have landed in LDS.
__device__ __forceinline__ void dma_wait() { __builtin_amdgcn_s_waitcnt(0); }
// Wait until at most N of this wave's vector memory operations are outstanding
// (the newest N may still be in flight; s_waitcnt vmcnt(N), gfx9 encoding).
template <int N>
__device__ __forceinline__ void dma_wait_but() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}
// Element offset of logical chunk c (8 bf16) of row r in a swizzled tile with CPR
// chunks per row, and its address.
template <int CPR, int SW = 0>
__device__ __forceinline__ int swz_off(int r, int c) {
  return r * (CPR * 8) + ((c ^ swz_key<SW>(r)) << 3);
}
template <int CPR, int SW = 0>
__device__ __forceinline__ const bf16* swz(const bf16* tile, int r, int c) {
  return tile + swz_off<CPR, SW>(r, c);
}

// MFMA A operand [m = col0 + lane%32][k = 16 rows from row0] read from a
// swizzled row-major LDS tile (CPR 16-byte chunks per row) with two gfx950
// transposing loads (ds_read_b64_tr_b16).  In each group of 16 lanes, source
// lane s addresses 4 consecutive elements of row row0 + 4g + s/4 (+8 for the
// second load) at column col0 + 16*((lane>>4)&1) + 4*(s&3); result lane j then
// receives element j%4 of source lanes 4e + j/4, e = 0..3 (checked on an
// MI355X), i.e. column col0 + lane%32 of rows row0 + 4g + e (+8).  Operand
// slot 8g + e therefore holds row jmap(8g + e) -- the order in which the D
// layout of a score tile delivers its keys -- so the result pairs with
// pack_b() exactly like a 16-byte read from a T-perm tile.
template <int CPR, int SW = 0>
__device__ __forceinline__ bf16x8 lds_tr_a(const bf16* tile, int row0, int col0) {
  typedef __attribute__((address_space(3))) bf16x4 lds_bf16x4;
  const int lane = threadIdx.x & 63, s = lane & 15;
  const int col = col0 + 16 * ((lane >> 4) & 1) + 4 * (s & 3);
  const int r1 = row0 + 4 * (lane >> 5) + (s >> 2);
  // (with SW = 0 rows r1 and r1 + 8 share the swizzle key)
  const int off1 = (((col >> 3) ^ swz_key<SW>(r1)) << 3) | (col & 7);
  const int off2 = (((col >> 3) ^ swz_key<SW>(r1 + 8)) << 3) | (col & 7);
  const bf16x4 v1 = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(tile + r1 * (CPR * 8) + off1));
  const bf16x4 v2 = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(tile + (r1 + 8) * (CPR * 8) + off2));
  return bf16x8{v1[0], v1[1], v1[2], v1[3], v2[0], v2[1], v2[2], v2[3]};
}

// lds_tr_a split into its lane part (once per kernel) and its tile part: the lane
// offset (elements) of the transposing read for column block col0 (a multiple of 32)
// at row0 = 0; rows row0 (a multiple of 16) then add row0 * CPR * 8, a constant that
// the compiler folds into the instruction's offset field.
template <int CPR>
__device__ __forceinline__ int lds_tr_lane_off(int col0) {
  const int lane = threadIdx.x & 63, s = lane & 15;
  const int col = col0 + 16 * ((lane >> 4) & 1) + 4 * (s & 3);
  const int r1 = 4 * (lane >> 5) + (s >> 2);
  return r1 * (CPR * 8) + ((((col >> 3) ^ (r1 & 7)) << 3) | (col & 7));
}
// The same for a tile with swizzle SW: the lane offsets of the two loads (rows r1 and
// r1 + 8, whose keys differ for SW = 1); rows row0 (a multiple of 16) add row0 * CPR * 8.
template <int CPR, int SW>
__device__ __forceinline__ void lds_tr_lane_offs(int col0, int& o1, int& o2) {
  const int lane = threadIdx.x & 63, s = lane & 15;
  const int col = col0 + 16 * ((lane >> 4) & 1) + 4 * (s & 3);
  const int r1 = 4 * (lane >> 5) + (s >> 2);
  o1 = r1 * (CPR * 8) + ((((col >> 3) ^ swz_key<SW>(r1)) << 3) | (col & 7));
  o2 = (r1 + 8) * (CPR * 8) + ((((col >> 3) ^ swz_key<SW>(r1 + 8)) << 3) | (col & 7));
}
template <int CPR>
__device__ __forceinline__ bf16x8 lds_tr_a_at2(const bf16* tile, int o1, int o2, int row0) {
  typedef __attribute__((address_space(3))) bf16x4 lds_bf16x4;
  const bf16x4 v1 = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(tile + o1 + row0 * (CPR * 8)));
  const bf16x4 v2 = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(tile + o2 + row0 * (CPR * 8)));
  return bf16x8{v1[0], v1[1], v1[2], v1[3], v2[0], v2[1], v2[2], v2[3]};
}
template <int CPR>
__device__ __forceinline__ bf16x8 lds_tr_a_at(const bf16* tile_lane, int row0) {
  typedef __attribute__((address_space(3))) bf16x4 lds_bf16x4;
  const bf16x4 v1 = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(tile_lane + row0 * (CPR * 8)));
  const bf16x4 v2 = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(tile_lane + (row0 + 8) * (CPR * 8)));
  return bf16x8{v1[0], v1[1], v1[2], v1[3], v2[0], v2[1], v2[2], v2[3]};
}

}  // namespace lucid
