// Shared helpers of the LUCID-Path kernels (head dim K = V = 64 or 128, small chunk 64,
// large chunk PR = 16 small chunks = 1024 positions).
//
// fp32 inputs (template flag F32): the caller's tensors are fp32, and every bf16 MFMA
// operand buffer of the workspace holds two bf16 planes, hi = bf16(x) and lo = bf16(x - hi),
// the lo plane at a fixed element offset from the hi plane (PathFwdWs / PathBwdWs lo_*).
// Each product then takes hi.hi + hi.lo + lo.hi (~fp32 accuracy, mm3 below).
#pragma once
#include <type_traits>
#include "lucid_common.h"

namespace lucid {

constexpr int PC = 64;  // small chunk (positions)
constexpr int PR = 16;  // small chunks per large chunk (S = 1024 positions)

// element type of the caller's tensors
template <bool F32>
using pin_t = std::conditional_t<F32, float, bf16>;

// acc + a b over the NP planes of each operand: a[0] b[0] (NP = 1), or the 3-term split
// a[0] b[0] + a[0] b[1] + a[1] b[0] (NP = 2)
template <int NP>
__device__ __forceinline__ f32x16 mm3(const bf16x8* a, const bf16x8* b, f32x16 acc) {
  acc = mfma32(a[0], b[0], acc);
  if constexpr (NP == 2) {
    acc = mfma32(a[0], b[1], acc);
    acc = mfma32(a[1], b[0], acc);
  }
  return acc;
}

// x as bf16 into hi[i], and (NP = 2) its residual into hi[i + lo]
template <int NP>
__device__ __forceinline__ void put_split(bf16* hi, int64_t lo, int64_t i, float x) {
  const bf16 h = (bf16)x;
  hi[i] = h;
  if constexpr (NP == 2) hi[i + lo] = (bf16)(x - (float)h);
}

// acc[i][j] += sum_k opA(A)[r0+i][k] * opB(B)[k][c0+j] for 64x64 fp32 LDS matrices
// (row stride 68); thread t owns the 4x4 block r0 = 4*(t/16), c0 = 4*(t%16).
// Four k-steps per iteration: every operand is read as 16-byte vectors (along k for
// the row-indexed operands, along the block for the others), 8 reads per 64 FMAs.
template <bool TA, bool TB>
__device__ __forceinline__ void lds_gemm64(const float (*A)[68], const float (*B)[68], float acc[4][4]) {
  const int tid = threadIdx.x;
  const int r0 = (tid >> 4) * 4, c0 = (tid & 15) * 4;
#pragma unroll 2
  for (int k = 0; k < 64; k += 4) {
    float a[4][4], b[4][4];  // a[kk][i] = opA[r0+i][k+kk], b[kk][j] = opB[k+kk][c0+j]
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      if (TA) {
        const f32x4 t4 = *reinterpret_cast<const f32x4*>(&A[k + q][r0]);
#pragma unroll
        for (int i = 0; i < 4; ++i) a[q][i] = t4[i];
      } else {
        const f32x4 t4 = *reinterpret_cast<const f32x4*>(&A[r0 + q][k]);
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) a[kk][q] = t4[kk];
      }
      if (TB) {
        const f32x4 t4 = *reinterpret_cast<const f32x4*>(&B[c0 + q][k]);
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) b[kk][q] = t4[kk];
      } else {
        const f32x4 t4 = *reinterpret_cast<const f32x4*>(&B[k + q][c0]);
#pragma unroll
        for (int j = 0; j < 4; ++j) b[q][j] = t4[j];
      }
    }
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(a[kk][i], b[kk][j], acc[i][j]);
  }
}

__device__ __forceinline__ void zero44(float acc[4][4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = 0.f;
}

// One merge of two inverted s x s diagonal blocks A = [a, a+s), B = [a+s, a+2s) of a
// unit lower matrix (I + N): X_BA = -X_B (N_BA X_A), computed in place in the N_BA block
// in two products; each thread owns 4 consecutive columns of one row of a pair.
template <int S>
__device__ __forceinline__ void merge_lower_blocks(float (*M)[68]) {
  constexpr int QPP = S * S / 4;         // column quads per pair
  constexpr int NQ = (64 / (2 * S)) * QPP;  // quads of all pairs
  const int qd = threadIdx.x;
  const bool act = qd < NQ;
  const int p = qd / QPP, rem = qd - p * QPP;
  const int i = rem / (S / 4), j0 = 4 * (rem - i * (S / 4));
  const int ao = 2 * p * S, bo = ao + S;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  if (act) {  // Y = N_BA X_A
#pragma unroll
    for (int kk = 0; kk < S; ++kk) {
      const float a = M[bo + i][ao + kk];
      const f32x4 x = *reinterpret_cast<const f32x4*>(&M[ao + kk][ao + j0]);
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[e] = fmaf(a, x[e], acc[e]);
    }
  }
  __syncthreads();
  if (act) *reinterpret_cast<f32x4*>(&M[bo + i][ao + j0]) = acc;
  __syncthreads();
  if (act) {  // X_BA = -X_B Y
    acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < S; ++kk) {
      const float a = M[bo + i][bo + kk];
      const f32x4 y = *reinterpret_cast<const f32x4*>(&M[bo + kk][ao + j0]);
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[e] = fmaf(a, y[e], acc[e]);
    }
  }
  __syncthreads();
  if (act) *reinterpret_cast<f32x4*>(&M[bo + i][ao + j0]) = -acc;
  __syncthreads();
}

// (I + M)^-1 in place for a strictly lower 64x64 fp32 LDS matrix M (its diagonal and
// strictly upper part must hold zeros; the result has a unit diagonal and zeros above).
// Called by all 256 threads of the block; the caller syncs before, the function syncs
// before returning.  Wave w inverts the 16x16 diagonal block w by forward substitution
// (lane c < 16 solves column c: x_r = delta_rc - sum_{k<r} M_rk x_k); the blocks are
// then merged 16 -> 32 -> 64 through X_BA = -X_B N_BA X_A.  A 64-deep solve in one
// wave has four times the dependent work and leaves three waves idle.
__device__ __forceinline__ void invert_unit_lower64(float (*M)[68]) {
  const int w = threadIdx.x >> 6, c = threadIdx.x & 63;
  if (c < 16) {
    const int o = 16 * w;
    float x[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      float a0 = (r == c) ? 1.f : 0.f, a1 = 0.f;
#pragma unroll
      for (int kk = 0; kk < (r & ~3); kk += 4) {
        const f32x4 m4 = *reinterpret_cast<const f32x4*>(&M[o + r][o + kk]);
        a0 = fmaf(-m4[0], x[kk], a0);
        a1 = fmaf(-m4[1], x[kk + 1], a1);
        a0 = fmaf(-m4[2], x[kk + 2], a0);
        a1 = fmaf(-m4[3], x[kk + 3], a1);
      }
#pragma unroll
      for (int kk = (r & ~3); kk < r; ++kk) a0 = fmaf(-M[o + r][o + kk], x[kk], a0);
      x[r] = a0 + a1;
    }
    // only this wave reads its diagonal block, so it may write it back right away
#pragma unroll
    for (int r = 0; r < 16; ++r) M[o + r][o + c] = x[r];
  }
  __syncthreads();
  merge_lower_blocks<16>(M);
  merge_lower_blocks<32>(M);
}

// Load a 64x64 block of fp32 rows (row stride st elements) into an fp32 LDS matrix.
__device__ __forceinline__ void load_rows64_f32(float (*dst)[68], const float* __restrict__ src, int64_t st) {
  const int tid = threadIdx.x;
  const int r = tid >> 2, c = (tid & 3) * 16;
#pragma unroll
  for (int q4 = 0; q4 < 4; ++q4)
    *reinterpret_cast<f32x4*>(&dst[r][c + 4 * q4]) = *reinterpret_cast<const f32x4*>(src + (int64_t)r * st + c + 4 * q4);
}
// The same from bf16 hi / lo planes (lo = element offset of the lo plane; 0: none).
__device__ __forceinline__ void load_rows64_split(float (*dst)[68], const bf16* __restrict__ src, int64_t st,
                                                  int64_t lo) {
  const int tid = threadIdx.x;
  const int r = tid >> 2, c = (tid & 3) * 16;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const bf16x8 x = ld8(src + (int64_t)r * st + c + 8 * h);
    bf16x8 y{};
    if (lo) y = ld8(src + lo + (int64_t)r * st + c + 8 * h);
#pragma unroll
    for (int e = 0; e < 8; ++e) dst[r][c + 8 * h + e] = (float)x[e] + (lo ? (float)y[e] : 0.f);
  }
}
// Load a 64x64 block of bf16 rows (row stride st elements) into an fp32 LDS matrix.
__device__ __forceinline__ void load_rows64_f32(float (*dst)[68], const bf16* __restrict__ src, int64_t st) {
  const int tid = threadIdx.x;
  const int r = tid >> 2, c = (tid & 3) * 16;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const bf16x8 x = ld8(src + (int64_t)r * st + c + 8 * h);
#pragma unroll
    for (int e = 0; e < 8; ++e) dst[r][c + 8 * h + e] = (float)x[e];
  }
}

// Load a 64x64 fp32 row-major matrix (contiguous) into LDS, optionally transposed.
template <bool TRANS>
__device__ __forceinline__ void load_mat64(float (*dst)[68], const float* __restrict__ src) {
  for (int idx = threadIdx.x; idx < 4096; idx += 256) {
    const int r = idx >> 6, c = idx & 63;
    if (TRANS)
      dst[c][r] = src[idx];
    else
      dst[r][c] = src[idx];
  }
}

// x <- x M for x [64 rows][64] in LDS (fp32) and M^T in LDS (MT[n][k] = M[k][n]),
// computed as D^T = M^T x^T with a 3-term bf16 split (~fp32 accuracy).  Each of the
// four waves produces one 32x32 tile; returns it in D layout (m = column n of the
// product, lane <-> row) through `o`; the caller syncs before writing it back.
__device__ __forceinline__ f32x16 mat_xM_tile(const float (*X)[68], const float (*MT)[68], int dt, int rt) {
  const int lane = threadIdx.x & 63, g = lane >> 5, l32 = lane & 31;
  f32x16 o = zero16();
#pragma unroll
  for (int st = 0; st < 4; ++st) {
    bf16x8 ah, al, bh8, bl;
    split8(&MT[dt * 32 + l32][16 * st + 8 * g], ah, al);
    split8(&X[rt * 32 + l32][16 * st + 8 * g], bh8, bl);
    o = mfma32(ah, bh8, o);
    o = mfma32(ah, bl, o);
    o = mfma32(al, bh8, o);
  }
  return o;
}

// ---------------------------------------------------------------------------
// 64x64 fp32 LDS matrix products on the matrix cores.  Wave w owns the 32x32 output
// tile (tm = w >> 1, tn = w & 1) in MFMA D layout: element e of lane l is
// C[32 tm + drow(e, l / 32)][32 tn + l % 32] (dl_row / dl_col below).
// acc += opA(A) opB(B) with a 3-term bf16 split (hi.hi + hi.lo + lo.hi, ~fp32
// accuracy); operands are read along k as 16-byte vectors where the layout allows
// (A not transposed, B transposed) and gathered otherwise.
// ---------------------------------------------------------------------------
__device__ __forceinline__ int dl_row(int e) {
  return 32 * ((int)threadIdx.x >> 7) + drow(e, ((int)threadIdx.x >> 5) & 1);
}
__device__ __forceinline__ int dl_col() { return 32 * (((int)threadIdx.x >> 6) & 1) + ((int)threadIdx.x & 31); }

__device__ __forceinline__ void split_vals(const float v[8], bf16x8& hi, bf16x8& lo) {
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const bf16 h = (bf16)v[e];
    hi[e] = h;
    lo[e] = (bf16)(v[e] - (float)h);
  }
}

template <bool TA, bool TB>
__device__ __forceinline__ f32x16 mgemm64(const float (*A)[68], const float (*B)[68], f32x16 acc) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, g = lane >> 5, l32 = lane & 31;
  const int m = 32 * (w >> 1) + l32, n = 32 * (w & 1) + l32;
#pragma unroll
  for (int st = 0; st < 4; ++st) {
    const int k0 = 16 * st + 8 * g;
    float a[8], b[8];
    if (TA) {
#pragma unroll
      for (int i = 0; i < 8; ++i) a[i] = A[k0 + i][m];
    } else {
      const f32x4 x = *reinterpret_cast<const f32x4*>(&A[m][k0]);
      const f32x4 y = *reinterpret_cast<const f32x4*>(&A[m][k0 + 4]);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        a[i] = x[i];
        a[4 + i] = y[i];
      }
    }
    if (TB) {
      const f32x4 x = *reinterpret_cast<const f32x4*>(&B[n][k0]);
      const f32x4 y = *reinterpret_cast<const f32x4*>(&B[n][k0 + 4]);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        b[i] = x[i];
        b[4 + i] = y[i];
      }
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) b[i] = B[k0 + i][n];
    }
    bf16x8 ah, al, bh, bl;
    split_vals(a, ah, al);
    split_vals(b, bh, bl);
    acc = mfma32(ah, bh, acc);
    acc = mfma32(ah, bl, acc);
    acc = mfma32(al, bh, acc);
  }
  return acc;
}

// D-layout tile helpers for mgemm64 results: S[row][col] <- x (masked), x <- S[row][col]
#define DL_FOR_E _Pragma("unroll") for (int e = 0; e < 16; ++e)
__device__ __forceinline__ void dl_store(float (*S)[68], const f32x16& x, int mode) {
  // mode 0: all, 1: col <= row (tril), 2: col < row (strictly lower)
  const int cl = dl_col();
  DL_FOR_E {
    const int r = dl_row(e);
    const bool keep = mode == 0 || (mode == 1 ? cl <= r : cl < r);
    S[r][cl] = keep ? x[e] : 0.f;
  }
}
__device__ __forceinline__ f32x16 dl_load(const float (*S)[68]) {
  const int cl = dl_col();
  f32x16 x;
  DL_FOR_E x[e] = S[dl_row(e)][cl];
  return x;
}
// 64 x 64 block of an fp32 row-major matrix (row stride ld) into an LDS block, and back
__device__ __forceinline__ void load_blk(float (*dst)[68], const float* __restrict__ src, int ld) {
  for (int idx = threadIdx.x; idx < 1024; idx += 256) {
    const int r = idx >> 4, c4 = (idx & 15) * 4;
    *reinterpret_cast<f32x4*>(&dst[r][c4]) = *reinterpret_cast<const f32x4*>(src + (int64_t)r * ld + c4);
  }
}
__device__ __forceinline__ void store_blk(float* __restrict__ dst, int ld, const float (*src)[68]) {
  for (int idx = threadIdx.x; idx < 1024; idx += 256) {
    const int r = idx >> 4, c4 = (idx & 15) * 4;
    *reinterpret_cast<f32x4*>(dst + (int64_t)r * ld + c4) = *reinterpret_cast<const f32x4*>(&src[r][c4]);
  }
}
// D-layout tile (this wave's 32 x 32 of a 64 x 64 block) to a row-major fp32 / bf16 matrix
__device__ __forceinline__ void dl_put(float* __restrict__ dst, int ld, const f32x16& x) {
  const int cl = dl_col();
  DL_FOR_E dst[(int64_t)dl_row(e) * ld + cl] = x[e];
}

// 64x64 fp32 row-major matrix: thread t holds rows (t + 256 i) / 16, 4 columns each
__device__ __forceinline__ void mat_fetch(f32x4 v[4], const float* __restrict__ src) {
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = *reinterpret_cast<const f32x4*>(src + 4 * (threadIdx.x + 256 * i));
}
__device__ __forceinline__ void mat_put(float (*S)[68], const f32x4 v[4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int f = 4 * (threadIdx.x + 256 * i);
    *reinterpret_cast<f32x4*>(&S[f >> 6][f & 63]) = v[i];
  }
}
__device__ __forceinline__ f32x16 dl_neg(f32x16 x) {
  DL_FOR_E x[e] = -x[e];
  return x;
}


}  // namespace lucid
