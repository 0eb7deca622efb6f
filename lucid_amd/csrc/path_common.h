// Shared helpers of the LUCID-Path kernels (head_dim K = V = 64, small chunk 64,
// large chunk 8 small chunks = 512 positions).
#pragma once
#include "lucid_common.h"

namespace lucid {

constexpr int PC = 64;  // small chunk (positions)
constexpr int PR = 8;   // small chunks per large chunk

// acc[i][j] += sum_k opA(A)[r0+i][k] * opB(B)[k][c0+j] for 64x64 fp32 LDS matrices
// (row stride 68); thread t owns the 4x4 block r0 = 4*(t/16), c0 = 4*(t%16).
template <bool TA, bool TB>
__device__ __forceinline__ void lds_gemm64(const float (*A)[68], const float (*B)[68], float acc[4][4]) {
  const int tid = threadIdx.x;
  const int r0 = (tid >> 4) * 4, c0 = (tid & 15) * 4;
#pragma unroll 4
  for (int k = 0; k < 64; ++k) {
    float a[4], b[4];
    if (TA) {
      const f32x4 t4 = *reinterpret_cast<const f32x4*>(&A[k][r0]);
      a[0] = t4[0]; a[1] = t4[1]; a[2] = t4[2]; a[3] = t4[3];
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = A[r0 + i][k];
    }
    if (TB) {
#pragma unroll
      for (int j = 0; j < 4; ++j) b[j] = B[c0 + j][k];
    } else {
      const f32x4 t4 = *reinterpret_cast<const f32x4*>(&B[k][c0]);
      b[0] = t4[0]; b[1] = t4[1]; b[2] = t4[2]; b[3] = t4[3];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(a[i], b[j], acc[i][j]);
  }
}

__device__ __forceinline__ void zero44(float acc[4][4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = 0.f;
}

// (I + M)^-1 in place for the strictly lower part of a 64x64 fp32 LDS matrix (the
// diagonal and upper part of M are ignored).  Called by ONE wave: lane c solves
// column c by forward substitution x_r = delta_rc - sum_{k<r} M_rk x_k.
__device__ __forceinline__ void invert_unit_lower64(float (*M)[68], int c) {
  float x[64];
#pragma unroll
  for (int r = 0; r < 64; ++r) {
    float acc = (r == c) ? 1.f : 0.f;
#pragma unroll
    for (int kk = 0; kk < (r & ~3); kk += 4) {
      const f32x4 p = *reinterpret_cast<const f32x4*>(&M[r][kk]);
      acc = fmaf(-p[0], x[kk], acc);
      acc = fmaf(-p[1], x[kk + 1], acc);
      acc = fmaf(-p[2], x[kk + 2], acc);
      acc = fmaf(-p[3], x[kk + 3], acc);
    }
#pragma unroll
    for (int kk = (r & ~3); kk < r; ++kk) acc = fmaf(-M[r][kk], x[kk], acc);
    x[r] = acc;
  }
#pragma unroll
  for (int r = 0; r < 64; ++r) M[r][c] = x[r];
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

}  // namespace lucid
