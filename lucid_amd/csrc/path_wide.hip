// LUCID-Path (and PaTH softmax) at head dim 128: the stages whose operands are 64 x K or
// K x K fp32 matrices (the WY form of a chunk, the Householder products of a large chunk,
// the query transport, the decode key cache, and their backward), with every 128-wide
// matrix held as 64 x 64 fp32 LDS blocks and every product taken block by block on the
// matrix cores (mgemm64: 3-term bf16 split, ~fp32 accuracy).  The algebra is that of the
// head-dim-64 kernels in path_fwd.hip / path_bwd.hip (reference parallel.py:27-177,
// cumprod_householder_fwd.py:13-79, transform_q.py:15-61, prepare_k_cache.py:12-74,
// cumprod_householder_bwd.py:13-95, intra_chunk_preprocess_bwd.py:14-110); only the
// staging differs, so that the operands fit the 160 KB of LDS.
//
// Workspace layouts at K = V = 128 (PathFwdWs / PathBwdWs): rows [..][T][128], K x K
// matrices row-major [..][128 * 128], in-chunk C x C matrices [..][64 * 64] as at 64.
#pragma once
#include "path_common.h"
#include "path_bwd.hip"  // PathBwdWs (path_bwd.hip has no include guard: included here only)

namespace lucid {

constexpr int WK = 128;  // head dim of this file's kernels

// ---------------------------------------------------------------------------
// WY form and in-chunk transforms at K = 128 (path_chunk_kernel's algebra).  grid (NT, B*HQ)
//   phase 1 (K halves h = 0, 1 accumulated): a = Wb W^T, WBK = Wb K^T, QW = Q W^T, QK = Q K^T
//   Tm = (I + stril a)^-1, TW = Tm stril(WBK), A_diag = tril(QK - tril(QW) TW), L_diag, Y
//   phase 2: Tmb = Tm diag(beta); W2_h = Tmb W_h; k~_h = K_h - TW^T W_h; q~_h = Q_h - QW W2_h;
//   Hc blocks (a, b) = delta_ab I - W_a^T W2_b
// LDS: seven 64 x 64 fp32 blocks.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void path_chunk128_kernel(const bf16* __restrict__ q, Strides qs,
                                                            const bf16* __restrict__ k, Strides ks,
                                                            const bf16* __restrict__ w, Strides wst,
                                                            const bf16* __restrict__ beta, Strides bst, int HQ, int H,
                                                            int T, float scale, int softmax, PathFwdWs ws) {
  __shared__ __attribute__((aligned(16))) float Bm[7][64][68];
  __shared__ float bsh[64];
  const int c = blockIdx.x, bhq = blockIdx.y;
  const int NT = T / PC;
  const int G = HQ / H;
  const int b = bhq / HQ, hq = bhq - b * HQ, h = hq / G;
  const int bh = b * H + h;
  const bool kvw = (hq % G) == 0;
  const int tid = threadIdx.x;
  const int t0 = c * PC;
  const f32x16 z = zero16();
  const int cl = dl_col();
  if (c == 0 && tid == 0) ws.counters[bhq] = 0;
  const bf16* wp = w + b * wst.b + h * wst.h + (int64_t)t0 * wst.t;
  const bf16* qp = q + b * qs.b + hq * qs.h + (int64_t)t0 * qs.t;
  const bf16* kp = k + b * ks.b + h * ks.h + (int64_t)t0 * ks.t;
  if (tid < 64) bsh[tid] = (float)beta[b * bst.b + h * bst.h + (int64_t)(t0 + tid) * bst.t];
  f32x16 aA = z, aWBK = z, aQW = z, aQK = z;
#pragma unroll 1
  for (int hh = 0; hh < 2; ++hh) {
    load_rows64_f32(Bm[0], wp + 64 * hh, wst.t);
    load_rows64_f32(Bm[1], qp + 64 * hh, qs.t);
    load_rows64_f32(Bm[2], kp + 64 * hh, ks.t);
    __syncthreads();
    {
      const int r = tid >> 2, cc = (tid & 3) * 16;
#pragma unroll
      for (int e = 0; e < 16; ++e) Bm[3][r][cc + e] = bsh[r] * Bm[0][r][cc + e];
    }
    __syncthreads();
    aA = mgemm64<false, true>(Bm[3], Bm[0], aA);
    aWBK = mgemm64<false, true>(Bm[3], Bm[2], aWBK);
    aQW = mgemm64<false, true>(Bm[1], Bm[0], aQW);
    aQK = mgemm64<false, true>(Bm[1], Bm[2], aQK);
    __syncthreads();
  }
  float(*Tm)[68] = Bm[4];
  float(*QW)[68] = Bm[5];
  float(*TW)[68] = Bm[6];
  dl_store(Tm, aA, 2);
  dl_store(QW, aWBK, 2);  // stril(WBK), until TW is formed
  __syncthreads();
  invert_unit_lower64(Tm);
  dl_store(TW, mgemm64<false, false>(Tm, QW, z), 0);
  __syncthreads();
  dl_store(QW, aQW, 1);  // tril(Q W^T)
  __syncthreads();
  {
    const f32x16 qt_ = mgemm64<false, false>(QW, TW, z);
    float* dst = ws.ld + ((int64_t)bhq * NT + c) * 4096;
    if (softmax) {
      DL_FOR_E {
        const int r = dl_row(e);
        dst[r * 64 + cl] = cl <= r ? aQK[e] - qt_[e] : 0.f;
      }
    } else {
      const float sl2 = scale * LOG2E_F, cc0 = LOG2E_F / scale;
      DL_FOR_E {
        const int r = dl_row(e);
        const float v = cl < r ? __builtin_amdgcn_exp2f(fmaf(aQK[e] - qt_[e], sl2, -cc0)) : 0.f;
        Bm[0][r][cl] = v;
        dst[r * 64 + cl] = v;
      }
      __syncthreads();
      invert_unit_lower64(Bm[0]);
      store_blk(ws.y + ((int64_t)bhq * NT + c) * 4096, 64, Bm[0]);
    }
  }
  __syncthreads();
  // Tmb = Tm diag(beta) in place (Tm is read only by the W2 products from here on)
  for (int idx = tid; idx < 4096; idx += 256) Tm[idx >> 6][idx & 63] *= bsh[idx & 63];
  load_rows64_f32(Bm[1], wp, wst.t);
  load_rows64_f32(Bm[2], wp + 64, wst.t);
  __syncthreads();
  const f32x16 w2a = mgemm64<false, false>(Tm, Bm[1], z), w2b = mgemm64<false, false>(Tm, Bm[2], z);
  dl_store(Bm[0], w2a, 0);
  dl_store(Bm[3], w2b, 0);
  if (kvw) {
    float* dst = ws.w2 + ((int64_t)bh * T + t0) * WK;
    dl_put(dst, WK, w2a);
    dl_put(dst + 64, WK, w2b);
  }
  __syncthreads();
#pragma unroll 1
  for (int hh = 0; hh < 2; ++hh) {
    float(*Wh)[68] = Bm[1 + hh];
    float(*W2h)[68] = hh ? Bm[3] : Bm[0];
    if (kvw) {  // k~_h = K_h - TW^T W_h
      const f32x16 a = mgemm64<true, false>(TW, Wh, z);
      bf16* dst = ws.kt + ((int64_t)bh * T + t0) * WK + 64 * hh;
      DL_FOR_E {
        const int r = dl_row(e);
        dst[r * WK + cl] = (bf16)((float)kp[(int64_t)r * ks.t + 64 * hh + cl] - a[e]);
      }
    }
    {  // q~_h = Q_h - QW W2_h
      const f32x16 a = mgemm64<false, false>(QW, W2h, z);
      float* dst = ws.qt + ((int64_t)bhq * T + t0) * WK + 64 * hh;
      DL_FOR_E {
        const int r = dl_row(e);
        dst[r * WK + cl] = (float)qp[(int64_t)r * qs.t + 64 * hh + cl] - a[e];
      }
    }
  }
  if (kvw) {  // Hc = I - W^T W2, block (ra, cb_)
    float* dst = ws.hc + ((int64_t)bh * NT + c) * (WK * WK);
    bf16* dsts = ws.hcs + ((int64_t)bh * NT + c) * (2 * WK * WK);
#pragma unroll 1
    for (int blk = 0; blk < 4; ++blk) {
      const int ra = blk >> 1, cb_ = blk & 1;
      const f32x16 a = mgemm64<true, false>(Bm[1 + ra], cb_ ? Bm[3] : Bm[0], z);
      DL_FOR_E {
        const int r = dl_row(e);
        const int i = (64 * ra + r) * WK + 64 * cb_ + cl;
        const float x = (ra == cb_ && r == cl ? 1.f : 0.f) - a[e];
        dst[i] = x;
        put_split<2>(dsts, WK * WK, i, x);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Per large chunk at K = 128 (path_large_kernel's algebra): SUF_c from the top down,
// KL_c = k~_c SUF_c^T, SUF_{c-1} = SUF_c Hc_c, HL = the last.  grid (NS, B*H)
// LDS: SUF as four blocks, and four operand blocks holding k~_c, then Hc_c.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void path_large128_kernel(int T, PathFwdWs ws) {
  __shared__ __attribute__((aligned(16))) float Sf[4][64][68];  // block (r, c) at 2 r + c
  __shared__ __attribute__((aligned(16))) float Op[4][64][68];
  const int s = blockIdx.x, bh = blockIdx.y;
  const int NT = T / PC, NS = (NT + PR - 1) / PR;
  const int tid = threadIdx.x;
  const int cb = s * PR, ce = min(cb + PR, NT) - 1;
  const f32x16 z = zero16();
  for (int idx = tid; idx < 4 * 4096; idx += 256) {
    const int blk = idx >> 12, r = (idx >> 6) & 63, cc = idx & 63;
    Sf[blk][r][cc] = ((blk == 0 || blk == 3) && r == cc) ? 1.f : 0.f;
  }
  __syncthreads();
#pragma unroll 1
  for (int c = ce; c >= cb; --c) {
    float* suf = ws.suf + ((int64_t)bh * NT + c) * (WK * WK);
#pragma unroll 1
    for (int blk = 0; blk < 4; ++blk) store_blk(suf + (blk >> 1) * 64 * WK + (blk & 1) * 64, WK, Sf[blk]);
    load_rows64_f32(Op[0], ws.kt + ((int64_t)bh * T + c * PC) * WK, WK);
    load_rows64_f32(Op[1], ws.kt + ((int64_t)bh * T + c * PC) * WK + 64, WK);
    __syncthreads();
    // KL_c[r][d] = sum_e k~[r][e] SUF[d][e]
#pragma unroll 1
    for (int dh = 0; dh < 2; ++dh) {
      f32x16 a = mgemm64<false, true>(Op[0], Sf[2 * dh], z);
      a = mgemm64<false, true>(Op[1], Sf[2 * dh + 1], a);
      bf16* dst = ws.kl + ((int64_t)bh * T + c * PC) * WK + 64 * dh;
      const int cl = dl_col();
      DL_FOR_E dst[dl_row(e) * WK + cl] = (bf16)a[e];
    }
    __syncthreads();
    const float* hc = ws.hc + ((int64_t)bh * NT + c) * (WK * WK);
#pragma unroll 1
    for (int blk = 0; blk < 4; ++blk) load_blk(Op[blk], hc + (blk >> 1) * 64 * WK + (blk & 1) * 64, WK);
    __syncthreads();
    f32x16 nb[4];
#pragma unroll
    for (int blk = 0; blk < 4; ++blk) {
      const int ra = blk >> 1, cb_ = blk & 1;
      nb[blk] = mgemm64<false, false>(Sf[2 * ra], Op[cb_], z);
      nb[blk] = mgemm64<false, false>(Sf[2 * ra + 1], Op[2 + cb_], nb[blk]);
    }
    __syncthreads();
#pragma unroll
    for (int blk = 0; blk < 4; ++blk) dl_store(Sf[blk], nb[blk], 0);
    __syncthreads();
  }
  float* hl = ws.hl + ((int64_t)bh * NS + s) * (WK * WK);
  bf16* hls = ws.hls + ((int64_t)bh * NS + s) * (2 * WK * WK);
#pragma unroll 1
  for (int blk = 0; blk < 4; ++blk) {
    const int o = (blk >> 1) * 64 * WK + (blk & 1) * 64;
    store_blk(hl + o, WK, Sf[blk]);
    for (int idx = threadIdx.x; idx < 4096; idx += 256) {
      const int r = idx >> 6, cc = idx & 63;
      put_split<2>(hls, WK * WK, o + r * WK + cc, Sf[blk][r][cc]);
    }
  }
}

// x <- x M for rows [r0, r0 + 32 nrt) of X [rows][128] (fp32 LDS) with M^T in MT
// (MT[n][k] = M[k][n]): output tile (value tile dt, row tile rt) in D layout (m = column
// of the product, lane <-> row), 3-term bf16 split products over the 128 columns
__device__ __forceinline__ f32x16 mat_xM128_tile(const float (*X)[132], const float (*MT)[132], int dt, int rt) {
  const int lane = threadIdx.x & 63, g = lane >> 5, l32 = lane & 31;
  f32x16 o = zero16();
#pragma unroll
  for (int st = 0; st < 8; ++st) {
    bf16x8 ah, al, bh8, bl;
    split8(&MT[dt * 32 + l32][16 * st + 8 * g], ah, al);
    split8(&X[rt * 32 + l32][16 * st + 8 * g], bh8, bl);
    o = mfma32(ah, bh8, o);
    o = mfma32(ah, bl, o);
    o = mfma32(al, bh8, o);
  }
  return o;
}

// M^T of a 128 x 128 fp32 row-major matrix into LDS (MT[c][r] = M[r][c]); TR = false: M itself
template <bool TR>
__device__ __forceinline__ void load_mat128(float (*dst)[132], const float* __restrict__ src) {
  for (int idx = threadIdx.x; idx < WK * WK / 4; idx += 256) {
    const int r = idx >> 5, c4 = (idx & 31) * 4;
    const f32x4 v = *reinterpret_cast<const f32x4*>(src + r * WK + c4);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if (TR)
        dst[c4 + e][r] = v[e];
      else
        dst[r][c4 + e] = v[e];
    }
  }
}

// ---------------------------------------------------------------------------
// Query transport at K = 128 (path_transport_kernel's algebra: QS slots inside the large
// chunk, then QB for every earlier large chunk), one workgroup per pair of chunks
// A = 2p, B = 2p + 1; wave w computes value tile w of every row tile.  grid (B*HQ, ceil(NT/2))
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void path_transport128_kernel(int HQ, int H, int T, PathFwdWs ws) {
  __shared__ __attribute__((aligned(16))) float X[128][132];  // rows 0..63 = chunk A, 64..127 = chunk B
  // the step's transition matrix M as bf16 hi and lo planes, row-major, swizzled (chunk c of
  // row r at c ^ (r & 7)); its columns (the A operand of D^T = M^T X^T) come through
  // transposing reads
  __shared__ __attribute__((aligned(16))) bf16 Ms[2][WK * WK];
  const int p = (int)gridDim.y - 1 - (int)blockIdx.y, bhq = blockIdx.x;
  const int NT = T / PC, NS = (NT + PR - 1) / PR;
  const int G = HQ / H;
  const int b = bhq / HQ, hq = bhq - b * HQ, bh = b * H + hq / G;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, g = lane >> 5, l32 = lane & 31;
  const int A = 2 * p;
  const bool hasB = A + 1 < NT;
  const int sI = A / PR, cb = sI * PR;
  {
    const float* src = ws.qt + ((int64_t)bhq * T + A * PC) * WK;  // A's and B's rows are adjacent
    for (int idx = tid; idx < (hasB ? 128 : 64) * 32; idx += 256) {
      const int r = idx >> 5, c4 = (idx & 31) * 4;
      *reinterpret_cast<f32x4*>(&X[r][c4]) = *reinterpret_cast<const f32x4*>(src + (int64_t)r * WK + c4);
    }
  }
  __syncthreads();
  auto emit = [&](bf16* dst, int r0, int nblk) {  // rows r0 .. r0 + 64 nblk of X -> bf16 rows (stride 128)
    for (int idx = tid; idx < 64 * nblk * 16; idx += 256) {
      const int r = r0 + (idx >> 4), c8 = (idx & 15) * 8;
      bf16x8 v;
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = (bf16)X[r][c8 + e];
      *reinterpret_cast<bf16x8*>(dst + (int64_t)r * WK + c8) = v;
    }
  };
  // Each step emits X, then multiplies it by the step's matrix; after the last emit X is not
  // used, so the last step only emits.  The next step's matrix is loaded into registers while
  // a step computes.
  const int nq = A - cb, nsteps = nq + sI;
  auto mat = [&](int j) {  // hi plane (lo plane WK * WK elements on); j = -1: Hc_A, B's own first step
    return (j < nq) ? ws.hcs + ((int64_t)bh * NT + (A - 1 - j)) * (2 * WK * WK)
                    : ws.hls + ((int64_t)bh * NS + (sI - 1 - (j - nq))) * (2 * WK * WK);
  };
  auto slot = [&](int j) {  // destination of the rows emitted before step j (row 0 = chunk A's first row)
    return ((j < nq) ? ws.qs + (((int64_t)bhq * PR + (A - 1 - j - cb)) * T) * WK
                     : ws.qb + (((int64_t)bhq * NS + (sI - 1 - (j - nq))) * T) * WK) +
           (int64_t)A * PC * WK;
  };
  bf16x8 mr[16];  // thread t: plane u >> 3, 16-byte chunk q = t + 256 (u & 7) (row q >> 4, chunk q & 15)
  auto mload = [&](int j) {
    const bf16* M = mat(j);
#pragma unroll
    for (int u = 0; u < 16; ++u) mr[u] = ld8(M + (u >> 3) * (WK * WK) + 8 * (tid + 256 * (u & 7)));
  };
  auto mstore = [&]() {
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const int q = tid + 256 * (u & 7);
      *reinterpret_cast<bf16x8*>(Ms[u >> 3] + swz_off<16>(q >> 4, q & 15)) = mr[u];
    }
  };
  // tile (value tile w, row tile xr) of X M in D layout (m = column of the product, lane <->
  // row), 3-term split: A operand = columns w*32 + lane of M, k slots in the transposing
  // read's order (rows 16 st + jmap(slot)); B operand = the same k of X row xr*32 + lane
  auto xm_tile = [&](int xr) {
    f32x16 o = zero16();
#pragma unroll
    for (int st = 0; st < 8; ++st) {
      const bf16x8 ah = lds_tr_a<16>(Ms[0], 16 * st, w * 32);
      const bf16x8 al = lds_tr_a<16>(Ms[1], 16 * st, w * 32);
      const f32x4 x0 = *reinterpret_cast<const f32x4*>(&X[xr * 32 + l32][16 * st + 4 * g]);
      const f32x4 x1 = *reinterpret_cast<const f32x4*>(&X[xr * 32 + l32][16 * st + 8 + 4 * g]);
      const float v[8] = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
      bf16x8 bh8, bl;
      split_vals(v, bh8, bl);
      o = mfma32(ah, bh8, o);
      o = mfma32(ah, bl, o);
      o = mfma32(al, bh8, o);
    }
    return o;
  };
  // rows [rt0, rt0 + 32 nrt) of X <- X M (every wave: value tile w); next: store the
  // prefetched matrix of the next step once every wave has read this one
  auto step = [&](int rt0, int nrt, bool next) {
    f32x16 o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (i < nrt) o[i] = xm_tile(rt0 + i);
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (i < nrt) {
#pragma unroll
        for (int e = 0; e < 16; ++e) X[(rt0 + i) * 32 + l32][w * 32 + drow(e, g)] = o[i][e];
      }
    if (next) mstore();
    __syncthreads();
  };
  if (hasB) {  // B's own first step: emit to QS slot A - cb, then X_B <- X_B Hc_A (if an emit follows)
    emit(ws.qs + (((int64_t)bhq * PR + (A - cb)) * T) * WK + (int64_t)A * PC * WK, 64, 1);
    if (nsteps > 0) {
      mload(-1);
      mstore();
      __syncthreads();
      if (nsteps > 1) mload(0);
      step(2, 2, nsteps > 1);
    }
  } else if (nsteps > 1) {
    mload(0);
    mstore();
    __syncthreads();
  }
  const int nblk = hasB ? 2 : 1;
#pragma unroll 1
  for (int j = 0; j < nsteps; ++j) {
    emit(slot(j), 0, nblk);
    if (j + 1 == nsteps) break;
    const bool next = j + 2 < nsteps;
    if (next) mload(j + 1);
    step(0, 2 * nblk, next);
  }
}

// ---------------------------------------------------------------------------
// k_cache at K = 128 (path_kcache_kernel's algebra): x = KL_J; x <- x HL_s^T for every
// later large chunk.  grid (NT, B*H)
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void path_kcache128_kernel(int T, bf16* __restrict__ kc, Strides kcs, int H,
                                                             PathFwdWs ws) {
  __shared__ __attribute__((aligned(16))) float X[64][132];
  __shared__ __attribute__((aligned(16))) float MT[128][132];
  const int J = blockIdx.x, bh = blockIdx.y;
  const int b = bh / H, h = bh - b * H;
  const int NT = T / PC, NS = (NT + PR - 1) / PR;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, g = lane >> 5, l32 = lane & 31;
  for (int idx = tid; idx < 64 * 16; idx += 256) {
    const int r = idx >> 4, c8 = (idx & 15) * 8;
    const bf16x8 v = ld8(ws.kl + ((int64_t)bh * T + J * PC + r) * WK + c8);
#pragma unroll
    for (int e = 0; e < 8; ++e) X[r][c8 + e] = (float)v[e];
  }
  __syncthreads();
#pragma unroll 1
  for (int s = J / PR + 1; s < NS; ++s) {
    load_mat128<false>(MT, ws.hl + ((int64_t)bh * NS + s) * (WK * WK));  // (HL^T)^T = HL
    __syncthreads();
    f32x16 o[2];
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) o[rt] = mat_xM128_tile(X, MT, w, rt);
    __syncthreads();
#pragma unroll
    for (int rt = 0; rt < 2; ++rt)
#pragma unroll
      for (int e = 0; e < 16; ++e) X[rt * 32 + l32][w * 32 + drow(e, g)] = o[rt][e];
    __syncthreads();
  }
  for (int idx = tid; idx < 64 * 16; idx += 256) {
    const int r = idx >> 4, c8 = (idx & 15) * 8;
    bf16x8 v;
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = (bf16)X[r][c8 + e];
    *reinterpret_cast<bf16x8*>(kc + b * kcs.b + h * kcs.h + (int64_t)(J * PC + r) * kcs.t + c8) = v;
  }
}

// ---------------------------------------------------------------------------
// Products backward at K = 128 (path_products_bwd_kernel's algebra) inside one large chunk:
//   F = dHL_s; for c from the bottom up: dHc_c += SUF_c^T F; F <- F Hc_c^T + dSUF_c
// F as four 64 x 64 blocks, SUF_c and then Hc_c as four more.  grid (NS, B*HQ)
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void path_products_bwd128_kernel(int HQ, int H, int T, PathFwdWs ws, PathBwdWs bw) {
  __shared__ __attribute__((aligned(16))) float Fb[4][64][68];  // block (r, c) at 2 r + c
  __shared__ __attribute__((aligned(16))) float Ob[4][64][68];
  const int NT = T / PC, NS = (NT + PR - 1) / PR;
  const int s = blockIdx.x, bhq = blockIdx.y;
  const int G_ = HQ / H;
  const int b = bhq / HQ, hq = bhq - b * HQ, bh = b * H + hq / G_;
  const int cb = s * PR, ce = min(cb + PR, NT) - 1;
  const int cl = dl_col();
  const f32x16 z = zero16();
  constexpr int KK = WK * WK;
  const float* dhl = bw.dhl + ((int64_t)bhq * NS + s) * KK;
#pragma unroll 1
  for (int blk = 0; blk < 4; ++blk) load_blk(Fb[blk], dhl + (blk >> 1) * 64 * WK + (blk & 1) * 64, WK);
#pragma unroll 1
  for (int c = cb; c <= ce; ++c) {
    const float* suf = ws.suf + ((int64_t)bh * NT + c) * KK;
#pragma unroll 1
    for (int blk = 0; blk < 4; ++blk) load_blk(Ob[blk], suf + (blk >> 1) * 64 * WK + (blk & 1) * 64, WK);
    __syncthreads();
    {  // dHc_c(a, b) += sum_k SUF_c(k, a)^T F(k, b)
      float* dhc = bw.dhc + ((int64_t)bhq * NT + c) * KK;
#pragma unroll 1
      for (int blk = 0; blk < 4; ++blk) {
        const int ra = blk >> 1, cb_ = blk & 1;
        f32x16 a = mgemm64<true, false>(Ob[ra], Fb[cb_], z);
        a = mgemm64<true, false>(Ob[2 + ra], Fb[2 + cb_], a);
        DL_FOR_E dhc[(int64_t)(64 * ra + dl_row(e)) * WK + 64 * cb_ + cl] += a[e];
      }
    }
    __syncthreads();
    const float* hc = ws.hc + ((int64_t)bh * NT + c) * KK;
#pragma unroll 1
    for (int blk = 0; blk < 4; ++blk) load_blk(Ob[blk], hc + (blk >> 1) * 64 * WK + (blk & 1) * 64, WK);
    __syncthreads();
    f32x16 nb[4];  // F(a, b) <- sum_k F(a, k) Hc_c(b, k)^T + dSUF_c(a, b)
#pragma unroll
    for (int blk = 0; blk < 4; ++blk) {
      const int ra = blk >> 1, cb_ = blk & 1;
      nb[blk] = mgemm64<false, true>(Fb[2 * ra], Ob[2 * cb_], z);
      nb[blk] = mgemm64<false, true>(Fb[2 * ra + 1], Ob[2 * cb_ + 1], nb[blk]);
    }
    __syncthreads();
    const float* ds = bw.dsuf + ((int64_t)bhq * NT + c) * KK;
#pragma unroll
    for (int blk = 0; blk < 4; ++blk) {
      const int ra = blk >> 1, cb_ = blk & 1;
      DL_FOR_E {
        const int r = dl_row(e);
        Fb[blk][r][cl] = nb[blk][e] + ds[(int64_t)(64 * ra + r) * WK + 64 * cb_ + cl];
      }
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// Backward of the WY form of one chunk at K = 128 (path_wy_bwd_kernel's algebra), with the
// 64 x 128 operands and results taken as 64-column halves and beta folded into row / column
// scalings of the products (Wb = diag(beta) W is formed only where it is an operand):
//   A: Tm = (I + stril(diag(b) W W^T))^-1, QW = tril(Q W^T), WBK = stril(diag(b) W K^T), TW = Tm WBK
//   B: dQW = -(dq~ W2^T + dA TW^T), dW2 = -(QW^T dq~ + W dHc), dTW = -(W dk~^T + QW^T dA),
//      dW = -(TW dk~ + W2 dHc^T) + ...
//   C: dTm = dTW WBK^T + dW2 Wb^T, dWBK = stril(Tm^T dTW), dWb = Tm^T dW2 + ...,
//      da = -stril((Tm^T dTm) Tm^T)
//   D (per half): dq = dq~ + dA K + tril(dQW) W, dk = dk~ + dA^T Q + dWBK^T Wb,
//      dWb += dWBK K + da W, dW += tril(dQW)^T Q + da^T Wb + diag(b) dWb, db = rowsum(dWb * W)
// LDS: nine 64 x 64 fp32 blocks.  grid (NT, B*HQ)
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void path_wy_bwd128_kernel(const bf16* __restrict__ q, Strides qs,
                                                             const bf16* __restrict__ k, Strides ks,
                                                             const bf16* __restrict__ w, Strides wst,
                                                             const bf16* __restrict__ beta, Strides bst, int HQ, int H,
                                                             int T, PathFwdWs ws, PathBwdWs bw) {
  __shared__ __attribute__((aligned(16))) float S[9][64][68];
  __shared__ float bsh[64];
  __shared__ float dbs[2][64];
  const int NT = T / PC;
  const int c = blockIdx.x, bhq = blockIdx.y;
  const int G_ = HQ / H;
  const int b = bhq / HQ, hq = bhq - b * HQ, h = hq / G_, bh = b * H + h;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, g = lane >> 5;
  const int t0 = c * PC;
  const f32x16 z = zero16();
  const int cl = dl_col();
  const bf16* wp = w + b * wst.b + h * wst.h + (int64_t)t0 * wst.t;
  const bf16* qp = q + b * qs.b + hq * qs.h + (int64_t)t0 * qs.t;
  const bf16* kp = k + b * ks.b + h * ks.h + (int64_t)t0 * ks.t;
  const float* w2p = ws.w2 + ((int64_t)bh * T + t0) * WK;
  const float* dqp = bw.dqt + ((int64_t)bhq * T + t0) * WK;
  const float* dkp = bw.dkt + ((int64_t)bhq * T + t0) * WK;
  if (tid < 64) bsh[tid] = (float)beta[b * bst.b + h * bst.h + (int64_t)(t0 + tid) * bst.t];
  // ---- A: the forward's in-chunk matrices ----
  f32x16 aA = z, aQW = z, aWK = z;
#pragma unroll 1
  for (int hh = 0; hh < 2; ++hh) {
    load_rows64_f32(S[0], wp + 64 * hh, wst.t);
    load_rows64_f32(S[1], qp + 64 * hh, qs.t);
    load_rows64_f32(S[2], kp + 64 * hh, ks.t);
    __syncthreads();
    aA = mgemm64<false, true>(S[0], S[0], aA);
    aQW = mgemm64<false, true>(S[1], S[0], aQW);
    aWK = mgemm64<false, true>(S[0], S[2], aWK);
    __syncthreads();
  }
  DL_FOR_E {
    const float br = bsh[dl_row(e)];
    aA[e] *= br;
    aWK[e] *= br;
  }
  float(*Tm)[68] = S[3];
  float(*QW)[68] = S[4];
  float(*WBK)[68] = S[5];
  float(*TW)[68] = S[6];
  float(*dA)[68] = S[7];
  dl_store(Tm, aA, 2);
  dl_store(QW, aQW, 1);
  dl_store(WBK, aWK, 2);
  __syncthreads();
  invert_unit_lower64(Tm);
  dl_store(TW, mgemm64<false, false>(Tm, WBK, z), 0);
  load_blk(dA, bw.dad + ((int64_t)bhq * NT + c) * 4096, 64);
  __syncthreads();
  // ---- B ----
  f32x16 aW2[2], aW[2], dQW = z, dTW = z;
#pragma unroll
  for (int hh = 0; hh < 2; ++hh) {
    load_blk(S[0], w2p + 64 * hh, WK);
    load_blk(S[1], dqp + 64 * hh, WK);
    __syncthreads();
    dQW = mgemm64<false, true>(S[1], S[0], dQW);          // dq~_h W2_h^T
    aW2[hh] = dl_neg(mgemm64<true, false>(QW, S[1], z));  // -QW^T dq~_h
    __syncthreads();
  }
  dQW = dl_neg(mgemm64<false, true>(dA, TW, dQW));  // -(dq~ W2^T + dA TW^T)
#pragma unroll
  for (int hh = 0; hh < 2; ++hh) {
    load_rows64_f32(S[0], wp + 64 * hh, wst.t);
    load_blk(S[1], dkp + 64 * hh, WK);
    __syncthreads();
    dTW = mgemm64<false, true>(S[0], S[1], dTW);         // W_h dk~_h^T
    aW[hh] = dl_neg(mgemm64<false, false>(TW, S[1], z));  // -TW dk~_h
    __syncthreads();
  }
  dTW = dl_neg(mgemm64<true, false>(QW, dA, dTW));  // -(W dk~^T + QW^T dA)
  __syncthreads();
  // dW2(:, b) -= W_a dHc(a, b), dW(:, a) -= W2_b dHc(a, b)^T
  load_rows64_f32(S[0], wp, wst.t);
  load_rows64_f32(S[1], wp + 64, wst.t);
  load_blk(S[2], w2p, WK);
  load_blk(S[4], w2p + 64, WK);
  {
    const float* dhc = bw.dhc + ((int64_t)bhq * NT + c) * (WK * WK);
#pragma unroll
    for (int blk = 0; blk < 4; ++blk) {
      const int ra = blk >> 1, cb_ = blk & 1;
      load_blk(S[6], dhc + (int64_t)64 * ra * WK + 64 * cb_, WK);
      __syncthreads();
      const f32x16 t1 = mgemm64<false, true>(cb_ ? S[4] : S[2], S[6], z);
      const f32x16 t2 = mgemm64<false, false>(ra ? S[1] : S[0], S[6], z);
      DL_FOR_E {
        aW[ra][e] -= t1[e];
        aW2[cb_][e] -= t2[e];
      }
      __syncthreads();
    }
  }
  // ---- C ----
  dl_store(S[8], dTW, 0);
  dl_store(S[2], aW2[0], 0);
  dl_store(S[4], aW2[1], 0);
  __syncthreads();
  f32x16 dTm = mgemm64<false, true>(S[8], WBK, z);  // dTW WBK^T
  {
    f32x16 t = mgemm64<false, true>(S[2], S[0], z);  // dW2 W^T, then the column scaling by beta
    t = mgemm64<false, true>(S[4], S[1], t);
    const float bc = bsh[cl];
    DL_FOR_E dTm[e] = fmaf(t[e], bc, dTm[e]);
  }
  f32x16 aWb[2];
  aWb[0] = mgemm64<true, false>(Tm, S[2], z);  // Tm^T dW2
  aWb[1] = mgemm64<true, false>(Tm, S[4], z);
  const f32x16 dWBK = mgemm64<true, false>(Tm, S[8], z);  // Tm^T dTW
  __syncthreads();
  dl_store(S[5], dWBK, 2);
  dl_store(S[6], dTm, 0);
  __syncthreads();
  dl_store(S[8], mgemm64<true, false>(Tm, S[6], z), 0);  // Tm^T dTm
  __syncthreads();
  const f32x16 da = dl_neg(mgemm64<false, true>(S[8], Tm, z));
  __syncthreads();
  dl_store(S[6], da, 2);
  dl_store(S[8], dQW, 1);
  // ---- D: per 64-column half ----
  float rs[16];
#pragma unroll
  for (int e = 0; e < 16; ++e) rs[e] = 0.f;
#pragma unroll 1
  for (int hh = 0; hh < 2; ++hh) {
    float(*Wh)[68] = hh ? S[1] : S[0];
    load_rows64_f32(S[4], qp + 64 * hh, qs.t);
    load_rows64_f32(S[3], kp + 64 * hh, ks.t);
    for (int idx = tid; idx < 4096; idx += 256) S[2][idx >> 6][idx & 63] = bsh[idx >> 6] * Wh[idx >> 6][idx & 63];
    __syncthreads();
    f32x16 aq = mgemm64<false, false>(dA, S[3], z);  // dA K_h
    aq = mgemm64<false, false>(S[8], Wh, aq);        // + tril(dQW) W_h
    f32x16 ak = mgemm64<true, false>(dA, S[4], z);   // dA^T Q_h
    ak = mgemm64<true, false>(S[5], S[2], ak);       // + dWBK^T Wb_h
    f32x16 wb = mgemm64<false, false>(S[5], S[3], aWb[hh]);  // + dWBK K_h
    wb = mgemm64<false, false>(S[6], Wh, wb);                 // + da W_h
    f32x16 dw = mgemm64<true, false>(S[8], S[4], aW[hh]);     // + tril(dQW)^T Q_h
    dw = mgemm64<true, false>(S[6], S[2], dw);                // + da^T Wb_h
    const int64_t rowbase = ((int64_t)bhq * T + t0) * WK + 64 * hh;
    DL_FOR_E {
      const int r = dl_row(e);
      const int64_t off = rowbase + (int64_t)r * WK + cl;
      bw.dq[off] = aq[e] + dqp[r * WK + 64 * hh + cl];
      bw.dk[off] = ak[e] + dkp[r * WK + 64 * hh + cl];
      bw.dw[off] = fmaf(bsh[r], wb[e], dw[e]);
      rs[e] = fmaf(wb[e], Wh[r][cl], rs[e]);
    }
    __syncthreads();
  }
  // db_r = sum over the 128 columns: the 32 lanes of a half-wave, then the two column-half waves
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    float x = rs[e];
    x += __shfl_xor(x, 1, 64);
    x += __shfl_xor(x, 2, 64);
    x += __shfl_xor(x, 4, 64);
    x += __shfl_xor(x, 8, 64);
    x += __shfl_xor(x, 16, 64);
    rs[e] = x;
  }
  if ((lane & 31) == 0) {
#pragma unroll
    for (int e = 0; e < 16; ++e) dbs[wv & 1][32 * (wv >> 1) + drow(e, g)] = rs[e];
  }
  __syncthreads();
  if (tid < 64) bw.db[(int64_t)bhq * T + t0 + tid] = dbs[0][tid] + dbs[1][tid];
}

}  // namespace lucid
