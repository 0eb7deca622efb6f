// LUCID attention forward on CDNA4 (gfx950).
//
//   K^ = K / sqrt(mean_d K^2 + eps)                       (modeling_lucid.py:409, :564)
//   P_ij = exp(s K^_i.K^_j - 1/s), j <= i                 (:565-569)
//   V'  = P^-1 V  (chained block forward substitution)    (:570, :285-312)
//   O   = softmax(s Q K^T, causal) V'                     (:520-530)
//
// Kernels (all 256 threads = 4 waves, MFMA 32x32x16 bf16, fp32 accumulate):
//   lucid_prep_kernel        per-row 1/rms of K, K^ rows in bf16, K^T in T-perm layout,
//                            inverses of the 64x64 diagonal blocks of P, zero chain counters
//   lucid_zx_kernel          the in-block coupling -X_B P_BA of every 128-row chain block and
//                            (precision "auto") the heads' row masses, lucid_mass_kernel's work
//   lucid_precond_fwd_kernel chained solve, one workgroup per (128-row block, kv head);
//                            it waits on a per-head progress counter for V'_j, j < i and
//                            sweeps the earlier keys 128 at a time
//   lucid_attn_fwd_kernel    causal online-softmax attention on V' (256 query rows / WG, LDS tiles)
#include <type_traits>

#include "lucid_common.h"

namespace lucid {

// ---------------------------------------------------------------------------
// prep: rinv[bh][t] = 1/sqrt(sum K^2 / dn + eps) (dn: the head dim, rows zero-padded beyond it;
// dn <= 0: keys already normalised, rinv = 1); kt[bh][d][perm(t)] = K[t][d];
// pinv[bh][blk] = inverse of the 64x64 diagonal block of P (fp32 forward
// substitution by wave 0); zero the chain counter and set the head's row mass
// to mass_init (0 before lucid_mass_kernel; a forced precision sets it directly);
// khat (if not null): khat[bh][t] = K^_t = r_t K_t rounded to bf16.
// grid (T/64, B*Hkv)
// ---------------------------------------------------------------------------
template <int D, bool F32 = false>
__global__ __launch_bounds__(256) void lucid_prep_kernel(const bf16* __restrict__ k, Strides ks, int Hkv, int T,
                                                         float eps, float dn, float scale, float* __restrict__ rinv,
                                                         bf16* __restrict__ kt, float* __restrict__ pinv,
                                                         int* __restrict__ counters, float* __restrict__ mass,
                                                         float mass_init, Lo lo, bf16* __restrict__ ktl,
                                                         bf16* __restrict__ khat) {
  constexpr int SEG = D / 4;
  constexpr int NKS = D / 16;
  __shared__ bf16 tile[F32 ? 2 : 1][D][64 + 8];
  __shared__ float rr[64];
  __shared__ __attribute__((aligned(16))) float Pd[64][68];
  const int blk = blockIdx.x, bh = blockIdx.y;
  const int b = bh / Hkv, h = bh - b * Hkv;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int g = lane >> 5, l32 = lane & 31;
  const bf16* kp = k + b * ks.b + h * ks.h + (int64_t)blk * 64 * ks.t;
  const bf16* klp = F32 ? lo.k + b * ks.b + h * ks.h + (int64_t)blk * 64 * ks.t : nullptr;
  const int row = tid >> 2, seg = tid & 3;
  float ss = 0.f;
  bf16x8 xs[SEG / 8];
#pragma unroll
  for (int c = 0; c < SEG; c += 8) {
    const bf16x8 x = ld8(kp + row * ks.t + seg * SEG + c);
    xs[c / 8] = x;
    bf16x8 xl;
    if constexpr (F32) xl = ld8(klp + row * ks.t + seg * SEG + c);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float f = (float)x[e];
      if constexpr (F32) {
        f += (float)xl[e];
        tile[1][seg * SEG + c + e][row] = xl[e];
      }
      ss += f * f;
      tile[0][seg * SEG + c + e][row] = x[e];
    }
  }
  ss += __shfl_xor(ss, 1, 64);
  ss += __shfl_xor(ss, 2, 64);
  // dn <= 0: the keys arrive normalised (the Lucid_Tril_Solver seam takes K^ itself): r = 1
  const float ri = dn > 0.f ? 1.0f / sqrtf(ss / dn + eps) : 1.0f;
  if (seg == 0) {
    rinv[(int64_t)bh * T + blk * 64 + row] = ri;
    rr[row] = ri;
  }
  if (khat) {  // K^ rows in bf16 (the bf16 chains' staged key tiles)
    bf16* dst = khat + ((int64_t)bh * T + blk * 64 + row) * D + seg * SEG;
#pragma unroll
    for (int c = 0; c < SEG; c += 8) *reinterpret_cast<bf16x8*>(dst + c) = scale8(xs[c / 8], ri);
  }
  if (blk == 0 && tid == 0) {
    counters[bh] = 0;
    mass[bh] = mass_init;
  }
  __syncthreads();
  // T-perm rows: kt[bh][d][blk*64 + slot], slot kappa holds t = jmap(kappa)
  for (int idx = tid; idx < D * 8; idx += 256) {
    const int dd = idx >> 3, c8 = idx & 7;
    bf16x8 out;
#pragma unroll
    for (int e = 0; e < 8; ++e) out[e] = tile[0][dd][(c8 >> 1) * 16 + jmap((c8 & 1) * 8 + e)];
    *reinterpret_cast<bf16x8*>(kt + ((int64_t)bh * D + dd) * T + blk * 64 + c8 * 8) = out;
    if constexpr (F32) {
#pragma unroll
      for (int e = 0; e < 8; ++e) out[e] = tile[1][dd][(c8 >> 1) * 16 + jmap((c8 & 1) * 8 + e)];
      *reinterpret_cast<bf16x8*>(ktl + ((int64_t)bh * D + dd) * T + blk * 64 + c8 * 8) = out;
    }
  }
  // diagonal block P[m][n] = exp(s r_m r_n K_m.K_n - 1/s) (n <= m); wave -> 32x32 quadrant
  {
    const float sl2 = scale * LOG2E_F;
    const float c0 = LOG2E_F / scale;
    const int mh = w >> 1, nh = w & 1;
    f32x16 sd = zero16();
    if (nh <= mh) {
#pragma unroll
      for (int st = 0; st < NKS; ++st) {
        const int64_t om = (mh * 32 + l32) * ks.t + 16 * st + 8 * g, on = (nh * 32 + l32) * ks.t + 16 * st + 8 * g;
        sd = mfma32(ld8(kp + om), ld8(kp + on), sd);
        if constexpr (F32) {
          sd = mfma32(ld8(kp + om), ld8(klp + on), sd);
          sd = mfma32(ld8(klp + om), ld8(kp + on), sd);
          sd = mfma32(ld8(klp + om), ld8(klp + on), sd);
        }
      }
    }
    const int n = nh * 32 + l32;
    const float an = sl2 * rr[n];
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int m = mh * 32 + drow(e, g);
      Pd[m][n] = (n <= m) ? __builtin_amdgcn_exp2f(fmaf(sd[e] * an, rr[m], -c0)) : 0.f;
    }
  }
  __syncthreads();
  if (w == 0) invert_lower64(Pd, lane, pinv + ((int64_t)bh * (T / 64) + blk) * 4096);
}

// ---------------------------------------------------------------------------
// Operands of the attention on a caller's V' (eager_lucid_attention_forward): V' rows
// (bf16 or fp32, strided) to the bf16 row-major copy vpb and the T-perm copy vpt the
// attention kernels read, 1/rms of K for the row-mass pass, and the head's row mass
// initialised to mass_init.  LO (fp32 V', fp32-input kernels): V' also as its bf16 lo
// parts vpbl (row-major) and vptl (T-perm), V' ~= hi + lo.  grid (T/64, B*Hkv)
// ---------------------------------------------------------------------------
template <int D, typename VT, bool LO = false>
__global__ __launch_bounds__(256) void lucid_vp_layout_kernel(const bf16* __restrict__ k, Strides ks,
                                                              const VT* __restrict__ vp, Strides vs, int Hkv, int T,
                                                              float eps, float dn, float* __restrict__ rinv,
                                                              bf16* __restrict__ vpb, bf16* __restrict__ vpt,
                                                              float* __restrict__ mass, float mass_init,
                                                              bf16* __restrict__ vpbl, bf16* __restrict__ vptl) {
  static_assert(!LO || std::is_same<VT, float>::value, "lo parts of an fp32 V' only");
  constexpr int SEG = D / 4;
  __shared__ bf16 tile[LO ? 2 : 1][D][64 + 8];
  const int blk = blockIdx.x, bh = blockIdx.y;
  const int b = bh / Hkv, h = bh - b * Hkv;
  const int tid = threadIdx.x;
  const int row = tid >> 2, seg = tid & 3;
  const int t = blk * 64 + row;
  const bf16* kr = k + b * ks.b + h * ks.h + (int64_t)t * ks.t;
  const VT* vr = vp + b * vs.b + h * vs.h + (int64_t)t * vs.t;
  bf16* ob = vpb + ((int64_t)bh * T + t) * D;
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < SEG; c += 8) {
    const bf16x8 x = ld8(kr + seg * SEG + c);
    bf16x8 y, yl;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float f = (float)x[e];
      ss += f * f;
      const float vv = (float)vr[seg * SEG + c + e];
      y[e] = (bf16)vv;
      tile[0][seg * SEG + c + e][row] = y[e];
      if constexpr (LO) {
        yl[e] = (bf16)(vv - (float)y[e]);
        tile[1][seg * SEG + c + e][row] = yl[e];
      }
    }
    *reinterpret_cast<bf16x8*>(ob + seg * SEG + c) = y;
    if constexpr (LO) *reinterpret_cast<bf16x8*>(vpbl + ((int64_t)bh * T + t) * D + seg * SEG + c) = yl;
  }
  ss += __shfl_xor(ss, 1, 64);
  ss += __shfl_xor(ss, 2, 64);
  if (seg == 0) rinv[(int64_t)bh * T + t] = 1.0f / sqrtf(ss / dn + eps);
  if (blk == 0 && tid == 0) mass[bh] = mass_init;
  __syncthreads();
  for (int idx = tid; idx < D * 8; idx += 256) {
    const int dd = idx >> 3, c8 = idx & 7;
    bf16x8 out;
#pragma unroll
    for (int e = 0; e < 8; ++e) out[e] = tile[0][dd][(c8 >> 1) * 16 + jmap((c8 & 1) * 8 + e)];
    *reinterpret_cast<bf16x8*>(vpt + ((int64_t)bh * D + dd) * T + blk * 64 + c8 * 8) = out;
    if constexpr (LO) {
#pragma unroll
      for (int e = 0; e < 8; ++e) out[e] = tile[1][dd][(c8 >> 1) * 16 + jmap((c8 & 1) * 8 + e)];
      *reinterpret_cast<bf16x8*>(vptl + ((int64_t)bh * D + dd) * T + blk * 64 + c8 * 8) = out;
    }
  }
}

// Rows of an fp32 [BH][T][D] buffer to a strided bf16 or fp32 tensor (the attention
// seam's dK and dV' outputs), scaled by `mul`.  grid (T/64, B*H)
template <int D, typename OT>
__global__ __launch_bounds__(256) void lucid_rows_out_kernel(const float* __restrict__ src, OT* __restrict__ dst,
                                                             Strides ds, int H, int T, float mul) {
  const int blk = blockIdx.x, bh = blockIdx.y;
  const int b = bh / H, h = bh - b * H;
  for (int idx = threadIdx.x; idx < 64 * D / 4; idx += 256) {
    const int r = idx / (D / 4), c4 = (idx % (D / 4)) * 4;
    const int t = blk * 64 + r;
    const f32x4 x = *reinterpret_cast<const f32x4*>(src + ((int64_t)bh * T + t) * D + c4);
    OT* o = dst + b * ds.b + h * ds.h + (int64_t)t * ds.t + c4;
#pragma unroll
    for (int u = 0; u < 4; ++u) o[u] = (OT)(x[u] * mul);
  }
}

// fp32 inputs: a strided fp32 [B][H][T][D] tensor to the bf16 pair the MFMA operands are
// built from, hi = bf16(x) and lo = bf16(x - hi) (x = hi + lo to ~2^-16 relative), both
// written as contiguous [BH][T][D] rows.  center (fp32 [BH][D], or null): x - center[bh]
// is split instead.  grid (T/64, B*H)
template <int D>
__global__ __launch_bounds__(256) void lucid_split_kernel(const float* __restrict__ src, Strides ss, int H, int T,
                                                          bf16* __restrict__ hi, bf16* __restrict__ lo,
                                                          const float* __restrict__ center) {
  constexpr int SEG = D / 4;
  const int bh = blockIdx.y, b = bh / H, h = bh - b * H;
  const int row = threadIdx.x >> 2, seg = threadIdx.x & 3;
  const int t = blockIdx.x * 64 + row;
  const float* s = src + b * ss.b + h * ss.h + (int64_t)t * ss.t + seg * SEG;
  const float* cen = center ? center + (int64_t)bh * D + seg * SEG : nullptr;
  const int64_t off = ((int64_t)bh * T + t) * D + seg * SEG;
#pragma unroll
  for (int c = 0; c < SEG; c += 8) {
    f32x4 x0 = *reinterpret_cast<const f32x4*>(s + c);
    f32x4 x1 = *reinterpret_cast<const f32x4*>(s + c + 4);
    if (cen) {
      const f32x4 c0 = *reinterpret_cast<const f32x4*>(cen + c);
      const f32x4 c1 = *reinterpret_cast<const f32x4*>(cen + c + 4);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        x0[u] -= c0[u];
        x1[u] -= c1[u];
      }
    }
    bf16x8 a, r;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      a[u] = (bf16)x0[u];
      a[u + 4] = (bf16)x1[u];
      r[u] = (bf16)(x0[u] - (float)a[u]);
      r[u + 4] = (bf16)(x1[u] - (float)a[u + 4]);
    }
    *reinterpret_cast<bf16x8*>(hi + off + c) = a;
    *reinterpret_cast<bf16x8*>(lo + off + c) = r;
  }
}

// Mean key of each head, mean[bh][d] = (1/T) sum_t K[t][d] (fp32 inputs).  The attention's
// scores are taken against K - mean: the softmax is unchanged (a per-row constant Q.mean
// leaves it as it is), dQ = s dS (K - mean) exactly because every row of dS sums to zero,
// and dK does not involve K.  Keys along a shared direction then reach the split products
// as their small deviations, so the 16-bit rounding of dS, dP and the scores no longer
// multiplies the shared part (a ~6-10x smaller dQ error there).  One workgroup per head:
// 256 / (D/4) row phases x D/4 four-column groups, fixed summation order.  grid (B*H)
template <int D>
__global__ __launch_bounds__(256) void lucid_key_mean_kernel(const float* __restrict__ k, Strides ks, int H, int T,
                                                             float* __restrict__ mean) {
  constexpr int CG = D / 4, PH = 256 / CG;
  static_assert(CG * PH == 256, "four-column groups x row phases = 256 threads");
  __shared__ f32x4 part[PH][CG];
  const int bh = blockIdx.x, b = bh / H, h = bh - b * H;
  const int ph = threadIdx.x / CG, c4 = threadIdx.x % CG;
  const float* kp = k + b * ks.b + h * ks.h + 4 * c4;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 8
  for (int t = ph; t < T; t += PH) {
    const f32x4 x = *reinterpret_cast<const f32x4*>(kp + (int64_t)t * ks.t);
#pragma unroll
    for (int u = 0; u < 4; ++u) acc[u] += x[u];
  }
  part[ph][c4] = acc;
  __syncthreads();
  if (ph == 0) {
    f32x4 tot = part[0][c4];
    for (int r = 1; r < PH; ++r)
#pragma unroll
      for (int u = 0; u < 4; ++u) tot[u] += part[r][c4][u];
#pragma unroll
    for (int u = 0; u < 4; ++u) tot[u] /= (float)T;
    *reinterpret_cast<f32x4*>(mean + (int64_t)bh * D + 4 * c4) = tot;
  }
}

// dV' of the preconditioner-only backward (bf16 or fp32, strided) to the fp32
// [BH][T][D] buffer the column chain reads; zero the chain counters.  grid (T/64, B*Hkv)
template <int D, typename IT>
__global__ __launch_bounds__(256) void lucid_rows_in_kernel(const IT* __restrict__ src, Strides ss,
                                                            float* __restrict__ dst, int H, int T,
                                                            int* __restrict__ counters) {
  const int blk = blockIdx.x, bh = blockIdx.y;
  const int b = bh / H, h = bh - b * H;
  if (blk == 0 && threadIdx.x == 0) counters[bh] = 0;
  for (int idx = threadIdx.x; idx < 64 * D / 4; idx += 256) {
    const int r = idx / (D / 4), c4 = (idx % (D / 4)) * 4;
    const int t = blk * 64 + r;
    const IT* i = src + b * ss.b + h * ss.h + (int64_t)t * ss.t + c4;
    f32x4 x;
#pragma unroll
    for (int u = 0; u < 4; ++u) x[u] = (float)i[u];
    *reinterpret_cast<f32x4*>(dst + ((int64_t)bh * T + t) * D + c4) = x;
  }
}

// ---------------------------------------------------------------------------
// Largest row mass m_i = sum_{j<i} P_ij^2 of a head (the quantity that sets the bf16
// error of the chain products, see kExactMass).  A workgroup covers the 64 rows of one
// block: the keys of its own block are summed exactly (j < i), the earlier keys are
// sampled, at most 128 keys spread evenly over the earlier 64-blocks (one key per block
// at a row offset that varies with the row block), each weighted by the number of
// earlier keys it stands for.  Each wave takes 32-key chunks as the transposed score tile
//   S^T[j][i] = K_j . K_i (lane <-> row i, the 16 values of a lane over keys j),
//   P = exp(s r_i r_j S - 1/s),
// so that a row's sum is taken inside its lanes (16 values, then the two lane halves).
// The block's largest row total goes to mass[bh] by an integer max of the (non-negative)
// float bits.  After lucid_prep_kernel (1/rms, mass[bh] = 0); run per 64-row block by the
// 256 threads of a workgroup (lucid_mass_kernel: grid (T/64, B*Hkv); lucid_zx_kernel runs
// it for the two blocks of its 128 rows when given `mass`).
// ---------------------------------------------------------------------------
template <int D>
__device__ __forceinline__ void row_mass_block(const bf16* __restrict__ k, Strides ks, int Hkv, int T,
                                               const float* __restrict__ rinv, float scale, float* __restrict__ mass,
                                               int blk, int bh) {
  constexpr int NKS = D / 16;
  __shared__ float part[4][64];
  __shared__ float kr[4][32];  // 1/rms of each wave's current 32 keys
  __shared__ float kw[4][32];  // their weights
  const int b = bh / Hkv, h = bh - b * Hkv;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int g = lane >> 5, l32 = lane & 31;
  const bf16* kp = k + b * ks.b + h * ks.h;
  const float* rv = rinv + (int64_t)bh * T;
  const int i0 = blk * 64;
  const float c0 = LOG2E_F / scale;
  bf16x8 kb[2][NKS];  // B operand: the block's rows (n-tiles of 32)
  float ri[2];        // s log2e / rms of this lane's rows
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
#pragma unroll
    for (int st = 0; st < NKS; ++st) kb[nt][st] = ld8(kp + (int64_t)(i0 + nt * 32 + l32) * ks.t + 16 * st + 8 * g);
    ri[nt] = rv[i0 + nt * 32 + l32] * scale * LOG2E_F;
  }
  float acc[2] = {0.f, 0.f};
  const int off = (blk * 29) & 63;           // sampled row inside a sampled block
  const int ns = min(blk, 128);              // sampled keys
  const int nchunk = 2 + (ns + 31) / 32;     // chunks 0, 1: own block; 2..: sampled
  const float wsample = ns ? 64.f * (float)blk / (float)ns : 0.f;
  for (int c = w; c < nchunk; c += 4) {
    const bool own = c < 2;
    const int n = 32 * (c - 2) + l32;        // this lane's sample (A-operand lane <-> key)
    const bool valid = own || n < ns;
    const int key = own ? i0 + 32 * c + l32 : (valid ? (int)(((int64_t)n * blk) / ns) : 0) * 64 + off;
    bf16x8 ka[NKS];
#pragma unroll
    for (int st = 0; st < NKS; ++st) ka[st] = ld8(kp + (int64_t)key * ks.t + 16 * st + 8 * g);
    if (g == 0) {
      kr[w][l32] = rv[key];
      kw[w][l32] = own ? 1.f : (valid ? wsample : 0.f);
    }
    __builtin_amdgcn_s_waitcnt(0);
    __builtin_amdgcn_wave_barrier();
    float rj[16], wj[16];
    lds_rows16(kr[w], g, rj);
    lds_rows16(kw[w], g, wj);
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      f32x16 sd = zero16();
#pragma unroll
      for (int st = 0; st < NKS; ++st) sd = mfma32(ka[st], kb[nt][st], sd);
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        float p = __builtin_amdgcn_exp2f(fmaf(sd[e] * ri[nt], rj[e], -c0));
        if (own && 32 * c + drow(e, g) >= nt * 32 + l32) p = 0.f;  // keys j < i only
        acc[nt] = fmaf(wj[e] * p, p, acc[nt]);
      }
    }
    __builtin_amdgcn_wave_barrier();  // every lane has read kr, kw before the next chunk writes them
  }
  // the two lane halves hold the two halves of each row's keys; then the sum over the waves
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    const float x = wave_sum32(acc[nt]);
    if (g == 0) part[w][nt * 32 + l32] = x;
  }
  __syncthreads();
  if (tid < 64) {
    float x = part[0][tid] + part[1][tid] + part[2][tid] + part[3][tid];
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) x = fmaxf(x, __shfl_xor(x, m, 64));
    if (tid == 0) atomicMax(reinterpret_cast<int*>(mass) + bh, __float_as_int(x));
  }
}

template <int D>
__global__ __launch_bounds__(256) void lucid_mass_kernel(const bf16* __restrict__ k, Strides ks, int Hkv, int T,
                                                         const float* __restrict__ rinv, float scale,
                                                         float* __restrict__ mass) {
  row_mass_block<D>(k, ks, Hkv, T, rinv, scale, mass, blockIdx.x, blockIdx.y);
}

// ---------------------------------------------------------------------------
// zx = -(X_B P_BA) for every 128-row chain block (A = its first 64 rows, B = the
// last 64; X_B = the inverse of P's diagonal block B from lucid_prep_kernel,
// P_BA[m][c] = exp(s r_m r_c K_m.K_c - 1/s)) (fp32 inputs: K.K over hi/lo with all four
// terms), columns in
// T-perm order so that the chain can add zx V'_A straight from its bf16 V'_A tile.
// wave -> 32x32 quadrant.  grid (T/128, B*Hkv)
// ---------------------------------------------------------------------------
template <int D, bool F32 = false>
__global__ __launch_bounds__(256) void lucid_zx_kernel(const bf16* __restrict__ k, Strides ks, int Hkv, int T,
                                                       const float* __restrict__ rinv, float scale,
                                                       const float* __restrict__ pinv, float* __restrict__ zx, Lo lo,
                                                       float* __restrict__ mass = nullptr) {
  constexpr int NKS = D / 16;
  __shared__ __attribute__((aligned(16))) float Xb[64][68];
  __shared__ __attribute__((aligned(16))) float PT[64][68];  // PT[c][m] = P_BA[m][c]
  const int blk = blockIdx.x, bh = blockIdx.y;
  const int b = bh / Hkv, h = bh - b * Hkv;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int g = lane >> 5, l32 = lane & 31;
  const int tm = w >> 1, tn = w & 1;
  const bf16* kp = k + b * ks.b + h * ks.h + (int64_t)blk * 128 * ks.t;  // A rows; B rows from 64 on
  const float* rv = rinv + (int64_t)bh * T + blk * 128;
  const float* xb = pinv + ((int64_t)bh * (T / 64) + 2 * blk + 1) * 4096;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int f = 4 * (tid + 256 * u);
    *reinterpret_cast<f32x4*>(&Xb[f >> 6][f & 63]) = *reinterpret_cast<const f32x4*>(xb + f);
  }
  {
    const float sl2 = scale * LOG2E_F;
    const float c0 = LOG2E_F / scale;
    f32x16 sd = zero16();
    const bf16* klp = F32 ? lo.k + b * ks.b + h * ks.h + (int64_t)blk * 128 * ks.t : nullptr;
#pragma unroll
    for (int st = 0; st < NKS; ++st) {
      const int64_t om = (int64_t)(64 + tm * 32 + l32) * ks.t + 16 * st + 8 * g;
      const int64_t on = (int64_t)(tn * 32 + l32) * ks.t + 16 * st + 8 * g;
      sd = mfma32(ld8(kp + om), ld8(kp + on), sd);
      if constexpr (F32) {
        sd = mfma32(ld8(kp + om), ld8(klp + on), sd);
        sd = mfma32(ld8(klp + om), ld8(kp + on), sd);
        sd = mfma32(ld8(klp + om), ld8(klp + on), sd);
      }
    }
    const int cc = tn * 32 + l32;
    const float ac = sl2 * rv[cc];
    float rm[16];
    load_rows16(rv + 64 + tm * 32, g, rm);
#pragma unroll
    for (int e = 0; e < 16; ++e) PT[cc][tm * 32 + drow(e, g)] = __builtin_amdgcn_exp2f(fmaf(sd[e] * ac, rm[e], -c0));
  }
  __syncthreads();
  f32x16 z = zero16();
#pragma unroll
  for (int st = 0; st < 4; ++st) {
    bf16x8 ah, al, bh8, bl;
    split8(&Xb[tm * 32 + l32][16 * st + 8 * g], ah, al);
    split8(&PT[tn * 32 + l32][16 * st + 8 * g], bh8, bl);
    z = mfma32(ah, bh8, z);
    z = mfma32(ah, bl, z);
    z = mfma32(al, bh8, z);
  }
  const int cc = tn * 32 + l32, slot = (cc & ~15) | jmap(cc & 15);
  float* zo = zx + ((int64_t)bh * (T / 128) + blk) * 4096 + slot;
#pragma unroll
  for (int e = 0; e < 16; ++e) zo[(tm * 32 + drow(e, g)) * 64] = -z[e];
  if constexpr (!F32) {
    if (mass) {  // the row masses of the two 64-row blocks (one launch less than lucid_mass_kernel)
      row_mass_block<D>(k, ks, Hkv, T, rinv, scale, mass, 2 * blk, bh);
      __syncthreads();
      row_mass_block<D>(k, ks, Hkv, T, rinv, scale, mass, 2 * blk + 1, bh);
    }
  }
}

// ---------------------------------------------------------------------------
// Chained preconditioner solve, 128 rows per workgroup made of two 64-row
// sub-blocks A (rows i0..i0+63) and B (i0+64..i0+127).
// Workgroup id -> (i2 = id / BH, bh = id % BH): ids grow with i2, so every
// wait is on a lower id (in-order dispatch keeps the chain deadlock free) and
// the blocks of one head share an XCD when BH % 8 == 0.  counters[bh] = number
// of 64-row blocks of V' already published (whole 128-row blocks at a time).
//
// The earlier keys are swept in pairs of 64-key tiles (128 keys per barrier):
// K^ rows (bf16, the bf16 chains; raw K rows and 1/rms, the exact ones) and V'^T (T-perm)
// of the pair are staged once per workgroup in LDS by direct global->LDS loads (double
// buffered, swizzled, no registers).
// wave w: ih = w & 1 -> rows i0 + 64*ih .. +64 (two 32-row n-tiles, lane <-> row)
//         kh = w >> 1 -> the 64-key tile 2*pair + kh of every staged pair
//   acc^T[d][i] += V'^T[d][j] P^T[j][i],  P^T[j][i] = exp(s r_i r_j K_j.K_i - 1/s)
// (the kh = 0 accumulators start at -V^T).  Then V'_A = X_A R_A and
// V'_B = X_B R_B + Z V'_A with Z = -(X_B P_BA), R = V - acc, X = P_diag^-1 (fp32, both
// from lucid_prep_kernel) applied through a 3-term bf16 split (hi*hi + hi*lo + lo*hi),
// Z through a 2-term split against bf16 V'_A.  The chain's critical path is the work
// after the last pair becomes visible, so everything that does not depend on it (V,
// the two inverses, Z) is loaded earlier.  At d = 64 two workgroups share a CU (LDS <= 80 KB,
// <= 256 registers per lane) so that one's MFMA work overlaps the other's exp.  At d = 128
// the bf16 chain runs NW = 8 waves (two per SIMD, 220 registers): wave w owns the 32 rows
// i0 + 32 (w % 4) .. of key half w / 4 (one n-tile instead of two), one solve tile each.
//
// EXACT (heads whose row mass exceeds kExactMass; the other instance returns at once for
// them and vice versa): V' is also kept as its bf16 residual lo = bf16(V' - bf16(V'))
// (vpbl row-major, vptl T-perm), the staged pairs carry the lo tile too, and every
// off-diagonal product is split: P V' ~= Ph Vh + Pl Vh + Ph Vl, as is Z V'_A.  The
// extra tile and registers allow one workgroup per CU; at d = 128 the staged pairs are
// single-buffered (three 32 KB tiles), each pair staged after the previous one's sweep.
// ---------------------------------------------------------------------------
template <int D, bool EXACT, bool F32 = false>
struct PfwdSmem;
template <int D>
struct PfwdSmem<D, false, false> {
  union {
    struct {
      bf16 k[2][128 * D];  // swizzled tiles (chunk c of row r at c ^ (r & 7))
      bf16 v[2][D * 128];
      float r[2][128];
    } st;
    struct {
      float Rt[D][132];     // R^T for the 128 rows (cols 0..63 = A, 64..127 = B)
      float X[64][68];      // inverse of the diagonal block being solved
      bf16 vT[D][128 + 8];  // V'^T of the block (bf16, T-perm within 16-groups)
    } fin;
  } u;
};
template <int D, bool F32>
struct PfwdSmem<D, true, F32> {
  static constexpr int NBUF = D == 128 ? 1 : 2;
  union {
    struct {
      bf16 k[NBUF][128 * D];
      bf16 kl[F32 ? NBUF : 1][F32 ? 128 * D : 8];  // lo part of K (fp32 inputs)
      bf16 v[NBUF][D * 128];
      bf16 vl[NBUF][D * 128];  // lo part of V'^T
      float r[NBUF][128];
    } st;
    struct {
      float Rt[D][132];
      float X[64][68];
      bf16 vT[D][128 + 8];
      bf16 vTl[D][128 + 8];  // lo part of V'^T of the block
    } fin;
  } u;
};

template <int D, bool EXACT, bool F32 = false, int NW = 4>
__global__ __launch_bounds__(64 * NW) LUCID_TWO_WAVES_IF((D == 64 || NW == 8) && !EXACT) void lucid_precond_fwd_kernel(
    const bf16* __restrict__ k, Strides ks, const bf16* __restrict__ v, Strides vs, int Hkv, int T, int BH,
    const float* __restrict__ rinv, const bf16* __restrict__ khat, float scale, float* __restrict__ vp32,
    bf16* __restrict__ vpb,
    bf16* __restrict__ vpt, bf16* __restrict__ vpbl, bf16* __restrict__ vptl, float* __restrict__ pinv,
    const float* __restrict__ zx, const float* __restrict__ mass, int* __restrict__ counters, Lo lo) {
  static_assert(EXACT || !F32, "fp32 inputs run the exact chains");
  static_assert(NW == 4 || (NW == 8 && D == 128 && !EXACT), "eight waves: the bf16 chain at head dim 128");
  constexpr int NDT = D / 32;
  constexpr int NKS = D / 16;
  constexpr int NTHR = 64 * NW;
  constexpr int NTW = 8 / NW;            // 32-row n-tiles per wave (two with four waves, one with eight)
  constexpr int RQ = NW / 2;             // row groups (waves per key half)
  constexpr bool SINGLE = EXACT && D == 128;  // one staging buffer
  __shared__ __attribute__((aligned(16))) PfwdSmem<D, EXACT, F32> sm;

  const int id = blockIdx.x;
  const int i2 = id / BH, bh = id - (id / BH) * BH;
  if ((mass[bh] > kExactMass) != EXACT) return;  // the other instance solves this head
  const int b = bh / Hkv, h = bh - b * Hkv;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int g = lane >> 5, l32 = lane & 31;
  const int ih = w % RQ, kh = w / RQ;  // rows i0 + 32 NTW ih .. (+32 NTW), key half kh of each pair
  const int i0 = i2 * 128;
  const int NT = T / 64;
  const bf16* kp = k + b * ks.b + h * ks.h;
  const bf16* vh = v + b * vs.b + h * vs.h;
  const float* rv = rinv + (int64_t)bh * T;
  const bf16* vpth = vpt + (int64_t)bh * D * T;
  const bf16* vptlh = vptl + (int64_t)bh * D * T;
  const float* pinv_blk = pinv + ((int64_t)bh * NT + 2 * i2) * 4096;
  int* cnt = counters + bh;
  const float sl2 = scale * LOG2E_F;
  const float c0 = LOG2E_F / scale;

  // bf16 chain: K^ tiles (khat) against the row keys scaled by s log2(e) r_i (one bf16
  // rounding), so that an MFMA gives the exponent E = s log2(e) r_i r_j K_i.K_j; P = exp2(E - c0)
  // = C exp2(E) with C = 2^-c0, so the sweep takes exp2(E) and the accumulators carry a factor
  // 1/C (they start at -V / C; R is multiplied by C).  The exact instance keeps raw K tiles and
  // the fp32 factors r_i r_j.
  const bf16* khh = EXACT ? nullptr : khat + (int64_t)bh * T * D;
  const float Cf = EXACT ? 1.f : __builtin_amdgcn_exp2f(-c0);
  const float invC = EXACT ? 1.f : __builtin_amdgcn_exp2f(c0);
  const bf16* klh = F32 ? lo.k + b * ks.b + h * ks.h : nullptr;
  bf16x8 kbi[NTW][NKS], kbil[NTW][NKS];
  float ai[NTW];
#pragma unroll
  for (int nt = 0; nt < NTW; ++nt) {
    const int row = i0 + ih * 32 * NTW + nt * 32 + l32;
    ai[nt] = sl2 * rv[row];
#pragma unroll
    for (int st = 0; st < NKS; ++st) {
      const bf16x8 kr = ld8(kp + (int64_t)row * ks.t + 16 * st + 8 * g);
      kbi[nt][st] = EXACT ? kr : scale8(kr, ai[nt]);
      if constexpr (F32) kbil[nt][st] = ld8(klh + (int64_t)row * ks.t + 16 * st + 8 * g);
    }
  }
  // accumulators: -V^T (/ C) for the kh = 0 waves, zero for the others
  f32x16 acc[NDT][NTW];
#pragma unroll
  for (int nt = 0; nt < NTW; ++nt) {
    const int64_t roff = (int64_t)(i0 + ih * 32 * NTW + nt * 32 + l32) * vs.t;
    const bf16* vrow = vh + roff;
#pragma unroll
    for (int t = 0; t < NDT; ++t)
#pragma unroll
      for (int qd = 0; qd < 4; ++qd) {
        float vv[4];
        if constexpr (F32) {  // the fp32 right-hand side itself
          const f32x4 x = *reinterpret_cast<const f32x4*>(lo.v + b * vs.b + h * vs.h + roff + t * 32 + 8 * qd + 4 * g);
#pragma unroll
          for (int u = 0; u < 4; ++u) vv[u] = x[u];
        } else {
          const bf16x4 x = *reinterpret_cast<const bf16x4*>(vrow + t * 32 + 8 * qd + 4 * g);
#pragma unroll
          for (int u = 0; u < 4; ++u) vv[u] = (float)x[u];
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) acc[t][nt][4 * qd + u] = kh ? 0.f : -vv[u] * invC;
      }
  }

  // ---- off-diagonal sweep over the i2 earlier pairs of 64-key tiles ----
  // pair pp (keys 128pp .. 128pp+127) is complete once the counter exceeds 2pp+1;
  // it is staged into buffer pp & 1 by direct global->LDS loads
  const int npair = i2;
  int ready = 0;
  int plan_k[128 * (D / 8) / NTHR], plan_v[D * 16 / NTHR];
  dma_plan<128, D / 8, NTHR>(EXACT ? ks.t : (int64_t)D, plan_k);
  dma_plan<D, 16, NTHR>(T, plan_v);
  auto stage = [&](int pp) {
    const int buf = SINGLE ? 0 : pp & 1;
    if constexpr (EXACT) {
      if (w < 2) dma_f32x64(rv + pp * 128 + 64 * w, &sm.u.st.r[buf][64 * w]);
      dma_stage<128, D / 8, NTHR>(plan_k, kp + (int64_t)pp * 128 * ks.t, sm.u.st.k[buf]);
    } else {
      dma_stage<128, D / 8, NTHR>(plan_k, khh + (int64_t)pp * 128 * D, sm.u.st.k[buf]);
    }
    if constexpr (F32) dma_stage<128, D / 8, NTHR>(plan_k, klh + (int64_t)pp * 128 * ks.t, sm.u.st.kl[buf]);
    dma_stage<D, 16, NTHR>(plan_v, vpth + pp * 128, sm.u.st.v[buf]);
    if constexpr (EXACT) dma_stage<D, 16, NTHR>(plan_v, vptlh + pp * 128, sm.u.st.vl[buf]);
  };
  // the two inverses X_A, X_B (2 x 64 x 64 fp32): chunk u -> sub-block u / XH
  constexpr int XPER = 2048 / NTHR, XH = XPER / 2;  // 16-byte chunks per thread, per sub-block
  f32x4 xr[XPER];
  auto xload = [&]() {
#pragma unroll
    for (int u = 0; u < XPER; ++u) {
      const int idx = tid + NTHR * u;
      const int sb = idx >> 10, r = (idx >> 4) & 63, c4 = (idx & 15) * 4;
      xr[u] = *reinterpret_cast<const f32x4*>(pinv_blk + sb * 4096 + r * 64 + c4);
    }
  };
  auto xstore = [&](int sb) {
#pragma unroll
    for (int u = XH * sb; u < XH * sb + XH; ++u) {
      const int idx = tid + NTHR * u;
      const int r = (idx >> 4) & 63, c4 = (idx & 15) * 4;
      *reinterpret_cast<f32x4*>(&sm.u.fin.X[r][c4]) = xr[u];
    }
  };
  auto sweep_pair = [&](int buf) {
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      const int key0 = kh * 64 + mt * 32;
      bf16x8 ka[NKS];
#pragma unroll
      for (int st = 0; st < NKS; ++st) ka[st] = ld8(swz<D / 8>(sm.u.st.k[buf], key0 + l32, 2 * st + g));
      float rj[16];
      if constexpr (EXACT) lds_rows16(&sm.u.st.r[buf][key0], g, rj);
      bf16x8 pb[NTW][2], pbl[NTW][2];
#pragma unroll
      for (int nt = 0; nt < NTW; ++nt) {
        f32x16 sc = zero16();
#pragma unroll
        for (int st = 0; st < NKS; ++st) sc = mfma32(ka[st], kbi[nt][st], sc);
        if constexpr (F32) {
#pragma unroll
          for (int st = 0; st < NKS; ++st) {
            const bf16x8 kal = ld8(swz<D / 8>(sm.u.st.kl[buf], key0 + l32, 2 * st + g));
            sc = mfma32(ka[st], kbil[nt][st], sc);
            sc = mfma32(kal, kbi[nt][st], sc);
            sc = mfma32(kal, kbil[nt][st], sc);
          }
        }
#pragma unroll
        for (int e = 0; e < 16; ++e)
          sc[e] = __builtin_amdgcn_exp2f(EXACT ? fmaf(sc[e] * ai[nt], rj[e], -c0) : sc[e]);
        pb[nt][0] = pack_b(sc, 0);
        pb[nt][1] = pack_b(sc, 1);
        if constexpr (EXACT) {
          pbl[nt][0] = pack_lo(sc, 0, pb[nt][0]);
          pbl[nt][1] = pack_lo(sc, 1, pb[nt][1]);
        }
      }
#pragma unroll
      for (int t = 0; t < NDT; ++t) {
        const bf16x8 va0 = ld8(swz<16>(sm.u.st.v[buf], t * 32 + l32, key0 / 8 + g));
        const bf16x8 va1 = ld8(swz<16>(sm.u.st.v[buf], t * 32 + l32, key0 / 8 + 2 + g));
#pragma unroll
        for (int nt = 0; nt < NTW; ++nt) {
          acc[t][nt] = mfma32(va0, pb[nt][0], acc[t][nt]);
          acc[t][nt] = mfma32(va1, pb[nt][1], acc[t][nt]);
        }
        if constexpr (EXACT) {
          const bf16x8 vl0 = ld8(swz<16>(sm.u.st.vl[buf], t * 32 + l32, key0 / 8 + g));
          const bf16x8 vl1 = ld8(swz<16>(sm.u.st.vl[buf], t * 32 + l32, key0 / 8 + 2 + g));
#pragma unroll
          for (int nt = 0; nt < NTW; ++nt) {
            acc[t][nt] = mfma32(va0, pbl[nt][0], acc[t][nt]);
            acc[t][nt] = mfma32(va1, pbl[nt][1], acc[t][nt]);
            acc[t][nt] = mfma32(vl0, pb[nt][0], acc[t][nt]);
            acc[t][nt] = mfma32(vl1, pb[nt][1], acc[t][nt]);
          }
        }
      }
    }
  };
  if (npair > 0) {
    ready = wait_counter_gt(cnt, 1);
    stage(0);
    dma_wait();
  } else {
    xload();
  }
  __syncthreads();
  // all pairs but the last; the last one is peeled so that the inverses it
  // prefetches do not hold registers through the loop
  for (int pp = 0; pp + 1 < npair; ++pp) {
    const int need = 2 * pp + 3;  // pair pp + 1 is complete once the counter exceeds this
    if constexpr (SINGLE) {
      sweep_pair(0);
      __syncthreads();  // every wave is done with the buffer
      if (need >= ready) ready = wait_counter_gt(cnt, need);
      stage(pp + 1);
      dma_wait();
      __syncthreads();
      continue;
    }
    if (need >= ready) {
      const int seen = poll_counter(cnt);
      if (seen > need) {
        chain_acquire();
        ready = seen;
      }
    }
    const bool early = need < ready;
    if (early) stage(pp + 1);
    sweep_pair(pp & 1);
    if (!early) {
      ready = wait_counter_gt(cnt, need);
      stage(pp + 1);
    }
    dma_wait();
    __syncthreads();
  }
  if (npair > 0) {
    xload();  // fetch the inverses while the last pair is processed
    sweep_pair(SINGLE ? 0 : (npair - 1) & 1);
    __syncthreads();
  }

  // ---- reduce the key halves: R^T = -(acc_0 + acc_1) (Rt columns = rows of this workgroup) ----
  float(*Rt)[132] = sm.u.fin.Rt;
  if (kh == 1) {
#pragma unroll
    for (int t = 0; t < NDT; ++t)
#pragma unroll
      for (int nt = 0; nt < NTW; ++nt)
#pragma unroll
        for (int e = 0; e < 16; ++e) Rt[t * 32 + drow(e, g)][ih * 32 * NTW + nt * 32 + l32] = acc[t][nt][e];
  }
  xstore(0);
  __syncthreads();
  if (kh == 0) {
#pragma unroll
    for (int t = 0; t < NDT; ++t)
#pragma unroll
      for (int nt = 0; nt < NTW; ++nt)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          float& x = Rt[t * 32 + drow(e, g)][ih * 32 * NTW + nt * 32 + l32];
          x = -Cf * (acc[t][nt][e] + x);
        }
  }
  // Z rows of this wave's B output tiles (row half rh = w & 1), 8 columns per lane half and
  // 16-column step, fetched while sub-block A is solved
  f32x4 zr[4][2];
  {
    const float* zrow = zx + ((int64_t)bh * (T / 128) + i2) * 4096 + ((w & 1) * 32 + l32) * 64 + 8 * g;
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      zr[st][0] = *reinterpret_cast<const f32x4*>(zrow + 16 * st);
      zr[st][1] = *reinterpret_cast<const f32x4*>(zrow + 16 * st + 4);
    }
  }
  __syncthreads();

  // V'^T[d][r] = sum_c R^T[d][c] X[r][c] for sub-block sb (X lower triangular)
  auto diag_solve = [&](int sb) {
    for (int tile = w; tile < NDT * 2; tile += NW) {
      const int dt = tile >> 1, rh = tile & 1;
      f32x16 o = zero16();
      const int kmax = rh ? 4 : 2;
      for (int st = 0; st < kmax; ++st) {
        bf16x8 ah, al, bh8, bl;
        split8(&Rt[dt * 32 + l32][sb * 64 + 16 * st + 8 * g], ah, al);
        split8(&sm.u.fin.X[rh * 32 + l32][16 * st + 8 * g], bh8, bl);
        o = mfma32(ah, bh8, o);
        o = mfma32(ah, bl, o);
        o = mfma32(al, bh8, o);
      }
      if (sb == 1) {  // + Z V'_A: V'_A^T from the bf16 T-perm tile, Z split into hi + lo
#pragma unroll
        for (int st = 0; st < 4; ++st) {
          bf16x8 zh, zl;
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float x = zr[st][e >> 2][e & 3];
            zh[e] = (bf16)x;
            zl[e] = (bf16)(x - (float)zh[e]);
          }
          const bf16x8 va = ld8(&sm.u.fin.vT[dt * 32 + l32][16 * st + 8 * g]);
          o = mfma32(va, zh, o);
          o = mfma32(va, zl, o);
          if constexpr (EXACT) o = mfma32(ld8(&sm.u.fin.vTl[dt * 32 + l32][16 * st + 8 * g]), zh, o);
        }
      }
      const int rl = rh * 32 + l32;
      const int r = i0 + sb * 64 + rl;
      const int lslot = sb * 64 + ((rl & ~15) | jmap(rl & 15));
      float* out32 = vp32 + ((int64_t)bh * T + r) * D;
      bf16* outb = vpb + ((int64_t)bh * T + r) * D;
#pragma unroll
      for (int qd = 0; qd < 4; ++qd) {
        const int d0 = dt * 32 + 8 * qd + 4 * g;
        f32x4 f;
        bf16x4 bb, bl;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          f[u] = o[4 * qd + u];
          bb[u] = (bf16)o[4 * qd + u];
          sm.u.fin.vT[d0 + u][lslot] = bb[u];
          if constexpr (EXACT) {
            bl[u] = (bf16)(o[4 * qd + u] - (float)bb[u]);
            sm.u.fin.vTl[d0 + u][lslot] = bl[u];
          }
        }
        *reinterpret_cast<f32x4*>(out32 + d0) = f;
        *reinterpret_cast<bf16x4*>(outb + d0) = bb;
        if constexpr (EXACT) *reinterpret_cast<bf16x4*>(vpbl + ((int64_t)bh * T + r) * D + d0) = bl;
      }
    }
  };
  diag_solve(0);
  __syncthreads();
  xstore(1);
  __syncthreads();
  diag_solve(1);
  __syncthreads();
  // V'^T of the whole block to the T-perm operand copy: 16-byte stores
  for (int c = tid; c < D * 16; c += NTHR) {
    const int dd = c >> 4, s8 = (c & 15) * 8;
    *reinterpret_cast<bf16x8*>(vpt + ((int64_t)bh * D + dd) * T + i0 + s8) = ld8(&sm.u.fin.vT[dd][s8]);
    if constexpr (EXACT)
      *reinterpret_cast<bf16x8*>(vptl + ((int64_t)bh * D + dd) * T + i0 + s8) = ld8(&sm.u.fin.vTl[dd][s8]);
  }
  publish_counter(cnt, 2 * i2 + 2);
}

// ---------------------------------------------------------------------------
// Causal attention on V'.  Workgroup = 256 query rows of one query head
// (heavy, late row blocks first); wave w owns rows 64w .. 64w+63 as two
// 32-row n-tiles (lane <-> row).  Every 64-key tile of K and V'^T is staged
// once per workgroup in LDS (double buffered, loaded one tile ahead with
// coalesced 16-byte global loads) and read by all four waves.
//   S^T[j][i] = K_j . Q_i;  online softmax per lane (lazy rescale: the
//   reference max only moves when a row grows by more than 2^8);
//   O^T[d][i] += V'^T[d][j] P^T[j][i].
// Writes O (bf16, caller layout) and lse2[bhq][i] (log2 domain, so that
// P = exp2(s*log2e*S - lse2)).  For heads that run the exact chains (row mass above
// kExactMass) it also writes O's bf16 residual olo[bhq][i][d] = bf16(O - bf16(O)): the
// backward's delta_i = dO_i . O_i enters dQ_i = s sum_j dS_ij K_j multiplied by the
// attention-weighted mean key, which is large when keys share a direction.
// ---------------------------------------------------------------------------
// NT: 32-row n-tiles per wave (2: 256 rows per workgroup; 1: 128 rows, for the fp32
// instance at head dim 128, whose hi/lo operands of two n-tiles do not fit the registers)
// DA: the head-dim columns that can be nonzero (a multiple of 16, <= D): rows of a smaller
// head dim are zero-padded to D, and the products skip the k-steps and value tiles that
// would only meet the zero columns (the outputs there stay 0)
template <int D, bool F32 = false, int NT = 2, int DA = D>
__global__ __launch_bounds__(256) LUCID_TWO_WAVES_IF(D == 64 && !F32) void lucid_attn_fwd_kernel(
    const bf16* __restrict__ q, Strides qs, const bf16* __restrict__ k, Strides ks, const bf16* __restrict__ vpt,
    std::conditional_t<F32, float, bf16>* __restrict__ o, Strides os, float* __restrict__ lse,
    const float* __restrict__ mass, bf16* __restrict__ olo, int Hq, int Hkv, int T, int BHq, float scale, Lo lo,
    const bf16* __restrict__ vptl, int skip_fast) {
  constexpr int NDT = D / 32;
  constexpr int NKS = D / 16;
  constexpr int NDT_A = (DA + 31) / 32, NKS_A = DA / 16;  // value tiles and k-steps that can be nonzero
  static_assert(DA % 16 == 0 && DA <= D && (DA == D || NT == 1), "active head dim");
  constexpr int CH = D / 32;  // 16-byte chunks per thread for each of the K and V'^T tiles
  constexpr int NST = F32 ? 4 * CH : 2 * CH;  // staging registers (fp32 inputs: hi and lo tiles)
  __shared__ __attribute__((aligned(16))) bf16 lk[2][64][D + 8];
  __shared__ __attribute__((aligned(16))) bf16 lv[2][D][64 + 8];
  __shared__ __attribute__((aligned(16))) bf16 lkl[F32 ? 2 : 1][F32 ? 64 : 1][D + 8];  // lo tiles (fp32 inputs)
  __shared__ __attribute__((aligned(16))) bf16 lvl[F32 ? 2 : 1][F32 ? D : 1][64 + 8];

  static_assert(NT == 2 || (NT == 1 && (D == 128 || F32)), "one n-tile per wave: the generic tile body only");
  constexpr int WGR = 128 * NT;  // rows per workgroup
  const int nblk = (T + WGR - 1) / WGR;
  const int id = blockIdx.x;
  const int bhq = id % BHq;
  const int ib = nblk - 1 - id / BHq;
  const int b = bhq / Hq, hq = bhq - b * Hq;
  const int h = hq / (Hq / Hkv);
  const int bh = b * Hkv + h;
  // skip_fast: the fused forward has already written O and lse for the heads of the bf16
  // chains; this launch covers the heads of the exact chains only
  if (skip_fast && !(mass[bh] > kExactMass)) return;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int g = lane >> 5, l32 = lane & 31;
  const int r0 = ib * WGR;
  const int row0 = r0 + w * 32 * NT;
  const bf16* qh = q + b * qs.b + hq * qs.h;
  const bf16* kh = k + b * ks.b + h * ks.h;
  const bf16* vth = vpt + (int64_t)bh * D * T;
  const bf16* qlh = F32 ? lo.q + b * qs.b + hq * qs.h : nullptr;
  const bf16* klh = F32 ? lo.k + b * ks.b + h * ks.h : nullptr;
  const bf16* vtlh = F32 ? vptl + (int64_t)bh * D * T : nullptr;
  const float c = scale * LOG2E_F;

  bf16x8 qb[NT][NKS], qbl[NT][NKS];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int rq = min(row0 + nt * 32 + l32, T - 1);
#pragma unroll
    for (int st = 0; st < NKS_A; ++st) {
      qb[nt][st] = ld8(qh + (int64_t)rq * qs.t + 16 * st + 8 * g);
      if constexpr (F32) qbl[nt][st] = ld8(qlh + (int64_t)rq * qs.t + 16 * st + 8 * g);
    }
  }
  f32x16 oacc[NDT][NT];
  float m[NT], lsum[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    m[nt] = -1e30f;
    lsum[nt] = 0.f;
#pragma unroll
    for (int t = 0; t < NDT; ++t) oacc[t][nt] = zero16();
  }

  const int ntile = (min(r0 + WGR, T) + 63) / 64;
  const int last_w = row0 / 64;         // this wave's diagonal tile
  const int roff = row0 - last_w * 64;  // this wave's first row inside it (32 at NT = 1 for odd waves)
  bf16x8 stg[NST];
  auto gload = [&](int j0) {
#pragma unroll
    for (int u = 0; u < CH; ++u) {
      const int cidx = tid + 256 * u;
      const int kr = cidx / (D / 8), kc = cidx % (D / 8);
      stg[u] = ld8(kh + (int64_t)(j0 + kr) * ks.t + kc * 8);
      const int vr = cidx >> 3, vc = cidx & 7;
      stg[CH + u] = ld8(vth + (int64_t)vr * T + j0 + vc * 8);
      if constexpr (F32) {
        stg[2 * CH + u] = ld8(klh + (int64_t)(j0 + kr) * ks.t + kc * 8);
        stg[3 * CH + u] = ld8(vtlh + (int64_t)vr * T + j0 + vc * 8);
      }
    }
  };
  auto lstore = [&](int buf) {
#pragma unroll
    for (int u = 0; u < CH; ++u) {
      const int cidx = tid + 256 * u;
      const int kr = cidx / (D / 8), kc = cidx % (D / 8);
      *reinterpret_cast<bf16x8*>(&lk[buf][kr][kc * 8]) = stg[u];
      const int vr = cidx >> 3, vc = cidx & 7;
      *reinterpret_cast<bf16x8*>(&lv[buf][vr][vc * 8]) = stg[CH + u];
      if constexpr (F32) {
        *reinterpret_cast<bf16x8*>(&lkl[buf][kr][kc * 8]) = stg[2 * CH + u];
        *reinterpret_cast<bf16x8*>(&lvl[buf][vr][vc * 8]) = stg[3 * CH + u];
      }
    }
  };
  gload(0);
  lstore(0);
  __syncthreads();
  for (int jt = 0; jt < ntile; ++jt) {
    const int buf = jt & 1;
    const bool more = jt + 1 < ntile;
    if (more) gload((jt + 1) * 64);
    if (jt <= last_w && row0 < T) {
      if constexpr (D == 64 && !F32 && NT == 2) {
        // Two 32-row halves (nt) per 64-key tile, staggered so that each half's softmax
        // VALU work overlaps the other half's MFMA work inside this wave:
        //   S(nt 0) | max(0) | S(nt 1) + exp(0) | max(1) | PV(nt 0) + exp(1) | PV(nt 1)
        const bool diag = jt == last_w;
        bf16x8 ka[2][NKS];
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
          for (int st = 0; st < NKS; ++st) ka[mt][st] = ld8(&lk[buf][mt * 32 + l32][16 * st + 8 * g]);
        f32x16 s[2][2];  // [nt][mt]
        auto sgemm = [&](int nt) {
#pragma unroll
          for (int mt = 0; mt < 2; ++mt) {
            s[nt][mt] = zero16();
#pragma unroll
            for (int st = 0; st < NKS; ++st) s[nt][mt] = mfma32(ka[mt][st], qb[nt][st], s[nt][mt]);
          }
        };
        // causal mask, row max and (lazy) rescale of half nt
        auto rowmax = [&](int nt) {
          if (diag) {
#pragma unroll
            for (int mt = 0; mt < 2; ++mt)
#pragma unroll
              for (int e = 0; e < 16; ++e)
                if (mt * 32 + drow(e, g) > nt * 32 + l32) s[nt][mt][e] = -INFINITY;
          }
          float mx = -INFINITY;
#pragma unroll
          for (int mt = 0; mt < 2; ++mt)
#pragma unroll
            for (int e = 0; e < 16; ++e) mx = fmaxf(mx, s[nt][mt][e]);
          mx = wave_max32(mx) * c;
          if (__builtin_amdgcn_ballot_w64(mx > m[nt] + 8.0f)) {
            const float mnew = fmaxf(m[nt], mx);
            const float alpha = __builtin_amdgcn_exp2f(m[nt] - mnew);
            m[nt] = mnew;
            lsum[nt] *= alpha;
#pragma unroll
            for (int t = 0; t < NDT; ++t)
#pragma unroll
              for (int e = 0; e < 16; ++e) oacc[t][nt][e] *= alpha;
          }
        };
        bf16x8 pb[2][4];
        auto softmax = [&](int nt) {
#pragma unroll
          for (int mt = 0; mt < 2; ++mt)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
              const float p = __builtin_amdgcn_exp2f(fmaf(s[nt][mt][e], c, -m[nt]));
              lsum[nt] += p;
              s[nt][mt][e] = p;
            }
          pb[nt][0] = pack_b(s[nt][0], 0);
          pb[nt][1] = pack_b(s[nt][0], 1);
          pb[nt][2] = pack_b(s[nt][1], 0);
          pb[nt][3] = pack_b(s[nt][1], 1);
        };
        auto pv = [&](int nt) {
#pragma unroll
          for (int t = 0; t < NDT; ++t)
#pragma unroll
            for (int k4 = 0; k4 < 4; ++k4)
              oacc[t][nt] = mfma32(ld8(&lv[buf][t * 32 + l32][16 * k4 + 8 * g]), pb[nt][k4], oacc[t][nt]);
        };
        sgemm(0);
        rowmax(0);
        sgemm(1);
        softmax(0);
        // half 0's P must be formed here, beside half 1's S products, and not sunk past
        // half 1's rescale branch into the block of its only use
#pragma unroll
        for (int k4 = 0; k4 < 4; ++k4) {
          const u32x4 pw = __builtin_bit_cast(u32x4, pb[0][k4]);
          asm volatile("" ::"v"(pw[0]), "v"(pw[1]), "v"(pw[2]), "v"(pw[3]));
        }
        rowmax(1);
        pv(0);
        softmax(1);
        pv(1);
      } else {  // D = 128 and fp32 inputs: both halves' products first (the staggered order spills)
        f32x16 s[2][NT];
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
          bf16x8 ka[NKS], kal[NKS];
#pragma unroll
          for (int st = 0; st < NKS_A; ++st) {
            ka[st] = ld8(&lk[buf][mt * 32 + l32][16 * st + 8 * g]);
            if constexpr (F32) kal[st] = ld8(&lkl[buf][mt * 32 + l32][16 * st + 8 * g]);
          }
#pragma unroll
          for (int nt = 0; nt < NT; ++nt) {
            s[mt][nt] = zero16();
#pragma unroll
            for (int st = 0; st < NKS_A; ++st) {
              s[mt][nt] = mfma32(ka[st], qb[nt][st], s[mt][nt]);
              if constexpr (F32) {
                s[mt][nt] = mfma32(ka[st], qbl[nt][st], s[mt][nt]);
                s[mt][nt] = mfma32(kal[st], qb[nt][st], s[mt][nt]);
                s[mt][nt] = mfma32(kal[st], qbl[nt][st], s[mt][nt]);
              }
            }
          }
        }
        if (jt == last_w) {
#pragma unroll
          for (int mt = 0; mt < 2; ++mt)
#pragma unroll
            for (int nt = 0; nt < NT; ++nt)
#pragma unroll
              for (int e = 0; e < 16; ++e)
                if (mt * 32 + drow(e, g) > roff + nt * 32 + l32) s[mt][nt][e] = -INFINITY;
        }
        bf16x8 pb[NT][4], pbl[NT][4];
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          float mx = -INFINITY;
#pragma unroll
          for (int mt = 0; mt < 2; ++mt)
#pragma unroll
            for (int e = 0; e < 16; ++e) mx = fmaxf(mx, s[mt][nt][e]);
          mx = wave_max32(mx) * c;
          if (__builtin_amdgcn_ballot_w64(mx > m[nt] + 8.0f)) {
            const float mnew = fmaxf(m[nt], mx);
            const float alpha = __builtin_amdgcn_exp2f(m[nt] - mnew);
            m[nt] = mnew;
            lsum[nt] *= alpha;
#pragma unroll
            for (int t = 0; t < NDT_A; ++t)
#pragma unroll
              for (int e = 0; e < 16; ++e) oacc[t][nt][e] *= alpha;
          }
#pragma unroll
          for (int mt = 0; mt < 2; ++mt)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
              const float p = __builtin_amdgcn_exp2f(fmaf(s[mt][nt][e], c, -m[nt]));
              lsum[nt] += p;
              s[mt][nt][e] = p;
            }
          pb[nt][0] = pack_b(s[0][nt], 0);
          pb[nt][1] = pack_b(s[0][nt], 1);
          pb[nt][2] = pack_b(s[1][nt], 0);
          pb[nt][3] = pack_b(s[1][nt], 1);
          if constexpr (F32) {
            pbl[nt][0] = pack_lo(s[0][nt], 0, pb[nt][0]);
            pbl[nt][1] = pack_lo(s[0][nt], 1, pb[nt][1]);
            pbl[nt][2] = pack_lo(s[1][nt], 0, pb[nt][2]);
            pbl[nt][3] = pack_lo(s[1][nt], 1, pb[nt][3]);
          }
        }
#pragma unroll
        for (int t = 0; t < NDT_A; ++t) {
          bf16x8 va[4];
#pragma unroll
          for (int k4 = 0; k4 < 4; ++k4) va[k4] = ld8(&lv[buf][t * 32 + l32][16 * k4 + 8 * g]);
#pragma unroll
          for (int nt = 0; nt < NT; ++nt)
#pragma unroll
            for (int k4 = 0; k4 < 4; ++k4) oacc[t][nt] = mfma32(va[k4], pb[nt][k4], oacc[t][nt]);
          if constexpr (F32) {
#pragma unroll
            for (int k4 = 0; k4 < 4; ++k4) {
              const bf16x8 val = ld8(&lvl[buf][t * 32 + l32][16 * k4 + 8 * g]);
#pragma unroll
              for (int nt = 0; nt < NT; ++nt) {
                oacc[t][nt] = mfma32(va[k4], pbl[nt][k4], oacc[t][nt]);
                oacc[t][nt] = mfma32(val, pb[nt][k4], oacc[t][nt]);
              }
            }
          }
        }
      }
    }
    if (more) lstore(buf ^ 1);
    __syncthreads();
  }
  const bool exact = !F32 && mass[bh] > kExactMass;  // fp32 O needs no lo part
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int irow = row0 + nt * 32 + l32;
    const float ls = wave_sum32(lsum[nt]);
    if (irow < T) {
      const float inv = 1.0f / ls;
      auto* op = o + b * os.b + hq * os.h + (int64_t)irow * os.t;
      bf16* ol = olo + ((int64_t)bhq * T + irow) * D;
#pragma unroll
      for (int t = 0; t < NDT; ++t)
#pragma unroll
        for (int qq = 0; qq < 4; ++qq) {
          if constexpr (F32) {
            f32x4 x;
#pragma unroll
            for (int u = 0; u < 4; ++u) x[u] = oacc[t][nt][4 * qq + u] * inv;
            *reinterpret_cast<f32x4*>(op + t * 32 + 8 * qq + 4 * g) = x;
          } else {
            bf16x4 bb, bl;
#pragma unroll
            for (int u = 0; u < 4; ++u) {
              const float x = oacc[t][nt][4 * qq + u] * inv;
              bb[u] = (bf16)x;
              bl[u] = (bf16)(x - (float)bb[u]);
            }
            *reinterpret_cast<bf16x4*>(op + t * 32 + 8 * qq + 4 * g) = bb;
            if (exact) *reinterpret_cast<bf16x4*>(ol + t * 32 + 8 * qq + 4 * g) = bl;
          }
        }
      if (g == 0) lse[(int64_t)bhq * T + irow] = m[nt] + log2f(ls);
    }
  }
}

// ---------------------------------------------------------------------------
// The bf16 forward chain at head dim 128 with 256 rows (two 128-row blocks 2p, 2p + 1) per
// workgroup, for T a multiple of 256: eight waves, wave w owns rows i0 + 32w .. +32 (block
// 2p: waves 0..3, block 2p + 1: waves 4..7) and sweeps all 128 keys of every staged pair, so
// that each staged pair (K^ rows, V'^T) serves 256 rows and a head's earlier pairs are
// fetched half as often (at this head dim the chain streams them from HBM).  After the sweep
// over the pairs before block 2p, block 2p is solved and published as in
// lucid_precond_fwd_kernel; then its K^ rows are staged and, with its V'^T from the solve's
// LDS copy, swept once more by the waves of block 2p + 1, which is solved and published in
// turn.  Heads of the exact chains return at once (lucid_precond_fwd_kernel<D, true>).
// ---------------------------------------------------------------------------
template <int D>
struct PfwdWideSmem {
  union {
    struct {
      bf16 k[2][128 * D];  // staged K^ rows of a pair (swizzled, chunk c of row r at c ^ (r & 7))
      bf16 v[2][D * 128];  // staged V'^T of a pair (T-perm rows, swizzled)
    } st;
    struct {
      float Rt[D][132];     // R^T of the block being solved (cols 0..63 = first sub-block)
      float X[64][68];      // inverse of the diagonal sub-block being solved
      bf16 vT[D][128 + 8];  // V'^T of the block just solved (bf16, T-perm within 16-groups)
    } fin;
  } u;
};

template <int D>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2))) void lucid_precond_fwd_wide_kernel(
    const bf16* __restrict__ k, Strides ks, const bf16* __restrict__ v, Strides vs, int Hkv, int T, int BH,
    const float* __restrict__ rinv, const bf16* __restrict__ khat, float scale, float* __restrict__ vp32,
    bf16* __restrict__ vpb, bf16* __restrict__ vpt, const float* __restrict__ pinv, const float* __restrict__ zx,
    const float* __restrict__ mass, int* __restrict__ counters) {
  static_assert(D == 128, "wide forward chain: head dim 128");
  constexpr int NDT = D / 32;
  constexpr int NKS = D / 16;
  constexpr int NTHR = 512;
  __shared__ __attribute__((aligned(16))) PfwdWideSmem<D> sm;
  static_assert(sizeof(bf16) * 128 * D <= sizeof(sm.u.fin.Rt), "block K^ rows must fit in R^T's bytes");

  const int id = blockIdx.x;
  const int p = id / BH, bh = id - (id / BH) * BH;  // ids grow with p: every wait is on a lower id
  if (mass[bh] > kExactMass) return;  // the exact instance of lucid_precond_fwd_kernel solves this head
  const int b = bh / Hkv, h = bh - b * Hkv;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int g = lane >> 5, l32 = lane & 31;
  const int i0 = p * 256;
  const int NT = T / 64;
  const int row = i0 + 32 * w + l32;  // this lane's row
  const bf16* kp = k + b * ks.b + h * ks.h;
  const bf16* vh = v + b * vs.b + h * vs.h;
  const float* rv = rinv + (int64_t)bh * T;
  const bf16* khh = khat + (int64_t)bh * T * D;
  const bf16* vpth = vpt + (int64_t)bh * D * T;
  int* cnt = counters + bh;
  const float sl2 = scale * LOG2E_F;
  const float c0 = LOG2E_F / scale;
  // as in lucid_precond_fwd_kernel's bf16 instance: K^ tiles against the row key scaled by
  // s log2(e) r_i, and P = exp2(E - c0) = C exp2(E): the accumulators carry a factor 1/C
  const float Cf = __builtin_amdgcn_exp2f(-c0), invC = __builtin_amdgcn_exp2f(c0);
  const float ai = sl2 * rv[row];
  bf16x8 kbi[NKS];
#pragma unroll
  for (int st = 0; st < NKS; ++st) kbi[st] = scale8(ld8(kp + (int64_t)row * ks.t + 16 * st + 8 * g), ai);
  f32x16 acc[NDT];  // -V^T / C
#pragma unroll
  for (int t = 0; t < NDT; ++t)
#pragma unroll
    for (int qd = 0; qd < 4; ++qd) {
      const bf16x4 x = *reinterpret_cast<const bf16x4*>(vh + (int64_t)row * vs.t + t * 32 + 8 * qd + 4 * g);
#pragma unroll
      for (int u = 0; u < 4; ++u) acc[t][4 * qd + u] = -(float)x[u] * invC;
    }

  int plan_k[128 * (D / 8) / NTHR], plan_v[D * 16 / NTHR];
  dma_plan<128, D / 8, NTHR>(D, plan_k);
  dma_plan<D, 16, NTHR>(T, plan_v);
  auto stage = [&](int pp) {
    const int buf = pp & 1;
    dma_stage<128, D / 8, NTHR>(plan_k, khh + (int64_t)pp * 128 * D, sm.u.st.k[buf]);
    dma_stage<D, 16, NTHR>(plan_v, vpth + pp * 128, sm.u.st.v[buf]);
  };
  // all 128 keys of a pair: K^ rows tk (staged layout), V'^T through vop(t, chunk)
  auto sweep_keys = [&](const bf16* tk, auto vop) {
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      const int key0 = mt * 32;
      f32x16 sc = zero16();
#pragma unroll
      for (int st = 0; st < NKS; ++st) sc = mfma32(ld8(swz<D / 8>(tk, key0 + l32, 2 * st + g)), kbi[st], sc);
#pragma unroll
      for (int e = 0; e < 16; ++e) sc[e] = __builtin_amdgcn_exp2f(sc[e]);
      const bf16x8 pb0 = pack_b(sc, 0), pb1 = pack_b(sc, 1);
#pragma unroll
      for (int t = 0; t < NDT; ++t) {
        acc[t] = mfma32(vop(t, key0 / 8 + g), pb0, acc[t]);
        acc[t] = mfma32(vop(t, key0 / 8 + 2 + g), pb1, acc[t]);
      }
    }
  };

  // ---- sweep over the 2p pairs before block 2p (pair pp is complete once the counter
  // exceeds 2pp + 1), double buffered ----
  const int npair = 2 * p;
  int ready = 0;
  if (npair > 0) {
    ready = wait_counter_gt(cnt, 1);
    stage(0);
    dma_wait();
  }
  __syncthreads();
  for (int pp = 0; pp < npair; ++pp) {
    const int buf = pp & 1;
    const bool more = pp + 1 < npair;
    const int need = 2 * pp + 3;  // pair pp + 1 is complete once the counter exceeds this
    bool early = false;
    if (more) {
      if (need >= ready) {
        const int seen = poll_counter(cnt);
        if (seen > need) {
          chain_acquire();
          ready = seen;
        }
      }
      early = need < ready;
      if (early) stage(pp + 1);
    }
    sweep_keys(sm.u.st.k[buf], [&](int t, int c) { return ld8(swz<16>(sm.u.st.v[buf], t * 32 + l32, c)); });
    if (more && !early) {
      ready = wait_counter_gt(cnt, need);
      stage(pp + 1);
    }
    dma_wait();
    __syncthreads();
  }

  // ---- solve one 128-row block q (2p or 2p + 1) whose R^T is in Rt: V'_A = X_A R_A,
  // V'_B = X_B R_B + Z V'_A, written out and kept as V'^T in LDS; then published ----
  f32x4 xr[4];
  auto xload = [&](int q) {
    const float* pinv_blk = pinv + ((int64_t)bh * NT + 2 * q) * 4096;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int idx = tid + NTHR * u;
      const int sb = idx >> 10, r = (idx >> 4) & 63, c4 = (idx & 15) * 4;
      xr[u] = *reinterpret_cast<const f32x4*>(pinv_blk + sb * 4096 + r * 64 + c4);
    }
  };
  auto xstore = [&](int sb) {
#pragma unroll
    for (int u = 2 * sb; u < 2 * sb + 2; ++u) {
      const int idx = tid + NTHR * u;
      const int r = (idx >> 4) & 63, c4 = (idx & 15) * 4;
      *reinterpret_cast<f32x4*>(&sm.u.fin.X[r][c4]) = xr[u];
    }
  };
  auto solve_block = [&](int q) {
    const int r0 = q * 128;
    // Z rows of this wave's B output tiles (row half rh = w & 1)
    f32x4 zr[4][2];
    {
      const float* zrow = zx + ((int64_t)bh * (T / 128) + q) * 4096 + ((w & 1) * 32 + l32) * 64 + 8 * g;
#pragma unroll
      for (int st = 0; st < 4; ++st) {
        zr[st][0] = *reinterpret_cast<const f32x4*>(zrow + 16 * st);
        zr[st][1] = *reinterpret_cast<const f32x4*>(zrow + 16 * st + 4);
      }
    }
    float(*Rt)[132] = sm.u.fin.Rt;
    // V'^T[d][r] = sum_c R^T[d][c] X[r][c] for sub-block sb (X lower triangular); tile w
    auto diag_solve = [&](int sb) {
      const int dt = w >> 1, rh = w & 1;
      f32x16 o = zero16();
      const int kmax = rh ? 4 : 2;
      for (int st = 0; st < kmax; ++st) {
        bf16x8 ah, al, bh8, bl;
        split8(&Rt[dt * 32 + l32][sb * 64 + 16 * st + 8 * g], ah, al);
        split8(&sm.u.fin.X[rh * 32 + l32][16 * st + 8 * g], bh8, bl);
        o = mfma32(ah, bh8, o);
        o = mfma32(ah, bl, o);
        o = mfma32(al, bh8, o);
      }
      if (sb == 1) {  // + Z V'_A: V'_A^T from the bf16 T-perm tile, Z split into hi + lo
#pragma unroll
        for (int st = 0; st < 4; ++st) {
          bf16x8 zh, zl;
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float x = zr[st][e >> 2][e & 3];
            zh[e] = (bf16)x;
            zl[e] = (bf16)(x - (float)zh[e]);
          }
          const bf16x8 va = ld8(&sm.u.fin.vT[dt * 32 + l32][16 * st + 8 * g]);
          o = mfma32(va, zh, o);
          o = mfma32(va, zl, o);
        }
      }
      const int rl = rh * 32 + l32;
      const int r = r0 + sb * 64 + rl;
      const int lslot = sb * 64 + ((rl & ~15) | jmap(rl & 15));
      float* out32 = vp32 + ((int64_t)bh * T + r) * D;
      bf16* outb = vpb + ((int64_t)bh * T + r) * D;
#pragma unroll
      for (int qd = 0; qd < 4; ++qd) {
        const int d0 = dt * 32 + 8 * qd + 4 * g;
        f32x4 f;
        bf16x4 bb;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          f[u] = o[4 * qd + u];
          bb[u] = (bf16)o[4 * qd + u];
          sm.u.fin.vT[d0 + u][lslot] = bb[u];
        }
        *reinterpret_cast<f32x4*>(out32 + d0) = f;
        *reinterpret_cast<bf16x4*>(outb + d0) = bb;
      }
    };
    xstore(0);
    __syncthreads();
    diag_solve(0);
    __syncthreads();
    xstore(1);
    __syncthreads();
    diag_solve(1);
    __syncthreads();
    // V'^T of the block to the T-perm operand copy: 16-byte stores
    for (int c = tid; c < D * 16; c += NTHR) {
      const int dd = c >> 4, s8 = (c & 15) * 8;
      *reinterpret_cast<bf16x8*>(vpt + ((int64_t)bh * D + dd) * T + r0 + s8) = ld8(&sm.u.fin.vT[dd][s8]);
    }
    publish_counter(cnt, 2 * q + 2);
  };
  // R^T = -C acc for the waves of block half `half` (waves 4 half .. 4 half + 3)
  auto store_r = [&](int half) {
    if ((w >> 2) == half) {
#pragma unroll
      for (int t = 0; t < NDT; ++t)
#pragma unroll
        for (int e = 0; e < 16; ++e) sm.u.fin.Rt[t * 32 + drow(e, g)][32 * (w & 3) + l32] = -Cf * acc[t][e];
    }
  };

  // ---- block 2p ----
  xload(2 * p);
  store_r(0);
  solve_block(2 * p);  // (its first barrier orders the R^T stores before the solve)
  // ---- block 2p + 1: block 2p's keys (K^ rows staged into R^T's bytes, V'^T from the
  // solve's copy), then its own solve ----
  bf16* kx = reinterpret_cast<bf16*>(&sm.u.fin.Rt[0][0]);
  dma_stage<128, D / 8, NTHR>(plan_k, khh + (int64_t)i0 * D, kx);
  xload(2 * p + 1);
  dma_wait();
  __syncthreads();
  if (w >= 4) sweep_keys(kx, [&](int t, int c) { return ld8(&sm.u.fin.vT[t * 32 + l32][8 * c]); });
  __syncthreads();
  store_r(1);
  solve_block(2 * p + 1);
}

// ---------------------------------------------------------------------------
// Fused forward at head dim 64 (bf16, one query head per kv head): the chained
// preconditioner solve of one 128-row block and the causal attention of the same 128
// query rows in one workgroup, so that every staged key tile and every LDS operand read
// feeds both.  The chain (ids, counters, staging, finalisation) is lucid_precond_fwd_kernel's;
// the attention is lucid_attn_fwd_kernel's online softmax.  Wave w owns rows
// i0 + 32w .. +32 (lane <-> row) of both and sweeps all 128 keys of each staged pair as
// four 32-key sub-tiles mt:
//   K_j rows (A operand, one LDS read)  -> S^T = K_j . K_i (chain) and K_j . Q_i (attention)
//   V'^T (A operand, one LDS read)      -> acc^T += V'^T P^T (chain) and O^T += V'^T A^T
// The chain's two products and the attention's two are independent, so the exp work of
// one overlaps the matrix products of the other inside the wave.  After the block's V' is
// solved and published, the attention finishes on the diagonal pair (the block's own keys,
// K rows staged again, V'^T from the solve's LDS copy) and writes O and lse2.
// Heads of the exact chains return at once (lucid_precond_fwd_kernel<D, true> and the
// attention kernel with skip_fast cover them).
// ---------------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(256) LUCID_TWO_WAVES_IF(true) void lucid_fused_fwd_kernel(
    const bf16* __restrict__ q, Strides qs, const bf16* __restrict__ k, Strides ks, const bf16* __restrict__ v,
    Strides vs, int Hkv, int T, int BH, const float* __restrict__ rinv, float scale, float* __restrict__ vp32,
    bf16* __restrict__ vpb, bf16* __restrict__ vpt, const float* __restrict__ pinv, const float* __restrict__ zx,
    const float* __restrict__ mass, int* __restrict__ counters, bf16* __restrict__ o, Strides os,
    float* __restrict__ lse) {
  static_assert(D == 64, "fused forward: head dim 64");
  constexpr int NDT = D / 32;
  constexpr int NKS = D / 16;
  __shared__ __attribute__((aligned(16))) PfwdSmem<D, false, false> sm;

  const int id = blockIdx.x;
  const int i2 = id / BH, bh = id - (id / BH) * BH;
  if (mass[bh] > kExactMass) return;  // the exact chain and attention kernels cover this head
  const int b = bh / Hkv, h = bh - b * Hkv;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int g = lane >> 5, l32 = lane & 31;
  const int i0 = i2 * 128;
  const int NT = T / 64;
  const int irow = i0 + 32 * w + l32;  // this lane's row (chain and attention)
  const bf16* kp = k + b * ks.b + h * ks.h;
  const bf16* vh = v + b * vs.b + h * vs.h;
  const float* rv = rinv + (int64_t)bh * T;
  const bf16* vpth = vpt + (int64_t)bh * D * T;
  const float* pinv_blk = pinv + ((int64_t)bh * NT + 2 * i2) * 4096;
  int* cnt = counters + bh;
  const float sl2 = scale * LOG2E_F;
  const float c0 = LOG2E_F / scale;
  const float c = sl2;  // attention: P = exp2(c S - m)

  // the row's key scaled by s log2(e) r_i (one bf16 rounding): with the staged raw K_j rows
  // (shared with the attention) the chain's exponent is r_j times the product, minus c0
  const float ai = sl2 * rv[irow];
  bf16x8 kbi[NKS], qbi[NKS];
#pragma unroll
  for (int st = 0; st < NKS; ++st) {
    kbi[st] = scale8(ld8(kp + (int64_t)irow * ks.t + 16 * st + 8 * g), ai);
    qbi[st] = ld8(q + b * qs.b + h * qs.h + (int64_t)irow * qs.t + 16 * st + 8 * g);
  }
  // chain accumulators start at -V^T (R = -acc after the sweep); attention at zero
  f32x16 acc[NDT], oacc[NDT];
#pragma unroll
  for (int t = 0; t < NDT; ++t) {
    oacc[t] = zero16();
#pragma unroll
    for (int qd = 0; qd < 4; ++qd) {
      const bf16x4 x = *reinterpret_cast<const bf16x4*>(vh + (int64_t)irow * vs.t + t * 32 + 8 * qd + 4 * g);
#pragma unroll
      for (int u = 0; u < 4; ++u) acc[t][4 * qd + u] = -(float)x[u];
    }
  }
  float m = -1e30f, lsum = 0.f;

  const int npair = i2;
  int ready = 0;
  int plan_k[128 * (D / 8) / 256], plan_v[D * 16 / 256];
  dma_plan<128, D / 8>(ks.t, plan_k);
  dma_plan<D, 16>(T, plan_v);
  auto stage = [&](int pp) {
    const int buf = pp & 1;
    if (w < 2) dma_f32x64(rv + pp * 128 + 64 * w, &sm.u.st.r[buf][64 * w]);
    dma_stage<128, D / 8>(plan_k, kp + (int64_t)pp * 128 * ks.t, sm.u.st.k[buf]);
    dma_stage<D, 16>(plan_v, vpth + pp * 128, sm.u.st.v[buf]);
  };
  f32x4 xr[8];
  auto xload = [&]() {
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int idx = tid + 256 * u;
      const int sb = idx >> 10, r = (idx >> 4) & 63, c4 = (idx & 15) * 4;
      xr[u] = *reinterpret_cast<const f32x4*>(pinv_blk + sb * 4096 + r * 64 + c4);
    }
  };
  auto xstore = [&](int sb) {
#pragma unroll
    for (int u = 4 * sb; u < 4 * sb + 4; ++u) {
      const int idx = tid + 256 * u;
      const int r = (idx >> 4) & 63, c4 = (idx & 15) * 4;
      *reinterpret_cast<f32x4*>(&sm.u.fin.X[r][c4]) = xr[u];
    }
  };
  // online softmax of one 32-key sub-tile of scores (lazy rescale: the reference max moves
  // only when a row grows by more than 2^8); returns the two bf16 B operands
  auto softmax = [&](f32x16& sa, bf16x8& pa0, bf16x8& pa1) {
    float mx = -INFINITY;
#pragma unroll
    for (int e = 0; e < 16; ++e) mx = fmaxf(mx, sa[e]);
    mx = wave_max32(mx) * c;
    if (__builtin_amdgcn_ballot_w64(mx > m + 8.0f)) {
      const float mnew = fmaxf(m, mx);
      const float alpha = __builtin_amdgcn_exp2f(m - mnew);
      m = mnew;
      lsum *= alpha;
#pragma unroll
      for (int t = 0; t < NDT; ++t)
#pragma unroll
        for (int e = 0; e < 16; ++e) oacc[t][e] *= alpha;
    }
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const float p = __builtin_amdgcn_exp2f(fmaf(sa[e], c, -m));
      lsum += p;
      sa[e] = p;
    }
    pa0 = pack_b(sa, 0);
    pa1 = pack_b(sa, 1);
  };
  // one staged pair: the chain's P V' and the attention, sub-tiles mt = 0..3
  auto sweep_pair = [&](int buf) {
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      const int key0 = mt * 32;
      bf16x8 ka[NKS];
#pragma unroll
      for (int st = 0; st < NKS; ++st) ka[st] = ld8(swz<D / 8>(sm.u.st.k[buf], key0 + l32, 2 * st + g));
      float rj[16];
      lds_rows16(&sm.u.st.r[buf][key0], g, rj);
      f32x16 sc = zero16(), sa = zero16();
#pragma unroll
      for (int st = 0; st < NKS; ++st) {
        sc = mfma32(ka[st], kbi[st], sc);
        sa = mfma32(ka[st], qbi[st], sa);
      }
#pragma unroll
      for (int e = 0; e < 16; ++e) sc[e] = __builtin_amdgcn_exp2f(fmaf(sc[e], rj[e], -c0));
      const bf16x8 pb0 = pack_b(sc, 0), pb1 = pack_b(sc, 1);
      bf16x8 pa0, pa1;
      softmax(sa, pa0, pa1);
#pragma unroll
      for (int t = 0; t < NDT; ++t) {
        const bf16x8 va0 = ld8(swz<16>(sm.u.st.v[buf], t * 32 + l32, key0 / 8 + g));
        const bf16x8 va1 = ld8(swz<16>(sm.u.st.v[buf], t * 32 + l32, key0 / 8 + 2 + g));
        acc[t] = mfma32(va0, pb0, acc[t]);
        acc[t] = mfma32(va1, pb1, acc[t]);
        oacc[t] = mfma32(va0, pa0, oacc[t]);
        oacc[t] = mfma32(va1, pa1, oacc[t]);
      }
    }
  };
  if (npair > 0) {
    ready = wait_counter_gt(cnt, 1);
    stage(0);
    dma_wait();
  } else {
    xload();
  }
  __syncthreads();
  for (int pp = 0; pp + 1 < npair; ++pp) {
    const int need = 2 * pp + 3;  // pair pp + 1 is complete once the counter exceeds this
    if (need >= ready) {
      const int seen = poll_counter(cnt);
      if (seen > need) {
        chain_acquire();
        ready = seen;
      }
    }
    const bool early = need < ready;
    if (early) stage(pp + 1);
    sweep_pair(pp & 1);
    if (!early) {
      ready = wait_counter_gt(cnt, need);
      stage(pp + 1);
    }
    dma_wait();
    __syncthreads();
  }
  if (npair > 0) {
    xload();  // fetch the inverses while the last pair is processed
    sweep_pair((npair - 1) & 1);
    __syncthreads();
  }

  // ---- the chain's block solve: R^T = -acc, V'_A = X_A R_A, V'_B = X_B R_B + Z V'_A ----
  float(*Rt)[132] = sm.u.fin.Rt;
#pragma unroll
  for (int t = 0; t < NDT; ++t)
#pragma unroll
    for (int e = 0; e < 16; ++e) Rt[t * 32 + drow(e, g)][32 * w + l32] = -acc[t][e];
  xstore(0);
  f32x4 zr[4][2];
  {
    const float* zrow = zx + ((int64_t)bh * (T / 128) + i2) * 4096 + ((w & 1) * 32 + l32) * 64 + 8 * g;
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      zr[st][0] = *reinterpret_cast<const f32x4*>(zrow + 16 * st);
      zr[st][1] = *reinterpret_cast<const f32x4*>(zrow + 16 * st + 4);
    }
  }
  __syncthreads();
  auto diag_solve = [&](int sb) {
    for (int tile = w; tile < NDT * 2; tile += 4) {
      const int dt = tile >> 1, rh = tile & 1;
      f32x16 ov = zero16();
      const int kmax = rh ? 4 : 2;
      for (int st = 0; st < kmax; ++st) {
        bf16x8 ah, al, bh8, bl;
        split8(&Rt[dt * 32 + l32][sb * 64 + 16 * st + 8 * g], ah, al);
        split8(&sm.u.fin.X[rh * 32 + l32][16 * st + 8 * g], bh8, bl);
        ov = mfma32(ah, bh8, ov);
        ov = mfma32(ah, bl, ov);
        ov = mfma32(al, bh8, ov);
      }
      if (sb == 1) {  // + Z V'_A
#pragma unroll
        for (int st = 0; st < 4; ++st) {
          bf16x8 zh, zl;
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float x = zr[st][e >> 2][e & 3];
            zh[e] = (bf16)x;
            zl[e] = (bf16)(x - (float)zh[e]);
          }
          const bf16x8 va = ld8(&sm.u.fin.vT[dt * 32 + l32][16 * st + 8 * g]);
          ov = mfma32(va, zh, ov);
          ov = mfma32(va, zl, ov);
        }
      }
      const int rl = rh * 32 + l32;
      const int r = i0 + sb * 64 + rl;
      const int lslot = sb * 64 + ((rl & ~15) | jmap(rl & 15));
      float* out32 = vp32 + ((int64_t)bh * T + r) * D;
      bf16* outb = vpb + ((int64_t)bh * T + r) * D;
#pragma unroll
      for (int qd = 0; qd < 4; ++qd) {
        const int d0 = dt * 32 + 8 * qd + 4 * g;
        f32x4 f;
        bf16x4 bb;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          f[u] = ov[4 * qd + u];
          bb[u] = (bf16)ov[4 * qd + u];
          sm.u.fin.vT[d0 + u][lslot] = bb[u];
        }
        *reinterpret_cast<f32x4*>(out32 + d0) = f;
        *reinterpret_cast<bf16x4*>(outb + d0) = bb;
      }
    }
  };
  diag_solve(0);
  __syncthreads();
  xstore(1);
  __syncthreads();
  diag_solve(1);
  __syncthreads();
  for (int cc = tid; cc < D * 16; cc += 256) {
    const int dd = cc >> 4, s8 = (cc & 15) * 8;
    *reinterpret_cast<bf16x8*>(vpt + ((int64_t)bh * D + dd) * T + i0 + s8) = ld8(&sm.u.fin.vT[dd][s8]);
  }
  publish_counter(cnt, 2 * i2 + 2);

  // ---- the attention's diagonal pair: keys i0 .. i0 + 127 ----
  // the block's K rows go to the first staging buffer (its bytes lie inside R^T and X,
  // both dead now; V'^T of the block stays in fin.vT)
  static_assert(sizeof(sm.u.st.k[0]) <= offsetof(decltype(sm.u.fin), vT), "diagonal K rows overlap V'^T");
  dma_stage<128, D / 8>(plan_k, kp + (int64_t)i0 * ks.t, sm.u.st.k[0]);
  dma_wait();
  __syncthreads();
  for (int mt = 0; mt <= w; ++mt) {
    const int key0 = mt * 32;
    f32x16 sa = zero16();
#pragma unroll
    for (int st = 0; st < NKS; ++st) sa = mfma32(ld8(swz<D / 8>(sm.u.st.k[0], key0 + l32, 2 * st + g)), qbi[st], sa);
    if (mt == w) {
#pragma unroll
      for (int e = 0; e < 16; ++e)
        if (drow(e, g) > l32) sa[e] = -INFINITY;
    }
    bf16x8 pa0, pa1;
    softmax(sa, pa0, pa1);
#pragma unroll
    for (int t = 0; t < NDT; ++t) {
      oacc[t] = mfma32(ld8(&sm.u.fin.vT[t * 32 + l32][key0 + 8 * g]), pa0, oacc[t]);
      oacc[t] = mfma32(ld8(&sm.u.fin.vT[t * 32 + l32][key0 + 16 + 8 * g]), pa1, oacc[t]);
    }
  }
  const float ls = wave_sum32(lsum);
  const float inv = 1.0f / ls;
  bf16* op = o + b * os.b + h * os.h + (int64_t)irow * os.t;
#pragma unroll
  for (int t = 0; t < NDT; ++t)
#pragma unroll
    for (int qq = 0; qq < 4; ++qq) {
      bf16x4 bb;
#pragma unroll
      for (int u = 0; u < 4; ++u) bb[u] = (bf16)(oacc[t][4 * qq + u] * inv);
      *reinterpret_cast<bf16x4*>(op + t * 32 + 8 * qq + 4 * g) = bb;
    }
  if (g == 0) lse[(int64_t)bh * T + irow] = m + log2f(ls);
}

// Workgroup id of an attention grid (nblk row blocks x B*Hkv kv heads x G query heads)
// -> (row block, kv-head row bh = b*Hkv + h, query head g of the group), heavy (late) row
// blocks first.  Workgroup ids go to the 8 XCDs round robin, so when B*Hkv is a multiple of
// 8 the ids of one XCD take the kv heads bh = xcd, xcd + 8, ... with all G of their query
// heads: the query heads that read the same K and V' tiles share one L2.  Otherwise the
// query head is the fastest index.
__device__ __forceinline__ void attn_block_of(int id, int nblk, int BH, int G, int& ib, int& bh, int& g) {
  if ((BH & 7) == 0) {
    const int xcd = id & 7, kk = id >> 3, per = (BH >> 3) * G;
    const int ibo = kk / per, rest = kk - ibo * per;
    ib = nblk - 1 - ibo;
    bh = xcd + 8 * (rest / G);
    g = rest - (rest / G) * G;
  } else {
    const int BHq = BH * G, bhq = id % BHq;
    ib = nblk - 1 - id / BHq;
    bh = bhq / G;
    g = bhq - bh * G;
  }
}

// ---------------------------------------------------------------------------
// Causal attention on V' at head dim 128 (bf16): 256 query rows per workgroup as eight
// waves of 32 rows (one n-tile each), two waves per SIMD, so that one wave's softmax runs
// beside the other's MFMAs; every KT-key tile of K and V'^T (KT = 64 or 128; the launch uses
// 128) is staged once per workgroup in LDS (double buffered, loaded one tile ahead by direct
// global -> LDS loads of all 512 threads, swizzled rows) and read by all eight waves.  Per wave and 64 keys:
// S^T[j][i] = K_j . Q_i (16 MFMAs), the online softmax (one row max per staged tile, lazy
// rescale by 2^8), O^T[d][i] += V'^T[d][j] P^T[j][i] (16 MFMAs).
// Outputs as lucid_attn_fwd_kernel (O, lse2, O's lo part for exact heads).
// ---------------------------------------------------------------------------
// DA: the head-dim columns that can be nonzero (as in lucid_attn_fwd_kernel)
template <int D, int KT = 64, int DA = D>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2))) void lucid_attn_fwd_wide_kernel(
    const bf16* __restrict__ q, Strides qs, const bf16* __restrict__ k, Strides ks, const bf16* __restrict__ vpt,
    bf16* __restrict__ o, Strides os, float* __restrict__ lse, const float* __restrict__ mass,
    bf16* __restrict__ olo, int Hq, int Hkv, int T, int BH, float scale) {
  constexpr int NDT = D / 32;
  constexpr int NKS = D / 16;
  constexpr int NDT_A = (DA + 31) / 32, NKS_A = DA / 16;
  static_assert(DA % 16 == 0 && DA <= D, "active head dim");
  constexpr int NMT = KT / 32;        // 32-key sub-tiles per staged tile
  static_assert(D == 128, "the wide attention kernel is the head-dim-128 path");
  static_assert(KT == 64 || KT == 128, "keys per staged tile");
  // staged tiles, unpadded and swizzled (chunk c of row r at c ^ (r & 7)), filled by direct
  // global -> LDS loads.  One LDS variable: with the K and V'^T tiles in two, the compiler
  // waits for the next tile's loads before the first read of the current tile.
  __shared__ __attribute__((aligned(16))) struct {
    bf16 k[2][KT * D];
    bf16 v[2][D * KT];
  } sm;
  auto& lk = sm.k;
  auto& lv = sm.v;

  const int G = Hq / Hkv;
  const int nblk = (T + 255) / 256;
  int ib, bh, gi;
  attn_block_of(blockIdx.x, nblk, BH, G, ib, bh, gi);
  const int b = bh / Hkv, h = bh - b * Hkv, hq = h * G + gi, bhq = b * Hq + hq;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int g = lane >> 5, l32 = lane & 31;
  const int r0 = ib * 256;
  const int row0 = r0 + w * 32;  // this wave's 32 rows
  const bf16* qh = q + b * qs.b + hq * qs.h;
  const bf16* kh = k + b * ks.b + h * ks.h;
  const bf16* vth = vpt + (int64_t)bh * D * T;
  const float c = scale * LOG2E_F;

  bf16x8 qb[NKS];
  {
    const int rq = min(row0 + l32, T - 1);
#pragma unroll
    for (int st = 0; st < NKS_A; ++st) qb[st] = ld8(qh + (int64_t)rq * qs.t + 16 * st + 8 * g);
  }
  f32x16 oacc[NDT];
#pragma unroll
  for (int t = 0; t < NDT; ++t) oacc[t] = zero16();
  float m = -1e30f, lsum = 0.f;

  const int ntile = (min(r0 + 256, T) + KT - 1) / KT;
  const int last_w = row0 / KT;  // the tile holding this wave's diagonal
  // T is a multiple of KT (checked by the launch), so every staged tile lies inside the rows
  int plan_k[KT * (D / 8) / 512], plan_v[D * (KT / 8) / 512];
  dma_plan<KT, D / 8, 512>(ks.t, plan_k);
  dma_plan<D, KT / 8, 512>(T, plan_v);
  auto stage = [&](int j0, int buf) {
    dma_stage<KT, D / 8, 512>(plan_k, kh + (int64_t)j0 * ks.t, lk[buf]);
    dma_stage<D, KT / 8, 512>(plan_v, vth + j0, lv[buf]);
  };
  stage(0, 0);
  // the Q rows are consumed here, so that they have landed before the loop: otherwise the
  // compiler moves their loads past this point and then waits for all loads (vmcnt(0)),
  // the next tile's direct loads included, before the first product of every tile
#pragma unroll
  for (int st = 0; st < NKS_A; ++st) asm volatile("" ::"v"(qb[st]));
  dma_wait();
  __syncthreads();
  for (int jt = 0; jt < ntile; ++jt) {
    const int buf = jt & 1;
    const bool more = jt + 1 < ntile;
    if (more) stage((jt + 1) * KT, buf ^ 1);
    if (jt <= last_w && row0 < T) {
      f32x16 s[NMT];
#pragma unroll
      for (int mt = 0; mt < NMT; ++mt) {
        s[mt] = zero16();
#pragma unroll
        for (int st = 0; st < NKS_A; ++st)
          s[mt] = mfma32(ld8(swz<D / 8>(lk[buf], mt * 32 + l32, 2 * st + g)), qb[st], s[mt]);
      }
      if (jt == last_w) {  // causal mask: key KT jt + mt 32 + drow > row
        const int rel = row0 - jt * KT + l32;  // the lane's row relative to the tile's first key
#pragma unroll
        for (int mt = 0; mt < NMT; ++mt)
#pragma unroll
          for (int e = 0; e < 16; ++e)
            if (mt * 32 + drow(e, g) > rel) s[mt][e] = -INFINITY;
      }
      float mx = -INFINITY;
#pragma unroll
      for (int mt = 0; mt < NMT; ++mt)
#pragma unroll
        for (int e = 0; e < 16; ++e) mx = fmaxf(mx, s[mt][e]);
      mx = wave_max32(mx) * c;
      if (__builtin_amdgcn_ballot_w64(mx > m + 8.0f)) {
        const float mnew = fmaxf(m, mx);
        const float alpha = __builtin_amdgcn_exp2f(m - mnew);
        m = mnew;
        lsum *= alpha;
#pragma unroll
        for (int t = 0; t < NDT_A; ++t)
#pragma unroll
          for (int e = 0; e < 16; ++e) oacc[t][e] *= alpha;
      }
      // per 32-key sub-tile: its exps, then its P V' products (key order within each O tile
      // as before), so that the exps of the next sub-tile can issue beside these MFMAs
#pragma unroll
      for (int mt = 0; mt < NMT; ++mt) {
#pragma unroll
        for (int e = 0; e < 16; ++e) s[mt][e] = __builtin_amdgcn_exp2f(fmaf(s[mt][e], c, -m));
        const bf16x8 pb0 = pack_b(s[mt], 0), pb1 = pack_b(s[mt], 1);
        lsum = add_sum8(pb1, add_sum8(pb0, lsum));  // sum of the bf16 P of P V'
#pragma unroll
        for (int t = 0; t < NDT_A; ++t) {
          oacc[t] = mfma32(ld8(swz<KT / 8>(lv[buf], t * 32 + l32, 4 * mt + g)), pb0, oacc[t]);
          oacc[t] = mfma32(ld8(swz<KT / 8>(lv[buf], t * 32 + l32, 4 * mt + 2 + g)), pb1, oacc[t]);
        }
      }
    }
    dma_wait();
    __syncthreads();
  }
  const bool exact = mass[bh] > kExactMass;
  const int irow = row0 + l32;
  const float ls = wave_sum32(lsum);
  if (irow < T) {
    const float inv = 1.0f / ls;
    bf16* op = o + b * os.b + hq * os.h + (int64_t)irow * os.t;
    bf16* ol = olo + ((int64_t)bhq * T + irow) * D;
#pragma unroll
    for (int t = 0; t < NDT; ++t)
#pragma unroll
      for (int qq = 0; qq < 4; ++qq) {
        bf16x4 bb, bl;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const float x = oacc[t][4 * qq + u] * inv;
          bb[u] = (bf16)x;
          bl[u] = (bf16)(x - (float)bb[u]);
        }
        *reinterpret_cast<bf16x4*>(op + t * 32 + 8 * qq + 4 * g) = bb;
        if (exact) *reinterpret_cast<bf16x4*>(ol + t * 32 + 8 * qq + 4 * g) = bl;
      }
    if (g == 0) lse[(int64_t)bhq * T + irow] = m + log2f(ls);
  }
}

}  // namespace lucid
