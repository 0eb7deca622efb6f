// LUCID decoding step on CDNA4 (gfx950): one new token per sequence against a
// (K, V') cache, with the exact preconditioner row (modeling_lucid.py:576-598 is
// the reference seam; its V' update drops the division by the diagonal P_tt, kept
// here so that a decoded row equals the same row of a prefill):
//   P_tj = exp(s r_t r_j (k_t . k_j) - 1/s),  r = 1 / rms(k)  (j < t)
//   v'_t = (v_t - sum_{j<t} P_tj v'_j) / P_tt,  P_tt = exp(s d ms_t / (ms_t + eps) - 1/s)
//   o_g  = softmax_j(s q_g . k_j) v'_j over j <= t, for the G query heads of the kv head
// Both sums read every cached row once (memory bound), so one pass over the cache
// computes them together, split over the sequence (flash-decoding):
//   lucid_decode_split_kernel    per (split, kv head): partial sum_j P_tj v'_j and the
//                                online-softmax state (m, l, O) of every query head
//   lucid_decode_combine_kernel  per (kv head, query head): v'_t, the token's own
//                                softmax term, the output, and the append of (k_t, v'_t)
//                                to the cache
#include "lucid_common.h"

namespace lucid {

constexpr float DEC_NEG = -1e30f;  // finite "minus infinity" for empty softmax states

#ifndef LUCID_DECODE_KB
#define LUCID_DECODE_KB 4  // keys per lane group and step of the split kernel
#endif
#ifndef LUCID_DECODE_EPL
#define LUCID_DECODE_EPL 8  // elements of a key row per lane (8 or 16)
#endif

struct DecodePartials {
  float* a;  // [nsplit][BH][D]     sum_j P_tj v'_j
  float* m;  // [nsplit][BH][G]     running max (log2 domain)
  float* l;  // [nsplit][BH][G]     running sum
  float* o;  // [nsplit][BH][G][D]  unnormalised output
};

// Each key row is read by LPK = D/EPL lanes (EPL elements each); a wave covers 64/LPK
// keys per step and each group of LPK lanes keeps its own partial state.
template <int D, int G>
__global__ __launch_bounds__(256) void lucid_decode_split_kernel(
    const bf16* __restrict__ q, Strides qs, const bf16* __restrict__ kn, Strides kns,
    const bf16* __restrict__ kc, Strides kcs, const bf16* __restrict__ vc, Strides vcs, int Hkv, int Tp, int KS,
    float scale, float eps, DecodePartials part) {
  constexpr int EPL = LUCID_DECODE_EPL, NV = EPL / 8;  // 16-byte loads per lane and row
  constexpr int LPK = D / EPL, NG = 256 / LPK;
  __shared__ float sa[4][D], so[4][G][D], sm_[4][G], sl[4][G];
  const int s = blockIdx.x, bh = blockIdx.y, BH = gridDim.y;
  const int b = bh / Hkv, h = bh - b * Hkv;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int sub = lane % LPK, grp = tid / LPK;
  const int j0 = s * KS, j1 = min(Tp, j0 + KS);

  float kt[EPL], qv[G][EPL];
#pragma unroll
  for (int c = 0; c < NV; ++c) {
    const bf16x8 x = ld8(kn + b * kns.b + h * kns.h + EPL * sub + 8 * c);
#pragma unroll
    for (int e = 0; e < 8; ++e) kt[8 * c + e] = (float)x[e];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const bf16x8 y = ld8(q + b * qs.b + (h * G + g) * qs.h + EPL * sub + 8 * c);
#pragma unroll
      for (int e = 0; e < 8; ++e) qv[g][8 * c + e] = (float)y[e];
    }
  }
  float nt = 0.f;
#pragma unroll
  for (int e = 0; e < EPL; ++e) nt = fmaf(kt[e], kt[e], nt);
#pragma unroll
  for (int off = 1; off < LPK; off <<= 1) nt += __shfl_xor(nt, off, 64);
  const float rt = rsqrtf(nt / D + eps);
  const float c1 = scale * rt * LOG2E_F, c0 = LOG2E_F / scale, sl2 = scale * LOG2E_F;

  float acc[EPL], oo[G][EPL], m[G], l[G];
#pragma unroll
  for (int e = 0; e < EPL; ++e) acc[e] = 0.f;
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = DEC_NEG;
    l[g] = 0.f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) oo[g][e] = 0.f;
  }
  const bf16* kbase = kc + b * kcs.b + h * kcs.h + EPL * sub;
  const bf16* vbase = vc + b * vcs.b + h * vcs.h + EPL * sub;
  // KB keys per group and step, all loads issued before the arithmetic (HBM latency);
  // a key past the split's end is loaded clamped and contributes nothing
  constexpr int KB = LUCID_DECODE_KB;
  for (int j = j0 + grp; j < j1; j += KB * NG) {
    bf16x8 kx[KB][NV], vx[KB][NV];
#pragma unroll
    for (int u = 0; u < KB; ++u) {
      const int jj = min(j + u * NG, j1 - 1);
#pragma unroll
      for (int c = 0; c < NV; ++c) {
        kx[u][c] = ld8(kbase + (int64_t)jj * kcs.t + 8 * c);
        vx[u][c] = ld8(vbase + (int64_t)jj * vcs.t + 8 * c);
      }
    }
    // scores of the KB keys, then one running-max update and rescale per query head
    float pk[KB], sg[KB][G];
#pragma unroll
    for (int u = 0; u < KB; ++u) {
      const bool ok = j + u * NG < j1;
      float kk = 0.f, nn = 0.f, qk[G];
#pragma unroll
      for (int g = 0; g < G; ++g) qk[g] = 0.f;
#pragma unroll
      for (int e = 0; e < EPL; ++e) {
        const float x = (float)kx[u][e >> 3][e & 7];
        kk = fmaf(kt[e], x, kk);
        nn = fmaf(x, x, nn);
#pragma unroll
        for (int g = 0; g < G; ++g) qk[g] = fmaf(qv[g][e], x, qk[g]);
      }
#pragma unroll
      for (int off = 1; off < LPK; off <<= 1) {
        kk += __shfl_xor(kk, off, 64);
        nn += __shfl_xor(nn, off, 64);
#pragma unroll
        for (int g = 0; g < G; ++g) qk[g] += __shfl_xor(qk[g], off, 64);
      }
      pk[u] = ok ? __builtin_amdgcn_exp2f(fmaf(c1 * rsqrtf(nn / D + eps), kk, -c0)) : 0.f;
#pragma unroll
      for (int g = 0; g < G; ++g) sg[u][g] = ok ? qk[g] * sl2 : 3.f * DEC_NEG;  // below any running max
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float mn = m[g];
#pragma unroll
      for (int u = 0; u < KB; ++u) mn = fmaxf(mn, sg[u][g]);
      const float al = __builtin_amdgcn_exp2f(m[g] - mn);
      m[g] = mn;
      l[g] *= al;
#pragma unroll
      for (int e = 0; e < EPL; ++e) oo[g][e] *= al;
#pragma unroll
      for (int u = 0; u < KB; ++u) sg[u][g] = __builtin_amdgcn_exp2f(sg[u][g] - mn);
    }
#pragma unroll
    for (int u = 0; u < KB; ++u) {
#pragma unroll
      for (int e = 0; e < EPL; ++e) {
        const float vv = (float)vx[u][e >> 3][e & 7];
        acc[e] = fmaf(pk[u], vv, acc[e]);
#pragma unroll
        for (int g = 0; g < G; ++g) oo[g][e] = fmaf(sg[u][g], vv, oo[g][e]);
      }
#pragma unroll
      for (int g = 0; g < G; ++g) l[g] += sg[u][g];
    }
  }
  // combine the groups of a wave (lanes with the same sub)
#pragma unroll
  for (int off = LPK; off < 64; off <<= 1) {
#pragma unroll
    for (int e = 0; e < EPL; ++e) acc[e] += __shfl_xor(acc[e], off, 64);
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float mp = __shfl_xor(m[g], off, 64), lp = __shfl_xor(l[g], off, 64);
      const float mn = fmaxf(m[g], mp);
      const float a0 = __builtin_amdgcn_exp2f(m[g] - mn), a1 = __builtin_amdgcn_exp2f(mp - mn);
      l[g] = l[g] * a0 + lp * a1;
#pragma unroll
      for (int e = 0; e < EPL; ++e) oo[g][e] = oo[g][e] * a0 + __shfl_xor(oo[g][e], off, 64) * a1;
      m[g] = mn;
    }
  }
  if (lane < LPK) {
#pragma unroll
    for (int e = 0; e < EPL; ++e) sa[w][EPL * sub + e] = acc[e];
#pragma unroll
    for (int g = 0; g < G; ++g) {
#pragma unroll
      for (int e = 0; e < EPL; ++e) so[w][g][EPL * sub + e] = oo[g][e];
      if (sub == 0) {
        sm_[w][g] = m[g];
        sl[w][g] = l[g];
      }
    }
  }
  __syncthreads();
  // combine the 4 waves: thread d of the first D threads owns column d
  if (tid < D) {
    const int d = tid;
    part.a[((int64_t)s * BH + bh) * D + d] = sa[0][d] + sa[1][d] + sa[2][d] + sa[3][d];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float mn = fmaxf(fmaxf(sm_[0][g], sm_[1][g]), fmaxf(sm_[2][g], sm_[3][g]));
      float lt = 0.f, ot = 0.f;
#pragma unroll
      for (int ww = 0; ww < 4; ++ww) {
        const float al = __builtin_amdgcn_exp2f(sm_[ww][g] - mn);
        lt = fmaf(sl[ww][g], al, lt);
        ot = fmaf(so[ww][g][d], al, ot);
      }
      part.o[(((int64_t)s * BH + bh) * G + g) * D + d] = ot;
      if (d == 0) {
        part.m[((int64_t)s * BH + bh) * G + g] = mn;
        part.l[((int64_t)s * BH + bh) * G + g] = lt;
      }
    }
  }
}

// grid (B*Hkv, G): workgroup (kv head, query head g).  The 256 threads are NSL = 256/D
// split lanes x D columns; each split lane reduces every NSL-th partial, then the
// lanes are combined in LDS.  Every workgroup of a kv head computes v'_t; the g = 0
// one writes it and appends (k_t, v'_t) to the caches.
template <int D, int G>
__global__ __launch_bounds__(256) void lucid_decode_combine_kernel(
    int nsplit, const bf16* __restrict__ q, Strides qs, const bf16* __restrict__ kn, Strides kns,
    const bf16* __restrict__ vn, Strides vns, bf16* __restrict__ kc, Strides kcs, bf16* __restrict__ vc, Strides vcs,
    bf16* __restrict__ o, Strides os, float* __restrict__ vp_new, int Hkv, int Tp, float scale, float eps,
    DecodePartials part) {
  constexpr int NSL = 256 / D;
  __shared__ float ra[NSL][D], ro[NSL][D], rm[NSL], rl[NSL], dots[2][D];
  const int bh = blockIdx.x, BH = gridDim.x, g = blockIdx.y;
  const int b = bh / Hkv, h = bh - b * Hkv;
  const int tid = threadIdx.x, sl = tid / D, d = tid - sl * D;
  const int hq = h * G + g;
  // running max of this query head over the splits
  float mx = DEC_NEG;
#pragma unroll 8
  for (int s = sl; s < nsplit; s += NSL) mx = fmaxf(mx, part.m[((int64_t)s * BH + bh) * G + g]);
  if (d == 0) rm[sl] = mx;
  if (sl == 0) {
    const float kd = (float)kn[b * kns.b + h * kns.h + d];
    dots[0][d] = kd * kd;
    dots[1][d] = (float)q[b * qs.b + hq * qs.h + d] * kd;
  }
  __syncthreads();
  float M = rm[0];
#pragma unroll
  for (int i = 1; i < NSL; ++i) M = fmaxf(M, rm[i]);
  float a = 0.f, lt = 0.f, ot = 0.f;
#pragma unroll 8
  for (int s = sl; s < nsplit; s += NSL) {
    const int64_t i = ((int64_t)s * BH + bh) * G + g;
    const float al = __builtin_amdgcn_exp2f(part.m[i] - M);
    a += part.a[((int64_t)s * BH + bh) * D + d];
    lt = fmaf(part.l[i], al, lt);
    ot = fmaf(part.o[i * D + d], al, ot);
  }
  ra[sl][d] = a;
  ro[sl][d] = ot;
  if (d == 0) rl[sl] = lt;
  __syncthreads();
  if (sl != 0) return;
  float nk = 0.f, qk = 0.f;
  for (int i = 0; i < D; ++i) {
    nk += dots[0][i];
    qk += dots[1][i];
  }
#pragma unroll
  for (int i = 1; i < NSL; ++i) {
    a += ra[i][d];
    ot += ro[i][d];
  }
  lt = 0.f;
#pragma unroll
  for (int i = 0; i < NSL; ++i) lt += rl[i];
  const float ms = nk / D;
  // P_tt = exp(s |K^_t|^2 - 1/s), |K^_t|^2 = D ms / (ms + eps)
  const float ptt = __builtin_amdgcn_exp2f(LOG2E_F * (scale * D * ms / (ms + eps) - 1.f / scale));
  const float vpt = ((float)vn[b * vns.b + h * vns.h + d] - a) / ptt;
  const bf16 vpb = (bf16)vpt;
  if (g == 0) {
    vp_new[(int64_t)bh * D + d] = vpt;
    kc[b * kcs.b + h * kcs.h + (int64_t)Tp * kcs.t + d] = kn[b * kns.b + h * kns.h + d];
    vc[b * vcs.b + h * vcs.h + (int64_t)Tp * vcs.t + d] = vpb;
  }
  // the token's own term joins the softmax
  const float st = qk * scale * LOG2E_F;
  const float M2 = fmaxf(M, st);
  const float c = __builtin_amdgcn_exp2f(M - M2), es = __builtin_amdgcn_exp2f(st - M2);
  o[b * os.b + hq * os.h + d] = (bf16)((ot * c + es * (float)vpb) / (lt * c + es));
}

}  // namespace lucid
