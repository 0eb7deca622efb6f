// LUCID attention backward on CDNA4 (gfx950).
//
// Attention part (FlashAttention-2 style, recomputing P from lse):
//   dV'_j = sum_i P_ij dO_i,  dS = P (dO V'^T - delta),  dK_attn = s dS^T Q,  dQ = s dS K
// Preconditioner part (modeling_lucid.py:314-382, Lucid_Tril_Solver.backward):
//   dV  = P^-T dV'                      (chained upper solve, last block first)
//   M   = tril((dV V'^T) * P)
//   dK^ = -s (M K^ + M^T K^),  dK = r (dK^ - K^ (K^.dK^)/d) + dK_attn   (RMSNorm backward)
//
// Kernels:
//   lucid_bwd_prep_kernel          delta = rowsum(dO * O), dO^T and Q^T in T-perm layout
//   lucid_attn_bwd_dkdv_kernel     column sweep: dV' (summed over the GQA group), dK_attn
//   lucid_attn_bwd_dq_kernel       row sweep: dQ
//   lucid_precond_bwd_col_kernel   chained transposed solve -> dV, and the M^T K^ column sums
//   lucid_precond_bwd_row_kernel   M K^ row sums, RMSNorm backward, dK
#include "lucid_common.h"

namespace lucid {

// grid (T/64, B*Hq)
template <int D>
__global__ __launch_bounds__(256) void lucid_bwd_prep_kernel(const bf16* __restrict__ dout, Strides dos,
                                                             const bf16* __restrict__ o, Strides os,
                                                             const bf16* __restrict__ q, Strides qs, int Hq, int T,
                                                             float* __restrict__ delta, bf16* __restrict__ dot,
                                                             bf16* __restrict__ qt, int* __restrict__ counters,
                                                             int BH) {
  constexpr int SEG = D / 4;
  __shared__ bf16 tdo[D][64 + 8];
  __shared__ bf16 tq[D][64 + 8];
  const int blk = blockIdx.x, bhq = blockIdx.y;
  const int b = bhq / Hq, hq = bhq - b * Hq;
  const int tid = threadIdx.x;
  const int row = tid >> 2, seg = tid & 3;
  const int t = blk * 64 + row;
  const bf16* dop = dout + b * dos.b + hq * dos.h + (int64_t)t * dos.t;
  const bf16* opp = o + b * os.b + hq * os.h + (int64_t)t * os.t;
  const bf16* qp = q + b * qs.b + hq * qs.h + (int64_t)t * qs.t;
  float acc = 0.f;
#pragma unroll
  for (int c = 0; c < SEG; c += 8) {
    const bf16x8 a = ld8(dop + seg * SEG + c);
    const bf16x8 bo = ld8(opp + seg * SEG + c);
    const bf16x8 qq = ld8(qp + seg * SEG + c);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      acc += (float)a[e] * (float)bo[e];
      tdo[seg * SEG + c + e][row] = a[e];
      tq[seg * SEG + c + e][row] = qq[e];
    }
  }
  acc += __shfl_xor(acc, 1, 64);
  acc += __shfl_xor(acc, 2, 64);
  if (seg == 0) delta[(int64_t)bhq * T + t] = acc;
  if (blk == 0 && tid == 0 && bhq < BH) counters[bhq] = 0;
  __syncthreads();
  for (int idx = tid; idx < D * 8; idx += 256) {
    const int dd = idx >> 3, c8 = idx & 7;
    bf16x8 a, bq;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int src = (c8 >> 1) * 16 + jmap((c8 & 1) * 8 + e);
      a[e] = tdo[dd][src];
      bq[e] = tq[dd][src];
    }
    const int64_t off = ((int64_t)bhq * D + dd) * T + blk * 64 + c8 * 8;
    *reinterpret_cast<bf16x8*>(dot + off) = a;
    *reinterpret_cast<bf16x8*>(qt + off) = bq;
  }
}

// ---------------------------------------------------------------------------
// Column sweep for the attention part.  Workgroup = 256 keys of one kv head,
// wave w owns keys 64w..64w+63 as two 32-key n-tiles (lane <-> key j); loops
// over the G query heads of the group and over every 64-row query tile at or
// below the diagonal.  Each query tile (Q, dO rows; Q^T, dO^T in T-perm
// layout; lse2 and delta) is staged once per workgroup in LDS, double buffered.
//   S[i][j] = Q_i . K_j, P = exp2(c S - lse2_i)
//   dV'^T[d][j] += dO^T[d][i] P[i][j];  dP[i][j] = dO_i . V'_j
//   dS = P (dP - delta_i);  dK^T[d][j] += Q^T[d][i] dS[i][j]
// ---------------------------------------------------------------------------
template <int D>
struct DkdvSmem {
  bf16 q[2][64][D + 8];
  bf16 dO[2][64][D + 8];
  bf16 qt[2][D][72];
  bf16 dot[2][D][72];
  float lse[2][64];
  float dl[2][64];
};

template <int D>
__global__ __launch_bounds__(256) void lucid_attn_bwd_dkdv_kernel(
    const bf16* __restrict__ q, Strides qs, const bf16* __restrict__ k, Strides ks, const bf16* __restrict__ vpb,
    const bf16* __restrict__ dout, Strides dos, const bf16* __restrict__ qt, const bf16* __restrict__ dot,
    const float* __restrict__ lse, const float* __restrict__ delta, float* __restrict__ dvp,
    float* __restrict__ dka, int Hq, int Hkv, int T, int BH, float scale) {
  constexpr int NDT = D / 32;
  constexpr int NKS = D / 16;
  constexpr int CH = D / 32;
  __shared__ __attribute__((aligned(16))) DkdvSmem<D> sm;
  const int id = blockIdx.x;
  const int jb = id / BH, bh = id - (id / BH) * BH;
  const int b = bh / Hkv, h = bh - b * Hkv;
  const int G = Hq / Hkv;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int g = lane >> 5, l32 = lane & 31;
  const int jw = jb * 256 + w * 64;  // first key of this wave
  const bf16* kh = k + b * ks.b + h * ks.h;
  const float c = scale * LOG2E_F;

  bf16x8 kb[2][NKS], vb[2][NKS];
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    const int jr = min(jw + nt * 32 + l32, T - 1);
#pragma unroll
    for (int st = 0; st < NKS; ++st) {
      kb[nt][st] = ld8(kh + (int64_t)jr * ks.t + 16 * st + 8 * g);
      vb[nt][st] = ld8(vpb + ((int64_t)bh * T + jr) * D + 16 * st + 8 * g);
    }
  }
  f32x16 adv[NDT][2], adk[NDT][2];
#pragma unroll
  for (int t = 0; t < NDT; ++t)
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      adv[t][nt] = zero16();
      adk[t][nt] = zero16();
    }
  const int nt64 = T / 64;
  const int it_first = jb * 4;  // first query tile any wave needs
  const int it_w = jw / 64;     // this wave's diagonal tile
  for (int gi = 0; gi < G; ++gi) {
    const int hq = h * G + gi;
    const int bhq = b * Hq + hq;
    const bf16* qh = q + b * qs.b + hq * qs.h;
    const bf16* doh = dout + b * dos.b + hq * dos.h;
    const bf16* qth = qt + (int64_t)bhq * D * T;
    const bf16* doth = dot + (int64_t)bhq * D * T;
    const float* lh = lse + (int64_t)bhq * T;
    const float* dh = delta + (int64_t)bhq * T;
    bf16x8 stg[4 * CH];
    f32x4 fstg;
    auto gload = [&](int it) {
      const int i0 = it * 64;
      g2r_rows<D>(qh, qs.t, i0, stg);
      g2r_rows<D>(doh, dos.t, i0, stg + CH);
      g2r_tp<D>(qth, T, i0, stg + 2 * CH);
      g2r_tp<D>(doth, T, i0, stg + 3 * CH);
      if (tid < 16) fstg = *reinterpret_cast<const f32x4*>(lh + i0 + 4 * tid);
      else if (tid < 32) fstg = *reinterpret_cast<const f32x4*>(dh + i0 + 4 * (tid - 16));
    };
    auto lstore = [&](int buf) {
      r2l_rows<D>(sm.q[buf], stg);
      r2l_rows<D>(sm.dO[buf], stg + CH);
      r2l_tp<D>(sm.qt[buf], stg + 2 * CH);
      r2l_tp<D>(sm.dot[buf], stg + 3 * CH);
      if (tid < 16) *reinterpret_cast<f32x4*>(&sm.lse[buf][4 * tid]) = fstg;
      else if (tid < 32) *reinterpret_cast<f32x4*>(&sm.dl[buf][4 * (tid - 16)]) = fstg;
    };
    if (it_first < nt64) {
      gload(it_first);
      lstore(0);
    }
    __syncthreads();
    for (int it = it_first; it < nt64; ++it) {
      const int buf = (it - it_first) & 1;
      const bool more = it + 1 < nt64;
      if (more) gload(it + 1);
      if (it >= it_w) {
        const bool diag = (it == it_w);
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
          float lr[16];
          lds_rows16(&sm.lse[buf][mt * 32], g, lr);
          bf16x8 pb[2][2];
          f32x16 pv[2];
          {
            bf16x8 qa[NKS];
#pragma unroll
            for (int st = 0; st < NKS; ++st) qa[st] = ld8(&sm.q[buf][mt * 32 + l32][16 * st + 8 * g]);
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) {
              f32x16 sc = zero16();
#pragma unroll
              for (int st = 0; st < NKS; ++st) sc = mfma32(qa[st], kb[nt][st], sc);
#pragma unroll
              for (int e = 0; e < 16; ++e) {
                float p = __builtin_amdgcn_exp2f(fmaf(sc[e], c, -lr[e]));
                if (diag && (mt * 32 + drow(e, g) < nt * 32 + l32)) p = 0.f;
                sc[e] = p;
              }
              pv[nt] = sc;
              pb[nt][0] = pack_b(sc, 0);
              pb[nt][1] = pack_b(sc, 1);
            }
          }
#pragma unroll
          for (int t = 0; t < NDT; ++t) {
            const bf16x8 a0 = ld8(&sm.dot[buf][t * 32 + l32][mt * 32 + 8 * g]);
            const bf16x8 a1 = ld8(&sm.dot[buf][t * 32 + l32][mt * 32 + 16 + 8 * g]);
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) {
              adv[t][nt] = mfma32(a0, pb[nt][0], adv[t][nt]);
              adv[t][nt] = mfma32(a1, pb[nt][1], adv[t][nt]);
            }
          }
          lds_rows16(&sm.dl[buf][mt * 32], g, lr);
          {
            bf16x8 da[NKS];
#pragma unroll
            for (int st = 0; st < NKS; ++st) da[st] = ld8(&sm.dO[buf][mt * 32 + l32][16 * st + 8 * g]);
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) {
              f32x16 dp = zero16();
#pragma unroll
              for (int st = 0; st < NKS; ++st) dp = mfma32(da[st], vb[nt][st], dp);
#pragma unroll
              for (int e = 0; e < 16; ++e) dp[e] = pv[nt][e] * (dp[e] - lr[e]);
              pb[nt][0] = pack_b(dp, 0);
              pb[nt][1] = pack_b(dp, 1);
            }
          }
#pragma unroll
          for (int t = 0; t < NDT; ++t) {
            const bf16x8 a0 = ld8(&sm.qt[buf][t * 32 + l32][mt * 32 + 8 * g]);
            const bf16x8 a1 = ld8(&sm.qt[buf][t * 32 + l32][mt * 32 + 16 + 8 * g]);
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) {
              adk[t][nt] = mfma32(a0, pb[nt][0], adk[t][nt]);
              adk[t][nt] = mfma32(a1, pb[nt][1], adk[t][nt]);
            }
          }
        }
      }
      if (more) lstore(buf ^ 1);
      __syncthreads();
    }
  }
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    const int jrow = jw + nt * 32 + l32;
    if (jrow >= T) continue;
    float* ov = dvp + ((int64_t)bh * T + jrow) * D;
    float* ok = dka + ((int64_t)bh * T + jrow) * D;
#pragma unroll
    for (int t = 0; t < NDT; ++t)
#pragma unroll
      for (int qq = 0; qq < 4; ++qq) {
        f32x4 a, bq;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          a[u] = adv[t][nt][4 * qq + u];
          bq[u] = adk[t][nt][4 * qq + u] * scale;
        }
        *reinterpret_cast<f32x4*>(ov + t * 32 + 8 * qq + 4 * g) = a;
        *reinterpret_cast<f32x4*>(ok + t * 32 + 8 * qq + 4 * g) = bq;
      }
  }
}

// ---------------------------------------------------------------------------
// Row sweep for dQ.  Workgroup = 256 query rows (heavy blocks first), wave w
// owns rows 64w..64w+63 (lane <-> row i).  Every key tile (K rows, V' rows,
// K^T in T-perm layout) is staged once per workgroup in LDS.
//   S^T[j][i] = K_j . Q_i, dP^T[j][i] = V'_j . dO_i, dS^T = P^T (dP^T - delta_i)
//   dQ^T[d][i] += K^T[d][j] dS^T[j][i]
// ---------------------------------------------------------------------------
template <int D>
struct DqSmem {
  bf16 k[2][64][D + 8];
  bf16 v[2][64][D + 8];
  bf16 kt[2][D][72];
};

template <int D>
__global__ __launch_bounds__(256) void lucid_attn_bwd_dq_kernel(
    const bf16* __restrict__ q, Strides qs, const bf16* __restrict__ k, Strides ks, const bf16* __restrict__ vpb,
    const bf16* __restrict__ dout, Strides dos, const bf16* __restrict__ kt, const float* __restrict__ lse,
    const float* __restrict__ delta, bf16* __restrict__ dq, Strides dqs, int Hq, int Hkv, int T, int BHq,
    float scale) {
  constexpr int NDT = D / 32;
  constexpr int NKS = D / 16;
  constexpr int CH = D / 32;
  __shared__ __attribute__((aligned(16))) DqSmem<D> sm;
  const int nblk = (T + 255) / 256;
  const int id = blockIdx.x;
  const int bhq = id % BHq;
  const int ib = nblk - 1 - id / BHq;
  const int b = bhq / Hq, hq = bhq - b * Hq;
  const int h = hq / (Hq / Hkv);
  const int bh = b * Hkv + h;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int g = lane >> 5, l32 = lane & 31;
  const int r0 = ib * 256;
  const int row0 = r0 + w * 64;
  const bf16* kh = k + b * ks.b + h * ks.h;
  const bf16* vh = vpb + (int64_t)bh * T * D;
  const bf16* kth = kt + (int64_t)bh * D * T;
  const float c = scale * LOG2E_F;

  bf16x8 qb[2][NKS], db[2][NKS];
  float li[2], di[2];
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    const int ir = min(row0 + nt * 32 + l32, T - 1);
#pragma unroll
    for (int st = 0; st < NKS; ++st) {
      qb[nt][st] = ld8(q + b * qs.b + hq * qs.h + (int64_t)ir * qs.t + 16 * st + 8 * g);
      db[nt][st] = ld8(dout + b * dos.b + hq * dos.h + (int64_t)ir * dos.t + 16 * st + 8 * g);
    }
    li[nt] = lse[(int64_t)bhq * T + ir];
    di[nt] = delta[(int64_t)bhq * T + ir];
  }
  f32x16 acc[NDT][2];
#pragma unroll
  for (int t = 0; t < NDT; ++t) {
    acc[t][0] = zero16();
    acc[t][1] = zero16();
  }
  const int ntile = (min(r0 + 256, T) + 63) / 64;
  const int last_w = row0 / 64;
  bf16x8 stg[3 * CH];
  auto gload = [&](int jt) {
    const int j0 = jt * 64;
    g2r_rows<D>(kh, ks.t, j0, stg);
    g2r_rows<D>(vh, D, j0, stg + CH);
    g2r_tp<D>(kth, T, j0, stg + 2 * CH);
  };
  auto lstore = [&](int buf) {
    r2l_rows<D>(sm.k[buf], stg);
    r2l_rows<D>(sm.v[buf], stg + CH);
    r2l_tp<D>(sm.kt[buf], stg + 2 * CH);
  };
  gload(0);
  lstore(0);
  __syncthreads();
  for (int jt = 0; jt < ntile; ++jt) {
    const int buf = jt & 1;
    const bool more = jt + 1 < ntile;
    if (more) gload(jt + 1);
    if (jt <= last_w && row0 < T) {
      const bool diag = (jt == last_w);
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        bf16x8 ka[NKS], va[NKS];
#pragma unroll
        for (int st = 0; st < NKS; ++st) {
          ka[st] = ld8(&sm.k[buf][mt * 32 + l32][16 * st + 8 * g]);
          va[st] = ld8(&sm.v[buf][mt * 32 + l32][16 * st + 8 * g]);
        }
        bf16x8 dsb[2][2];
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
          f32x16 sc = zero16(), dp = zero16();
#pragma unroll
          for (int st = 0; st < NKS; ++st) {
            sc = mfma32(ka[st], qb[nt][st], sc);
            dp = mfma32(va[st], db[nt][st], dp);
          }
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            float p = __builtin_amdgcn_exp2f(fmaf(sc[e], c, -li[nt]));
            if (diag && (mt * 32 + drow(e, g) > nt * 32 + l32)) p = 0.f;
            sc[e] = p * (dp[e] - di[nt]);
          }
          dsb[nt][0] = pack_b(sc, 0);
          dsb[nt][1] = pack_b(sc, 1);
        }
#pragma unroll
        for (int t = 0; t < NDT; ++t) {
          const bf16x8 a0 = ld8(&sm.kt[buf][t * 32 + l32][mt * 32 + 8 * g]);
          const bf16x8 a1 = ld8(&sm.kt[buf][t * 32 + l32][mt * 32 + 16 + 8 * g]);
#pragma unroll
          for (int nt = 0; nt < 2; ++nt) {
            acc[t][nt] = mfma32(a0, dsb[nt][0], acc[t][nt]);
            acc[t][nt] = mfma32(a1, dsb[nt][1], acc[t][nt]);
          }
        }
      }
    }
    if (more) lstore(buf ^ 1);
    __syncthreads();
  }
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    const int irow = row0 + nt * 32 + l32;
    if (irow >= T) continue;
    bf16* op = dq + b * dqs.b + hq * dqs.h + (int64_t)irow * dqs.t;
#pragma unroll
    for (int t = 0; t < NDT; ++t)
#pragma unroll
      for (int qq = 0; qq < 4; ++qq) {
        bf16x4 bb;
#pragma unroll
        for (int u = 0; u < 4; ++u) bb[u] = (bf16)(acc[t][nt][4 * qq + u] * scale);
        *reinterpret_cast<bf16x4*>(op + t * 32 + 8 * qq + 4 * g) = bb;
      }
  }
}

// ---------------------------------------------------------------------------
// Chained transposed solve dV = P^-T dV' (Lucid_Tril_Solver.backward :328-334)
// and the column sums C_J = sum_{I >= J} M_IJ^T K^_I.
// WG id -> (J = NT-1 - id/BH, bh = id % BH): ids grow as J falls, so block J
// waits only on later blocks that have lower ids.  Counter value n means
// blocks NT-1 .. NT-n are published.
// wave w: ch = w & 1 -> columns J0 + 32ch .. (lane <-> column),
//         ih = w >> 1 -> rows I0 + 32ih .. of every later 64-row block.
// ---------------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(256) void lucid_precond_bwd_col_kernel(
    const bf16* __restrict__ k, Strides ks, int Hkv, int T, int BH, const float* __restrict__ rinv, float scale,
    const bf16* __restrict__ kt, const bf16* __restrict__ vpb, const float* __restrict__ pinv,
    const float* __restrict__ dvp, bf16* __restrict__ dvb, bf16* __restrict__ dvt, bf16* __restrict__ dv_out,
    Strides dvs, float* __restrict__ colsum, int* __restrict__ counters) {
  constexpr int NDT = D / 32;
  constexpr int NKS = D / 16;
  __shared__ __attribute__((aligned(16))) float Ps[64][68];    // P_JJ, lower
  __shared__ __attribute__((aligned(16))) float Xt[64][68];    // Xt[c][r] = (P_JJ^-1)[r][c]
  __shared__ __attribute__((aligned(16))) float Rt[D][68];     // reductions, R^T
  __shared__ __attribute__((aligned(16))) bf16 dvl[64][D + 8]; // dV_J rows (bf16)

  const int NT = T / 64;
  const int id = blockIdx.x;
  const int J = NT - 1 - id / BH, bh = id - (id / BH) * BH;
  const int b = bh / Hkv, h = bh - b * Hkv;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int g = lane >> 5, l32 = lane & 31;
  const int ch = w & 1, ih = w >> 1;
  const int J0 = J * 64;
  const int jcol = J0 + ch * 32 + l32;
  const bf16* kh = k + b * ks.b + h * ks.h;
  const float* rv = rinv + (int64_t)bh * T;
  const bf16* kth = kt + (int64_t)bh * D * T;
  const bf16* dvth = dvt + (int64_t)bh * D * T;
  const bf16* dvbh = dvb + (int64_t)bh * T * D;
  const float sl2 = scale * LOG2E_F;
  const float c0 = LOG2E_F / scale;

  bf16x8 kbJ[NKS], vbJ[NKS];
#pragma unroll
  for (int s = 0; s < NKS; ++s) {
    kbJ[s] = ld8(kh + (int64_t)jcol * ks.t + 16 * s + 8 * g);
    vbJ[s] = ld8(vpb + ((int64_t)bh * T + jcol) * D + 16 * s + 8 * g);
  }
  const float aJ = sl2 * rv[jcol];
  {
    f32x16 sd = zero16();
#pragma unroll
    for (int s = 0; s < NKS; ++s)
      sd = mfma32(ld8(kh + (int64_t)(J0 + ih * 32 + l32) * ks.t + 16 * s + 8 * g), kbJ[s], sd);
    const int n = ch * 32 + l32;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int m = ih * 32 + drow(e, g);
      Ps[m][n] = (n <= m) ? __builtin_amdgcn_exp2f(sd[e] * aJ * rv[J0 + m] - c0) : 0.f;
    }
  }
  {
    const float* xp = pinv + ((int64_t)bh * NT + J) * 4096;
    for (int idx = tid; idx < 4096; idx += 256) Xt[idx & 63][idx >> 6] = xp[idx];
  }

  f32x16 adv[NDT], acs[NDT];
#pragma unroll
  for (int t = 0; t < NDT; ++t) {
    adv[t] = zero16();
    acs[t] = zero16();
  }
  int ready = 0;
  for (int I = NT - 1; I > J; --I) {
    const int need = NT - 1 - I;
    if (need >= ready) ready = wait_counter_gt(counters + bh, need);
    const int I0 = I * 64 + ih * 32;
    f32x16 s = zero16(), gg = zero16();
#pragma unroll
    for (int st = 0; st < NKS; ++st) {
      s = mfma32(ld8(kh + (int64_t)(I0 + l32) * ks.t + 16 * st + 8 * g), kbJ[st], s);
      gg = mfma32(ld8(dvbh + (int64_t)(I0 + l32) * D + 16 * st + 8 * g), vbJ[st], gg);
    }
    float rI[16];
    load_rows16(rv + I0, g, rI);
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const float p = __builtin_amdgcn_exp2f(s[e] * aJ * rI[e] - c0);
      s[e] = p;
      gg[e] = gg[e] * p * rI[e];
    }
    const bf16x8 p0 = pack_b(s, 0), p1 = pack_b(s, 1);
    const bf16x8 m0 = pack_b(gg, 0), m1 = pack_b(gg, 1);
#pragma unroll
    for (int t = 0; t < NDT; ++t) {
      const bf16* ap = dvth + (int64_t)(t * 32 + l32) * T + I0 + 8 * g;
      adv[t] = mfma32(ld8(ap), p0, adv[t]);
      adv[t] = mfma32(ld8(ap + 16), p1, adv[t]);
      const bf16* kp = kth + (int64_t)(t * 32 + l32) * T + I0 + 8 * g;
      acs[t] = mfma32(ld8(kp), m0, acs[t]);
      acs[t] = mfma32(ld8(kp + 16), m1, acs[t]);
    }
  }

  // ---- R_J = dV'_J - sum_{I>J} P_IJ^T dV_I (reduce the two row halves) ----
  if (ih == 1) {
#pragma unroll
    for (int t = 0; t < NDT; ++t)
#pragma unroll
      for (int e = 0; e < 16; ++e) Rt[t * 32 + drow(e, g)][ch * 32 + l32] = adv[t][e];
  }
  __syncthreads();
  if (ih == 0) {
    const float* src = dvp + ((int64_t)bh * T + jcol) * D;
#pragma unroll
    for (int t = 0; t < NDT; ++t)
#pragma unroll
      for (int qq = 0; qq < 4; ++qq) {
        const int d0 = t * 32 + 8 * qq + 4 * g;
        const f32x4 x = *reinterpret_cast<const f32x4*>(src + d0);
#pragma unroll
        for (int u = 0; u < 4; ++u)
          Rt[d0 + u][ch * 32 + l32] = x[u] - (adv[t][4 * qq + u] + Rt[d0 + u][ch * 32 + l32]);
      }
  }
  __syncthreads();

  // ---- dV^T[d][c] = sum_r R^T[d][r] X[r][c]  (X lower: r >= c) ----
  for (int tile = w; tile < NDT * 2; tile += 4) {
    const int dt = tile >> 1, chh = tile & 1;
    f32x16 o = zero16();
    for (int s = chh ? 2 : 0; s < 4; ++s) {
      bf16x8 ah, al, bh8, bl;
      split8(&Rt[dt * 32 + l32][16 * s + 8 * g], ah, al);
      split8(&Xt[chh * 32 + l32][16 * s + 8 * g], bh8, bl);
      o = mfma32(ah, bh8, o);
      o = mfma32(ah, bl, o);
      o = mfma32(al, bh8, o);
    }
    const int cl = chh * 32 + l32;
    const int r = J0 + cl;
    const int slot = (r & ~15) | jmap(r & 15);
    bf16* ob = dvb + ((int64_t)bh * T + r) * D;
    bf16* ou = dv_out + b * dvs.b + h * dvs.h + (int64_t)r * dvs.t;
#pragma unroll
    for (int qq = 0; qq < 4; ++qq) {
      const int d0 = dt * 32 + 8 * qq + 4 * g;
      bf16x4 bb;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        bb[u] = (bf16)o[4 * qq + u];
        vpth_w(dvt, bh, D, T, d0 + u, slot, bb[u]);
        dvl[cl][d0 + u] = bb[u];
      }
      *reinterpret_cast<bf16x4*>(ob + d0) = bb;
      *reinterpret_cast<bf16x4*>(ou + d0) = bb;
    }
  }
  publish_counter(counters + bh, NT - J);

  // ---- diagonal block of the column sums: M_JJ = tril((dV_J V'_J^T) * P_JJ) ----
  {
    f32x16 gg = zero16();
#pragma unroll
    for (int st = 0; st < NKS; ++st) gg = mfma32(ld8(&dvl[ih * 32 + l32][16 * st + 8 * g]), vbJ[st], gg);
    float rr[16];
    load_rows16(rv + J0 + ih * 32, g, rr);
    const int n = ch * 32 + l32;
#pragma unroll
    for (int e = 0; e < 16; ++e) gg[e] = gg[e] * Ps[ih * 32 + drow(e, g)][n] * rr[e];
    const bf16x8 m0 = pack_b(gg, 0), m1 = pack_b(gg, 1);
#pragma unroll
    for (int t = 0; t < NDT; ++t) {
      const bf16* kp = kth + (int64_t)(t * 32 + l32) * T + J0 + ih * 32 + 8 * g;
      acs[t] = mfma32(ld8(kp), m0, acs[t]);
      acs[t] = mfma32(ld8(kp + 16), m1, acs[t]);
    }
  }
  __syncthreads();
  if (ih == 1) {
#pragma unroll
    for (int t = 0; t < NDT; ++t)
#pragma unroll
      for (int e = 0; e < 16; ++e) Rt[t * 32 + drow(e, g)][ch * 32 + l32] = acs[t][e];
  }
  __syncthreads();
  if (ih == 0) {
    float* dst = colsum + ((int64_t)bh * T + jcol) * D;
#pragma unroll
    for (int t = 0; t < NDT; ++t)
#pragma unroll
      for (int qq = 0; qq < 4; ++qq) {
        const int d0 = t * 32 + 8 * qq + 4 * g;
        f32x4 x;
#pragma unroll
        for (int u = 0; u < 4; ++u) x[u] = acs[t][4 * qq + u] + Rt[d0 + u][ch * 32 + l32];
        *reinterpret_cast<f32x4*>(dst + d0) = x;
      }
  }
}

// ---------------------------------------------------------------------------
// Row sums R_I = sum_{J <= I} M_IJ K^_J, then dK^ = -s (R + C), RMSNorm
// backward and the attention dK.  No chain: every dV is known.
// wave w: ih = w & 1 -> rows (lane <-> row I), jh = w >> 1 -> key half.
// ---------------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(256) void lucid_precond_bwd_row_kernel(
    const bf16* __restrict__ k, Strides ks, int Hkv, int T, int BH, const float* __restrict__ rinv, float scale,
    const bf16* __restrict__ kt, const bf16* __restrict__ vpb, const bf16* __restrict__ dvb,
    const float* __restrict__ colsum, const float* __restrict__ dka, bf16* __restrict__ dk_out, Strides dks) {
  constexpr int NDT = D / 32;
  constexpr int NKS = D / 16;
  __shared__ __attribute__((aligned(16))) float Rt[D][68];
  const int NT = T / 64;
  const int id = blockIdx.x;
  const int I = NT - 1 - id / BH, bh = id - (id / BH) * BH;
  const int b = bh / Hkv, h = bh - b * Hkv;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int g = lane >> 5, l32 = lane & 31;
  const int ih = w & 1, jh = w >> 1;
  const int irow = I * 64 + ih * 32 + l32;
  const bf16* kh = k + b * ks.b + h * ks.h;
  const float* rv = rinv + (int64_t)bh * T;
  const bf16* kth = kt + (int64_t)bh * D * T;
  const bf16* vh = vpb + (int64_t)bh * T * D;
  const float sl2 = scale * LOG2E_F;
  const float c0 = LOG2E_F / scale;

  bf16x8 kbI[NKS], dbI[NKS];
#pragma unroll
  for (int s = 0; s < NKS; ++s) {
    kbI[s] = ld8(kh + (int64_t)irow * ks.t + 16 * s + 8 * g);
    dbI[s] = ld8(dvb + ((int64_t)bh * T + irow) * D + 16 * s + 8 * g);
  }
  const float ri = rv[irow];
  const float aI = sl2 * ri;
  f32x16 acc[NDT];
#pragma unroll
  for (int t = 0; t < NDT; ++t) acc[t] = zero16();
  for (int J = 0; J <= I; ++J) {
    const int J0 = J * 64 + jh * 32;
    f32x16 s = zero16(), gg = zero16();
#pragma unroll
    for (int st = 0; st < NKS; ++st) {
      s = mfma32(ld8(kh + (int64_t)(J0 + l32) * ks.t + 16 * st + 8 * g), kbI[st], s);
      gg = mfma32(ld8(vh + (int64_t)(J0 + l32) * D + 16 * st + 8 * g), dbI[st], gg);
    }
    float rJ[16];
    load_rows16(rv + J0, g, rJ);
    const bool diag = (J == I);
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      float p = __builtin_amdgcn_exp2f(s[e] * aI * rJ[e] - c0);
      if (diag && (J0 + drow(e, g) > irow)) p = 0.f;
      gg[e] = gg[e] * p * rJ[e];
    }
    const bf16x8 m0 = pack_b(gg, 0), m1 = pack_b(gg, 1);
#pragma unroll
    for (int t = 0; t < NDT; ++t) {
      const bf16* kp = kth + (int64_t)(t * 32 + l32) * T + J0 + 8 * g;
      acc[t] = mfma32(ld8(kp), m0, acc[t]);
      acc[t] = mfma32(ld8(kp + 16), m1, acc[t]);
    }
  }
  if (jh == 1) {
#pragma unroll
    for (int t = 0; t < NDT; ++t)
#pragma unroll
      for (int e = 0; e < 16; ++e) Rt[t * 32 + drow(e, g)][ih * 32 + l32] = acc[t][e];
  }
  __syncthreads();
  if (jh == 0) {
    const float* cs = colsum + ((int64_t)bh * T + irow) * D;
    const float* da = dka + ((int64_t)bh * T + irow) * D;
    const bf16* kr = kh + (int64_t)irow * ks.t;
    float dkh[NDT][16], khat[NDT][16];
    float dotp = 0.f;
#pragma unroll
    for (int t = 0; t < NDT; ++t)
#pragma unroll
      for (int qq = 0; qq < 4; ++qq) {
        const int d0 = t * 32 + 8 * qq + 4 * g;
        const f32x4 cv = *reinterpret_cast<const f32x4*>(cs + d0);
        const bf16x4 kv = *reinterpret_cast<const bf16x4*>(kr + d0);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int e = 4 * qq + u;
          const float x = -scale * (acc[t][e] + Rt[d0 + u][ih * 32 + l32] + cv[u]);
          const float kk = ri * (float)kv[u];
          dkh[t][e] = x;
          khat[t][e] = kk;
          dotp += x * kk;
        }
      }
    dotp += wave_xor32(dotp);
    const float f = dotp / (float)D;
    bf16* op = dk_out + b * dks.b + h * dks.h + (int64_t)irow * dks.t;
#pragma unroll
    for (int t = 0; t < NDT; ++t)
#pragma unroll
      for (int qq = 0; qq < 4; ++qq) {
        const int d0 = t * 32 + 8 * qq + 4 * g;
        const f32x4 av = *reinterpret_cast<const f32x4*>(da + d0);
        bf16x4 bb;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int e = 4 * qq + u;
          bb[u] = (bf16)(ri * (dkh[t][e] - khat[t][e] * f) + av[u]);
        }
        *reinterpret_cast<bf16x4*>(op + d0) = bb;
      }
  }
}

}  // namespace lucid
