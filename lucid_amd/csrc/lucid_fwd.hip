// LUCID attention forward on CDNA4 (gfx950).
//
//   K^ = K / sqrt(mean_d K^2 + eps)                       (modeling_lucid.py:409, :564)
//   P_ij = exp(s K^_i.K^_j - 1/s), j <= i                 (:565-569)
//   V'  = P^-1 V  (chained block forward substitution)    (:570, :285-312)
//   O   = softmax(s Q K^T, causal) V'                     (:520-530)
//
// Kernels (all 256 threads = 4 waves, MFMA 32x32x16 bf16, fp32 accumulate):
//   lucid_prep_kernel        per-row 1/rms of K, K^T in T-perm layout, zero chain counters
//   lucid_precond_fwd_kernel chained solve, one workgroup per (64-row block, kv head);
//                            block i waits on a per-head progress counter for V'_j, j < i
//   lucid_attn_fwd_kernel    causal online-softmax attention on V' (256 query rows / WG, LDS tiles)
#include "lucid_common.h"

namespace lucid {

// ---------------------------------------------------------------------------
// prep: rinv[bh][t] = 1/sqrt(mean K^2 + eps); kt[bh][d][perm(t)] = K[t][d]
// grid (T/64, B*Hkv)
// ---------------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(256) void lucid_prep_kernel(const bf16* __restrict__ k, Strides ks, int Hkv, int T,
                                                         float eps, float* __restrict__ rinv,
                                                         bf16* __restrict__ kt, int* __restrict__ counters) {
  constexpr int SEG = D / 4;
  __shared__ bf16 tile[D][64 + 8];
  const int blk = blockIdx.x, bh = blockIdx.y;
  const int b = bh / Hkv, h = bh - b * Hkv;
  const int tid = threadIdx.x;
  const bf16* kp = k + b * ks.b + h * ks.h + (int64_t)blk * 64 * ks.t;
  const int row = tid >> 2, seg = tid & 3;
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < SEG; c += 8) {
    bf16x8 x = ld8(kp + row * ks.t + seg * SEG + c);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float f = (float)x[e];
      ss += f * f;
      tile[seg * SEG + c + e][row] = x[e];
    }
  }
  ss += __shfl_xor(ss, 1, 64);
  ss += __shfl_xor(ss, 2, 64);
  if (seg == 0) rinv[(int64_t)bh * T + blk * 64 + row] = 1.0f / sqrtf(ss / (float)D + eps);
  if (blk == 0 && tid == 0) counters[bh] = 0;
  __syncthreads();
  // T-perm rows: kt[bh][d][blk*64 + slot], slot kappa holds t = jmap(kappa)
  for (int idx = tid; idx < D * 8; idx += 256) {
    const int dd = idx >> 3, c8 = idx & 7;
    bf16x8 out;
#pragma unroll
    for (int e = 0; e < 8; ++e) out[e] = tile[dd][(c8 >> 1) * 16 + jmap((c8 & 1) * 8 + e)];
    *reinterpret_cast<bf16x8*>(kt + ((int64_t)bh * D + dd) * T + blk * 64 + c8 * 8) = out;
  }
}

// ---------------------------------------------------------------------------
// Chained preconditioner solve.  Workgroup id -> (i = id / BH, bh = id % BH):
// ids grow with i, so every wait is on a lower id (in-order dispatch keeps the
// chain deadlock free) and the blocks of one head share an XCD when BH % 8 == 0.
//
// wave w: ih = w & 1 selects rows i0 + 32*ih .. +32 (lane <-> row),
//         jh = w >> 1 selects keys j0 + 32*jh .. +32 of every 64-key tile.
// acc^T[d][i] = sum_{j < i0} V'^T[d][j] P[i][j]  (MFMA, bf16 operands)
// V'_i = X (V_i - acc), X = P_ii^-1 computed in fp32 by wave 0 before the wait,
// applied with a 3-term bf16 split (hi*hi + hi*lo + lo*hi) for ~fp32 accuracy.
// ---------------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(256) void lucid_precond_fwd_kernel(
    const bf16* __restrict__ k, Strides ks, const bf16* __restrict__ v, Strides vs, int Hkv, int T, int BH,
    const float* __restrict__ rinv, float scale, float* __restrict__ vp32, bf16* __restrict__ vpb,
    bf16* __restrict__ vpt, float* __restrict__ pinv, int* __restrict__ counters) {
  constexpr int NDT = D / 32;  // 32-row d tiles
  constexpr int NKS = D / 16;  // 16-deep k steps over d
  __shared__ __attribute__((aligned(16))) float Ps[64][68];           // P_ii, then X = P_ii^-1 (row-major [r][c])
  __shared__ __attribute__((aligned(16))) float Rt[D][68];            // R^T[d][c] (also used for the cross-wave reduction)

  const int id = blockIdx.x;
  const int i = id / BH, bh = id - (id / BH) * BH;
  const int b = bh / Hkv, h = bh - b * Hkv;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int g = lane >> 5, l32 = lane & 31;
  const int ih = w & 1, jh = w >> 1;
  const int i0 = i * 64;
  const bf16* kh = k + b * ks.b + h * ks.h;
  const bf16* vh = v + b * vs.b + h * vs.h;
  const float* rv = rinv + (int64_t)bh * T;
  const bf16* vpth = vpt + (int64_t)bh * D * T;
  const float sl2 = scale * LOG2E_F;
  const float c0 = LOG2E_F / scale;

  bf16x8 kbi[NKS];
#pragma unroll
  for (int s = 0; s < NKS; ++s) kbi[s] = ld8(kh + (int64_t)(i0 + ih * 32 + l32) * ks.t + 16 * s + 8 * g);
  const float ai = sl2 * rv[i0 + ih * 32 + l32];

  // ---- diagonal block P_ii (symmetric S, lower mask) ----
  {
    f32x16 sd = zero16();
#pragma unroll
    for (int s = 0; s < NKS; ++s)
      sd = mfma32(ld8(kh + (int64_t)(i0 + jh * 32 + l32) * ks.t + 16 * s + 8 * g), kbi[s], sd);
    const int n = ih * 32 + l32;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int m = jh * 32 + drow(e, g);
      Ps[m][n] = (n <= m) ? __builtin_amdgcn_exp2f(sd[e] * ai * rv[i0 + m] - c0) : 0.f;
    }
  }
  __syncthreads();
  if (w == 0) invert_lower64(Ps, lane, pinv + ((int64_t)bh * (T / 64) + i) * 4096);

  // ---- off-diagonal accumulation over all earlier blocks ----
  f32x16 acc[NDT];
#pragma unroll
  for (int t = 0; t < NDT; ++t) acc[t] = zero16();
  int ready = 0;
  for (int j = 0; j < i; ++j) {
    if (j >= ready) ready = wait_counter_gt(counters + bh, j);
    const int j0 = j * 64 + jh * 32;
    f32x16 s = zero16();
#pragma unroll
    for (int st = 0; st < NKS; ++st) s = mfma32(ld8(kh + (int64_t)(j0 + l32) * ks.t + 16 * st + 8 * g), kbi[st], s);
    float rj[16];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      f32x4 t4 = *reinterpret_cast<const f32x4*>(rv + j0 + 8 * q + 4 * g);
      rj[4 * q] = t4[0]; rj[4 * q + 1] = t4[1]; rj[4 * q + 2] = t4[2]; rj[4 * q + 3] = t4[3];
    }
#pragma unroll
    for (int e = 0; e < 16; ++e) s[e] = __builtin_amdgcn_exp2f(s[e] * ai * rj[e] - c0);
    const bf16x8 p0 = pack_b(s, 0), p1 = pack_b(s, 1);
#pragma unroll
    for (int t = 0; t < NDT; ++t) {
      const bf16* ap = vpth + (int64_t)(t * 32 + l32) * T + j0 + 8 * g;
      acc[t] = mfma32(ld8(ap), p0, acc[t]);
      acc[t] = mfma32(ld8(ap + 16), p1, acc[t]);
    }
  }

  // ---- reduce the two key halves: waves jh=1 hand their partials to jh=0 ----
  if (jh == 1) {
#pragma unroll
    for (int t = 0; t < NDT; ++t)
#pragma unroll
      for (int e = 0; e < 16; ++e) Rt[t * 32 + drow(e, g)][ih * 32 + l32] = acc[t][e];
  }
  __syncthreads();  // also orders wave 0's X in Ps before its use below
  if (jh == 0) {
    const int r = i0 + ih * 32 + l32;
#pragma unroll
    for (int t = 0; t < NDT; ++t)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int d0 = t * 32 + 8 * q + 4 * g;
        bf16x4 vv = *reinterpret_cast<const bf16x4*>(vh + (int64_t)r * vs.t + d0);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int e = 4 * q + u;
          Rt[d0 + u][ih * 32 + l32] = (float)vv[u] - (acc[t][e] + Rt[d0 + u][ih * 32 + l32]);
        }
      }
  }
  __syncthreads();

  // ---- diagonal solve V'^T[d][r] = sum_c R^T[d][c] X[r][c] ----
  for (int tile = w; tile < NDT * 2; tile += 4) {
    const int dt = tile >> 1, rh = tile & 1;
    f32x16 o = zero16();
    const int kmax = rh ? 4 : 2;  // X[r][c] = 0 for c > r
    for (int s = 0; s < kmax; ++s) {
      bf16x8 ah, al, bh8, bl;
      split8(&Rt[dt * 32 + l32][16 * s + 8 * g], ah, al);
      split8(&Ps[rh * 32 + l32][16 * s + 8 * g], bh8, bl);
      o = mfma32(ah, bh8, o);
      o = mfma32(ah, bl, o);
      o = mfma32(al, bh8, o);
    }
    // lane: r = rh*32 + l32; elements: d = dt*32 + drow(e, g)
    const int r = i0 + rh * 32 + l32;
    float* out32 = vp32 + ((int64_t)bh * T + r) * D;
    bf16* outb = vpb + ((int64_t)bh * T + r) * D;
    const int slot = (r & ~15) | jmap(r & 15);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int d0 = dt * 32 + 8 * q + 4 * g;
      f32x4 f;
      bf16x4 bb;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        f[u] = o[4 * q + u];
        bb[u] = (bf16)o[4 * q + u];
        vpth_w(vpt, bh, D, T, d0 + u, slot, bb[u]);
      }
      *reinterpret_cast<f32x4*>(out32 + d0) = f;
      *reinterpret_cast<bf16x4*>(outb + d0) = bb;
    }
  }
  publish_counter(counters + bh, i + 1);
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
// P = exp2(s*log2e*S - lse2)).
// ---------------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(256) void lucid_attn_fwd_kernel(const bf16* __restrict__ q, Strides qs,
                                                             const bf16* __restrict__ k, Strides ks,
                                                             const bf16* __restrict__ vpt, bf16* __restrict__ o,
                                                             Strides os, float* __restrict__ lse, int Hq, int Hkv,
                                                             int T, int BHq, float scale) {
  constexpr int NDT = D / 32;
  constexpr int NKS = D / 16;
  constexpr int CH = D / 32;  // 16-byte chunks per thread for each of the K and V'^T tiles
  __shared__ __attribute__((aligned(16))) bf16 lk[2][64][D + 8];
  __shared__ __attribute__((aligned(16))) bf16 lv[2][D][64 + 8];

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
  const bf16* qh = q + b * qs.b + hq * qs.h;
  const bf16* kh = k + b * ks.b + h * ks.h;
  const bf16* vth = vpt + (int64_t)bh * D * T;
  const float c = scale * LOG2E_F;

  bf16x8 qb[2][NKS];
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    const int rq = min(row0 + nt * 32 + l32, T - 1);
#pragma unroll
    for (int st = 0; st < NKS; ++st) qb[nt][st] = ld8(qh + (int64_t)rq * qs.t + 16 * st + 8 * g);
  }
  f32x16 oacc[NDT][2];
#pragma unroll
  for (int t = 0; t < NDT; ++t) {
    oacc[t][0] = zero16();
    oacc[t][1] = zero16();
  }
  float m[2] = {-1e30f, -1e30f}, lsum[2] = {0.f, 0.f};

  const int ntile = (min(r0 + 256, T) + 63) / 64;
  const int last_w = row0 / 64;  // this wave's diagonal tile
  bf16x8 stg[2 * CH];
  auto gload = [&](int j0) {
#pragma unroll
    for (int u = 0; u < CH; ++u) {
      const int cidx = tid + 256 * u;
      const int kr = cidx / (D / 8), kc = cidx % (D / 8);
      stg[u] = ld8(kh + (int64_t)(j0 + kr) * ks.t + kc * 8);
      const int vr = cidx >> 3, vc = cidx & 7;
      stg[CH + u] = ld8(vth + (int64_t)vr * T + j0 + vc * 8);
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
      const int j0 = jt * 64;
      f32x16 s[2][2];
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        bf16x8 ka[NKS];
#pragma unroll
        for (int st = 0; st < NKS; ++st) ka[st] = ld8(&lk[buf][mt * 32 + l32][16 * st + 8 * g]);
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
          s[mt][nt] = zero16();
#pragma unroll
          for (int st = 0; st < NKS; ++st) s[mt][nt] = mfma32(ka[st], qb[nt][st], s[mt][nt]);
        }
      }
      if (jt == last_w) {
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
          for (int nt = 0; nt < 2; ++nt)
#pragma unroll
            for (int e = 0; e < 16; ++e)
              if (mt * 32 + drow(e, g) > nt * 32 + l32) s[mt][nt][e] = -INFINITY;
      }
      bf16x8 pb[2][4];
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) {
        float mx = -INFINITY;
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
          for (int e = 0; e < 16; ++e) mx = fmaxf(mx, s[mt][nt][e]);
        mx = fmaxf(mx, wave_xor32(mx)) * c;
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
      }
#pragma unroll
      for (int t = 0; t < NDT; ++t) {
        bf16x8 va[4];
#pragma unroll
        for (int k4 = 0; k4 < 4; ++k4) va[k4] = ld8(&lv[buf][t * 32 + l32][16 * k4 + 8 * g]);
#pragma unroll
        for (int nt = 0; nt < 2; ++nt)
#pragma unroll
          for (int k4 = 0; k4 < 4; ++k4) oacc[t][nt] = mfma32(va[k4], pb[nt][k4], oacc[t][nt]);
      }
    }
    if (more) lstore(buf ^ 1);
    __syncthreads();
  }
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    const int irow = row0 + nt * 32 + l32;
    const float ls = lsum[nt] + wave_xor32(lsum[nt]);
    if (irow < T) {
      const float inv = 1.0f / ls;
      bf16* op = o + b * os.b + hq * os.h + (int64_t)irow * os.t;
#pragma unroll
      for (int t = 0; t < NDT; ++t)
#pragma unroll
        for (int qq = 0; qq < 4; ++qq) {
          bf16x4 bb;
#pragma unroll
          for (int u = 0; u < 4; ++u) bb[u] = (bf16)(oacc[t][nt][4 * qq + u] * inv);
          *reinterpret_cast<bf16x4*>(op + t * 32 + 8 * qq + 4 * g) = bb;
        }
      if (g == 0) lse[(int64_t)bhq * T + irow] = m[nt] + log2f(ls);
    }
  }
}

}  // namespace lucid
