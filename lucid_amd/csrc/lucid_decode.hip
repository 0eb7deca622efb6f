// LUCID decoding step on CDNA4 (gfx950): L new tokens per sequence against a (K, V')
// cache, with the exact preconditioner rows (modeling_lucid.py:576-598 is the reference
// seam; its V' update drops the division by the diagonal P_tt and the coupling among the
// new tokens, both kept here so that decoded rows equal the same rows of a prefill):
//   P_tj = exp(s r_t r_j (k_t . k_j) - 1/s),  r = 1 / rms(k)  (j < t, cached or new)
//   v'_t = (v_t - sum_{j<t} P_tj v'_j) / P_tt,  P_tt = exp(s dn ms_t / (ms_t + eps) - 1/s)
//   o_tg = softmax_j(s q_tg . k_j) v'_j over j <= t, for the G query heads of the kv head
// (dn: the head dim; rows may be zero-padded beyond it, ms = sum k^2 / dn).
// The cached part of both sums reads every cached row once (memory bound), so one pass
// over the cache computes it for all L tokens together, split over the sequence
// (flash-decoding):
//   lucid_decode_split_kernel    per (split, kv head): partial sum_j P_tj v'_j of every new
//                                token and the online-softmax state (m, l, O) of every
//                                (token, query head), as MFMA tiles (the L (G + 1) query
//                                heads and new keys are the columns of one score tile)
//   lucid_decode_combine_kernel  per (kv head, query head): merges the splits, solves the
//                                new tokens' rows in order (their coupling among each
//                                other), adds the new keys to each token's softmax, writes
//                                the outputs and appends (k_t, v'_t) to the caches
#include "lucid_common.h"

namespace lucid {

constexpr float DEC_NEG = -1e30f;  // finite "minus infinity" for empty softmax states

// Tokens of one pass: the L (G + 1) columns of a 32-column score tile.  G = 0 is the
// generic instance (the group size Gs a runtime argument, 3 <= Gs <= 31): its per-token
// arrays hold the 8 tokens of its smallest group.
template <int G>
constexpr int decode_tokens_per_pass() {
  return G > 0 ? 32 / (G + 1) : 8;
}

struct DecodePartials {
  float* a;  // [nsplit][BH][L][D]     sum_j P_tj v'_j over the split's cached rows
  float* m;  // [nsplit][BH][L*Gs]     running max (log2 domain), column t*Gs + g
  float* l;  // [nsplit][BH][L*Gs]     running sum
  float* o;  // [nsplit][BH][L*Gs][D]  unnormalised output
};

// Split pass on the matrix cores.  Each wave sweeps its own 32-key tiles of the split
// (tiles w, w+4, ...) and computes, per tile, one MFMA score tile
//   S^T[j][c] = K_j . X_c,  column c = t (G + 1) + i:  X_c = q_{t, hG+i} (i < G),  k_t (i = G),
// other columns zero, so every query head and the preconditioner row of every new token
// share one product.  Query columns take the online softmax p = exp2(s' S - m_c); key
// columns take p = exp2(s' r_t r_j S - 1/s log2 e), with 1/rms r_j of the cached key from
// the key registers and r_t of the column's own key.  O^T[d][c] += V'^T[d][j] p^T[j][c]
// (V' rows staged per wave into LDS by direct loads and read transposed) accumulates the
// outputs and, in the key columns, sum_j P_tj v'_j.  Keys reach registers one tile ahead;
// no barrier in the sweep.  Every new token sees every cached row (all are earlier).
// The columns hold the Gs query heads g0 .. g0+Gs-1 of the kv head's Gt (query head
// h Gt + g0 + i); G > 0 fixes Gs = G at compile time, G = 0 takes Gs at run time.  A key
// column's partials do not depend on the other columns of the tile.
template <int D, int G>
struct DecodeMfmaSmem {
  union {
    bf16 v[4][2][32 * D];  // per wave, double buffered, swizzled (chunk c of row r at c ^ (r & 7))
    struct {
      float so[4][32][D];  // per wave: the columns of O^T
      float m[4][32], l[4][32];
    } fin;
  } u;
  float nn[4][32];  // per wave: squared norms of the tile's keys
};

template <int D, int G>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void lucid_decode_split_kernel(
    const bf16* __restrict__ q, Strides qs, const bf16* __restrict__ kn, Strides kns,
    const bf16* __restrict__ kc, Strides kcs, const bf16* __restrict__ vc, Strides vcs, int Hkv, int Tp, int KS,
    int L, float scale, float eps, float dn, DecodePartials part, int Gs, int Gt, int g0) {
  constexpr int NKS = D / 16, NDT = D / 32, CPR = D / 8, NST = 32 * CPR / 64;  // NST: staging loads per tile
  static_assert(G + 1 <= 32, "query heads + the preconditioner row must fit one 32-column tile");
  const int GG = G > 0 ? G : Gs;  // query columns per token (GG + 1 <= 32, checked by the host)
  __shared__ __attribute__((aligned(16))) DecodeMfmaSmem<D, G> sm;
  const int s = blockIdx.x, bh = blockIdx.y, BH = gridDim.y;
  const int b = bh / Hkv, h = bh - b * Hkv;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 5, l32 = lane & 31;
  const int col = l32;  // score / output column of this lane
  const int tok = col / (GG + 1), hi = col - tok * (GG + 1);
  const bool valid = tok < L, isq = valid && hi < GG, isk = valid && hi == GG;
  const int j0 = s * KS, j1 = min(Tp, j0 + KS);

  // B operand: column col of X^T (k = d), zero for the padding columns
  bf16x8 xb[NKS];
  float nt = 0.f;
#pragma unroll
  for (int st = 0; st < NKS; ++st) {
    bf16x8 x;
    if (isq) {
      x = ld8(q + b * qs.b + (h * Gt + g0 + hi) * qs.h + (int64_t)tok * qs.t + 16 * st + 8 * g);
    } else if (isk) {
      x = ld8(kn + b * kns.b + h * kns.h + (int64_t)tok * kns.t + 16 * st + 8 * g);
#pragma unroll
      for (int e = 0; e < 8; ++e) nt = fmaf((float)x[e], (float)x[e], nt);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = (bf16)0.f;
    }
    xb[st] = x;
  }
  nt = wave_sum32(nt);  // squared norm of this column's key (both lane halves)
  const float rt = rsqrtf(nt / dn + eps);
  const float sl2 = scale * LOG2E_F, c1 = sl2 * rt, c0 = LOG2E_F / scale;

  f32x16 oacc[NDT];
#pragma unroll
  for (int t = 0; t < NDT; ++t) oacc[t] = zero16();
  float m = DEC_NEG, l = 0.f;

  const bf16* kbase = kc + b * kcs.b + h * kcs.h;
  const bf16* vbase = vc + b * vcs.b + h * vcs.h;
  const int ntile = (j1 - j0 + 31) / 32;  // 32-key tiles of the split; wave w takes w, w+4, ...
  bf16x8 kcur[NKS], knx[NKS];  // this tile's and the next tile's key rows
  auto kload = [&](int t, bf16x8* dst) {  // A operand: key row j (lane row l32), clamped into the split
    const int jr = min(j0 + 32 * t + l32, j1 - 1);
#pragma unroll
    for (int st = 0; st < NKS; ++st) dst[st] = ld8(kbase + (int64_t)jr * kcs.t + 16 * st + 8 * g);
  };
  auto vstage = [&](int t, bf16* dst) {  // 32 V' rows of tile t into this wave's buffer
#pragma unroll
    for (int i = 0; i < NST; ++i) {
      const int qq = i * 64 + lane, r = qq / CPR, c = (qq % CPR) ^ (r & 7);
      const int jr = min(j0 + 32 * t + r, j1 - 1);
      __builtin_amdgcn_global_load_lds(vbase + (int64_t)jr * vcs.t + c * 8, dst + i * 512, 16, 0, 0);
    }
  };
  int it = 0;
  if (w < ntile) {
    kload(w, kcur);
    vstage(w, sm.u.v[w][0]);
  }
  for (int t = w; t < ntile; t += 4, ++it) {
    const int cur = it & 1;
    const bool more = t + 4 < ntile;
    if (more) {
      kload(t + 4, knx);
      vstage(t + 4, sm.u.v[w][cur ^ 1]);
    }
    const int jb = j0 + 32 * t;
    // scores and the squared norms of the tile's keys
    f32x16 sc = zero16();
    float nn = 0.f;
#pragma unroll
    for (int st = 0; st < NKS; ++st) {
      sc = mfma32(kcur[st], xb[st], sc);
#pragma unroll
      for (int e = 0; e < 8; ++e) nn = fmaf((float)kcur[st][e], (float)kcur[st][e], nn);
    }
    nn = wave_sum32(nn);
    if (g == 0) sm.nn[w][l32] = nn;
    float nr[16];
    lds_rows16(&sm.nn[w][0], g, nr);
    // online max of the query columns (lazy: rescale only when a row grows by 2^8)
    float mx = DEC_NEG;
#pragma unroll
    for (int e = 0; e < 16; ++e)
      if (jb + drow(e, g) < j1) mx = fmaxf(mx, sc[e]);
    mx = isq ? wave_max32(mx) * sl2 : DEC_NEG;
    if (__builtin_amdgcn_ballot_w64(mx > m + 8.0f)) {
      const float mnew = fmaxf(m, mx);
      const float al = __builtin_amdgcn_exp2f(m - mnew);
      m = mnew;
      l *= al;
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int e = 0; e < 16; ++e) oacc[dt][e] *= isq ? al : 1.f;
    }
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const bool ok = jb + drow(e, g) < j1 && valid;
      const float arg = isq ? fmaf(sc[e], sl2, -m) : fmaf(c1 * rsqrtf(nr[e] / dn + eps), sc[e], -c0);
      const float p = ok ? __builtin_amdgcn_exp2f(arg) : 0.f;
      if (isq) l += p;
      sc[e] = p;
    }
    const bf16x8 p0 = pack_b(sc, 0), p1 = pack_b(sc, 1);
    // this tile's V' rows have landed once at most the next tile's loads are in flight
    if (more)
      dma_wait_but<NKS + NST>();
    else
      dma_wait();
    const bf16* vt = sm.u.v[w][cur];
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
      oacc[dt] = mfma32(lds_tr_a<CPR>(vt, 0, dt * 32), p0, oacc[dt]);
      oacc[dt] = mfma32(lds_tr_a<CPR>(vt, 16, dt * 32), p1, oacc[dt]);
    }
    if (more) {
#pragma unroll
      for (int st = 0; st < NKS; ++st) kcur[st] = knx[st];
    }
  }
  l = wave_sum32(l);
  __syncthreads();  // every wave is done with its staging buffers (aliased below)
  if (valid) {
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int e = 0; e < 16; ++e) sm.u.fin.so[w][col][dt * 32 + drow(e, g)] = oacc[dt][e];
    if (isq && g == 0) {
      sm.u.fin.m[w][col] = m;
      sm.u.fin.l[w][col] = l;
    }
  }
  __syncthreads();
  // combine the 4 waves: thread d of the first D threads owns column d of every token
  if (tid < D) {
    const int d = tid;
    for (int t = 0; t < L; ++t) {
      const int ck = t * (GG + 1) + GG;
      part.a[(((int64_t)s * BH + bh) * L + t) * D + d] =
          sm.u.fin.so[0][ck][d] + sm.u.fin.so[1][ck][d] + sm.u.fin.so[2][ck][d] + sm.u.fin.so[3][ck][d];
      for (int gg = 0; gg < GG; ++gg) {
        const int cq = t * (GG + 1) + gg;
        const float mn =
            fmaxf(fmaxf(sm.u.fin.m[0][cq], sm.u.fin.m[1][cq]), fmaxf(sm.u.fin.m[2][cq], sm.u.fin.m[3][cq]));
        float lt = 0.f, ot = 0.f;
#pragma unroll
        for (int ww = 0; ww < 4; ++ww) {
          const float al = __builtin_amdgcn_exp2f(sm.u.fin.m[ww][cq] - mn);
          lt = fmaf(sm.u.fin.l[ww][cq], al, lt);
          ot = fmaf(sm.u.fin.so[ww][cq][d], al, ot);
        }
        const int64_t pi = ((int64_t)s * BH + bh) * (L * GG) + t * GG + gg;
        part.o[pi * D + d] = ot;
        if (d == 0) {
          part.m[pi] = mn;
          part.l[pi] = lt;
        }
      }
    }
  }
}

// grid (B*Hkv, Gs): workgroup (kv head, query head g0 + g of the kv head's Gt), for the L
// tokens of the pass (G and Gs as in the split kernel; L <= its token capacity).  The
// 256 threads are D/4 column groups (4 columns each, 16-byte loads) x NSL = 1024/D split
// lanes, the lanes of one group adjacent in the wave: each lane merges every NSL-th split
// of every token at once (online rescaling; the tokens' loads interleave), then the
// lanes of a group are merged by lane shuffles.  The new tokens' own rows follow in
// order: v'_t needs v'_u of the earlier new tokens (u < t), each column only its own
// column, so the first lane of each group solves its 4 columns of every token without a
// barrier.  Every workgroup of a kv head computes the v'_t; the g = 0 one writes them and
// appends (k_t, v'_t) to the caches at rows Tp + t (if write_cache: a group split into
// chunks of query heads runs this once per chunk, and only the first writes).
template <int D, int G>
__global__ __launch_bounds__(256) void lucid_decode_combine_kernel(
    int nsplit, int L, const bf16* __restrict__ q, Strides qs, const bf16* __restrict__ kn, Strides kns,
    const bf16* __restrict__ vn, Strides vns, bf16* __restrict__ kc, Strides kcs, bf16* __restrict__ vc, Strides vcs,
    bf16* __restrict__ o, Strides os, float* __restrict__ vp_new, int vp_rows, int Hkv, int Tp, float scale,
    float eps, float dn, DecodePartials part, int Gs, int Gt, int g0, int write_cache) {
  constexpr int CG = D / 4, NSL = 256 / CG;
  static_assert(NSL * CG == 256 && NSL <= 64 && (NSL & (NSL - 1)) == 0, "split lanes of a group within a wave");
  constexpr int LM = decode_tokens_per_pass<G>();
  __shared__ float kk[LM][LM], qk[LM][LM];  // k_t . k_u (u <= t) and q_tg . k_u (u <= t)
  // merged O, sum_j P_tj v'_j and the new v' rows of every token
  __shared__ __attribute__((aligned(16))) float ovs[LM][D];
  __shared__ __attribute__((aligned(16))) float avs[LM][D];
  __shared__ __attribute__((aligned(16))) float vps[LM][D];
  __shared__ float ms_[LM], ls_[LM];                                              // merged max and sum
  const int bh = blockIdx.x, BH = gridDim.x, g = blockIdx.y;
  const int b = bh / Hkv, h = bh - b * Hkv;
  const int tid = threadIdx.x, cg = tid / NSL, sl = tid - cg * NSL, d0 = 4 * cg;
  const int GG = G > 0 ? G : Gs;
  const int hq = h * Gt + g0 + g;
  // dot products among the new tokens: k_t . k_u and q_tg . k_u for u <= t
  for (int idx = tid; idx < L * L; idx += 256) {
    const int t = idx / L, u = idx - t * L;
    if (u > t) continue;
    const bf16* kt = kn + b * kns.b + h * kns.h + (int64_t)t * kns.t;
    const bf16* ku = kn + b * kns.b + h * kns.h + (int64_t)u * kns.t;
    const bf16* qt = q + b * qs.b + hq * qs.h + (int64_t)t * qs.t;
    float dkk = 0.f, dqk = 0.f;
#pragma unroll
    for (int i = 0; i < D; i += 8) {
      const bf16x8 a8 = ld8(kt + i), b8 = ld8(ku + i), q8 = ld8(qt + i);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        dkk = fmaf((float)a8[e], (float)b8[e], dkk);
        dqk = fmaf((float)q8[e], (float)b8[e], dqk);
      }
    }
    kk[t][u] = dkk;
    qk[t][u] = dqk;
  }
  // the splits' partials of every token: its key column (sum P_tj v'_j) and its query
  // column (t, g), merged with a running max per token
  float M[LM], lv[LM];
  f32x4 ov[LM], av[LM];
#pragma unroll
  for (int t = 0; t < LM; ++t) {
    M[t] = DEC_NEG;
    lv[t] = 0.f;
    ov[t] = av[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  for (int s = sl; s < nsplit; s += NSL) {
    const int64_t base = ((int64_t)s * BH + bh) * (L * GG) + g;
#pragma unroll
    for (int t = 0; t < LM; ++t) {
      if (t < L) {
        const int64_t i = base + t * GG;
        const float mi = part.m[i], li = part.l[i];
        const f32x4 oi = *reinterpret_cast<const f32x4*>(part.o + i * D + d0);
        const f32x4 ai = *reinterpret_cast<const f32x4*>(part.a + (((int64_t)s * BH + bh) * L + t) * D + d0);
        const float mn = fmaxf(M[t], mi);
        const float c = __builtin_amdgcn_exp2f(M[t] - mn), e = __builtin_amdgcn_exp2f(mi - mn);
        lv[t] = fmaf(lv[t], c, li * e);
#pragma unroll
        for (int x = 0; x < 4; ++x) {
          ov[t][x] = fmaf(ov[t][x], c, oi[x] * e);
          av[t][x] += ai[x];
        }
        M[t] = mn;
      }
    }
  }
  // merge the NSL adjacent split lanes of each column group
#pragma unroll
  for (int off = 1; off < NSL; off <<= 1) {
#pragma unroll
    for (int t = 0; t < LM; ++t) {
      if (t < L) {
        const float mo = __shfl_xor(M[t], off, 64), lo = __shfl_xor(lv[t], off, 64);
        const float mn = fmaxf(M[t], mo);
        const float c = __builtin_amdgcn_exp2f(M[t] - mn), co = __builtin_amdgcn_exp2f(mo - mn);
        lv[t] = fmaf(lv[t], c, lo * co);
#pragma unroll
        for (int x = 0; x < 4; ++x) {
          ov[t][x] = fmaf(ov[t][x], c, __shfl_xor(ov[t][x], off, 64) * co);
          av[t][x] += __shfl_xor(av[t][x], off, 64);
        }
        M[t] = mn;
      }
    }
  }
  // the merged state of every token into LDS (the first lane of each column group)
  if (sl == 0) {
#pragma unroll
    for (int t = 0; t < LM; ++t) {
      if (t < L) {
        *reinterpret_cast<f32x4*>(&ovs[t][d0]) = ov[t];
        *reinterpret_cast<f32x4*>(&avs[t][d0]) = av[t];
        if (cg == 0) {
          ms_[t] = M[t];
          ls_[t] = lv[t];
        }
      }
    }
  }
  __syncthreads();  // kk, qk and the merged states
  if (sl != 0) return;
  // the new rows in order: v'_t = (v_t - a_t - sum_{u<t} P_tu v'_u) / P_tt (columns d0 .. d0+3)
  const float sl2 = scale * LOG2E_F, c0 = LOG2E_F / scale;
  for (int t = 0; t < L; ++t) {
    const float rt = rsqrtf(kk[t][t] / dn + eps);
    const bf16x4 v4 = *reinterpret_cast<const bf16x4*>(vn + b * vns.b + h * vns.h + (int64_t)t * vns.t + d0);
    const f32x4 a4 = *reinterpret_cast<const f32x4*>(&avs[t][d0]);
    f32x4 x;
#pragma unroll
    for (int j = 0; j < 4; ++j) x[j] = (float)v4[j] - a4[j];
    for (int u = 0; u < t; ++u) {
      const float ru = rsqrtf(kk[u][u] / dn + eps);
      const float p = __builtin_amdgcn_exp2f(fmaf(sl2 * rt * ru, kk[t][u], -c0));
      const f32x4 vu = *reinterpret_cast<const f32x4*>(&vps[u][d0]);
#pragma unroll
      for (int j = 0; j < 4; ++j) x[j] = fmaf(-p, vu[j], x[j]);
    }
    // P_tt = exp(s |K^_t|^2 - 1/s), |K^_t|^2 = dn ms / (ms + eps)
    const float ms = kk[t][t] / dn;
    const float inv = 1.f / __builtin_amdgcn_exp2f(LOG2E_F * (scale * dn * ms / (ms + eps) - 1.f / scale));
#pragma unroll
    for (int j = 0; j < 4; ++j) x[j] *= inv;
    *reinterpret_cast<f32x4*>(&vps[t][d0]) = x;  // read back only by this thread
  }
  // outputs: the cached part merged with the new keys u <= t (values bf16(v'_u), as cached)
  for (int t = 0; t < L; ++t) {
    float M2 = ms_[t];
    for (int u = 0; u <= t; ++u) M2 = fmaxf(M2, qk[t][u] * sl2);
    const float c = __builtin_amdgcn_exp2f(ms_[t] - M2);
    const f32x4 o4 = *reinterpret_cast<const f32x4*>(&ovs[t][d0]);
    f32x4 num;
#pragma unroll
    for (int j = 0; j < 4; ++j) num[j] = o4[j] * c;
    float den = ls_[t] * c;
    for (int u = 0; u <= t; ++u) {
      const float es = __builtin_amdgcn_exp2f(fmaf(qk[t][u], sl2, -M2));
      const f32x4 vu = *reinterpret_cast<const f32x4*>(&vps[u][d0]);
#pragma unroll
      for (int j = 0; j < 4; ++j) num[j] = fmaf(es, (float)(bf16)vu[j], num[j]);
      den += es;
    }
    const float rden = 1.f / den;
    const f32x4 vt = *reinterpret_cast<const f32x4*>(&vps[t][d0]);
    bf16x4 ob, vb;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      ob[j] = (bf16)(num[j] * rden);
      vb[j] = (bf16)vt[j];
    }
    *reinterpret_cast<bf16x4*>(o + b * os.b + hq * os.h + (int64_t)t * os.t + d0) = ob;
    if (g == 0 && write_cache) {
      *reinterpret_cast<f32x4*>(vp_new + ((int64_t)bh * vp_rows + t) * D + d0) = vt;
      *reinterpret_cast<bf16x4*>(kc + b * kcs.b + h * kcs.h + (int64_t)(Tp + t) * kcs.t + d0) =
          *reinterpret_cast<const bf16x4*>(kn + b * kns.b + h * kns.h + (int64_t)t * kns.t + d0);
      *reinterpret_cast<bf16x4*>(vc + b * vcs.b + h * vcs.h + (int64_t)(Tp + t) * vcs.t + d0) = vb;
    }
  }
}

}  // namespace lucid
