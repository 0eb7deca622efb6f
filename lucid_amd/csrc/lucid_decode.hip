// LUCID decoding step on CDNA4 (gfx950): one new token per sequence against a
// (K, V') cache, with the exact preconditioner row (modeling_lucid.py:576-598 is
// the reference seam; its V' update drops the division by the diagonal P_tt, kept
// here so that a decoded row equals the same row of a prefill):
//   P_tj = exp(s r_t r_j (k_t . k_j) - 1/s),  r = 1 / rms(k)  (j < t)
//   v'_t = (v_t - sum_{j<t} P_tj v'_j) / P_tt,  P_tt = exp(s dn ms_t / (ms_t + eps) - 1/s)
// (dn: the head dim; rows may be zero-padded beyond it, ms = sum k^2 / dn)
//   o_g  = softmax_j(s q_g . k_j) v'_j over j <= t, for the G query heads of the kv head
// Both sums read every cached row once (memory bound), so one pass over the cache
// computes them together, split over the sequence (flash-decoding):
//   lucid_decode_split_kernel    per (split, kv head): partial sum_j P_tj v'_j and the
//                                online-softmax state (m, l, O) of every query head, as
//                                MFMA tiles (the G query heads and the token's key are
//                                the columns of one score tile)
//   lucid_decode_combine_kernel  per (kv head, query head): v'_t, the token's own
//                                softmax term, the output, and the append of (k_t, v'_t)
//                                to the cache
#include "lucid_common.h"

namespace lucid {

constexpr float DEC_NEG = -1e30f;  // finite "minus infinity" for empty softmax states

struct DecodePartials {
  float* a;  // [nsplit][BH][D]     sum_j P_tj v'_j
  float* m;  // [nsplit][BH][G]     running max (log2 domain)
  float* l;  // [nsplit][BH][G]     running sum
  float* o;  // [nsplit][BH][G][D]  unnormalised output
};

// Split pass on the matrix cores.  Each wave sweeps its own 32-key tiles of the split
// (tiles w, w+4, ...) and computes, per tile, one MFMA score tile
//   S^T[j][c] = K_j . X_c,  X_c = q_{hG+c} (c < G),  X_G = k_t,  other columns zero,
// so the G query heads and the preconditioner row of the new token share one product.
// Column c < G takes the online softmax p = exp2(s' S - m_c); column G takes
// p = exp2(s' r_t r_j S - 1/s log2 e), with 1/rms r_j of the cached key from the key
// registers.  O^T[d][c] += V'^T[d][j] p^T[j][c] (V' rows staged per wave into LDS by
// direct loads and read transposed) accumulates the G outputs and, in column G, the
// sum_j P_tj v'_j.  Keys reach registers one tile ahead; no barrier in the sweep.
template <int D, int G>
struct DecodeMfmaSmem {
  union {
    bf16 v[4][2][32 * D];  // per wave, double buffered, swizzled (chunk c of row r at c ^ (r & 7))
    struct {
      float so[4][G + 1][D];  // per wave: columns 0..G of O^T
      float m[4][G], l[4][G];
    } fin;
  } u;
  float nn[4][32];  // per wave: squared norms of the tile's keys
};

template <int D, int G>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void lucid_decode_split_kernel(
    const bf16* __restrict__ q, Strides qs, const bf16* __restrict__ kn, Strides kns,
    const bf16* __restrict__ kc, Strides kcs, const bf16* __restrict__ vc, Strides vcs, int Hkv, int Tp, int KS,
    float scale, float eps, float dn, DecodePartials part) {
  constexpr int NKS = D / 16, NDT = D / 32, CPR = D / 8, NST = 32 * CPR / 64;  // NST: staging loads per tile
  static_assert(G + 1 <= 32, "query heads + the preconditioner row must fit one 32-column tile");
  __shared__ __attribute__((aligned(16))) DecodeMfmaSmem<D, G> sm;
  const int s = blockIdx.x, bh = blockIdx.y, BH = gridDim.y;
  const int b = bh / Hkv, h = bh - b * Hkv;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 5, l32 = lane & 31;
  const int col = l32;  // score / output column of this lane
  const int j0 = s * KS, j1 = min(Tp, j0 + KS);

  // B operand: column col of X^T (k = d), zero for the padding columns
  bf16x8 xb[NKS];
  float nt = 0.f;
#pragma unroll
  for (int st = 0; st < NKS; ++st) {
    bf16x8 x;
    if (col < G) {
      x = ld8(q + b * qs.b + (h * G + col) * qs.h + 16 * st + 8 * g);
    } else if (col == G) {
      x = ld8(kn + b * kns.b + h * kns.h + 16 * st + 8 * g);
#pragma unroll
      for (int e = 0; e < 8; ++e) nt = fmaf((float)x[e], (float)x[e], nt);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = (bf16)0.f;
    }
    xb[st] = x;
  }
  nt = wave_sum32(nt);
  const float rt = rsqrtf(__builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, nt), G)) / dn + eps);
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
    mx = (col < G) ? wave_max32(mx) * sl2 : DEC_NEG;
    if (__builtin_amdgcn_ballot_w64(mx > m + 8.0f)) {
      const float mnew = fmaxf(m, mx);
      const float al = __builtin_amdgcn_exp2f(m - mnew);
      m = mnew;
      l *= al;
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int e = 0; e < 16; ++e) oacc[dt][e] *= (col < G) ? al : 1.f;
    }
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const bool ok = jb + drow(e, g) < j1 && col <= G;
      const float arg = (col < G) ? fmaf(sc[e], sl2, -m) : fmaf(c1 * rsqrtf(nr[e] / dn + eps), sc[e], -c0);
      const float p = ok ? __builtin_amdgcn_exp2f(arg) : 0.f;
      if (col < G) l += p;
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
  if (col <= G) {
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int e = 0; e < 16; ++e) sm.u.fin.so[w][col][dt * 32 + drow(e, g)] = oacc[dt][e];
    if (col < G && g == 0) {
      sm.u.fin.m[w][col] = m;
      sm.u.fin.l[w][col] = l;
    }
  }
  __syncthreads();
  // combine the 4 waves: thread d of the first D threads owns column d
  if (tid < D) {
    const int d = tid;
    part.a[((int64_t)s * BH + bh) * D + d] =
        sm.u.fin.so[0][G][d] + sm.u.fin.so[1][G][d] + sm.u.fin.so[2][G][d] + sm.u.fin.so[3][G][d];
#pragma unroll
    for (int gg = 0; gg < G; ++gg) {
      const float mn = fmaxf(fmaxf(sm.u.fin.m[0][gg], sm.u.fin.m[1][gg]), fmaxf(sm.u.fin.m[2][gg], sm.u.fin.m[3][gg]));
      float lt = 0.f, ot = 0.f;
#pragma unroll
      for (int ww = 0; ww < 4; ++ww) {
        const float al = __builtin_amdgcn_exp2f(sm.u.fin.m[ww][gg] - mn);
        lt = fmaf(sm.u.fin.l[ww][gg], al, lt);
        ot = fmaf(sm.u.fin.so[ww][gg][d], al, ot);
      }
      part.o[(((int64_t)s * BH + bh) * G + gg) * D + d] = ot;
      if (d == 0) {
        part.m[((int64_t)s * BH + bh) * G + gg] = mn;
        part.l[((int64_t)s * BH + bh) * G + gg] = lt;
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
    bf16* __restrict__ o, Strides os, float* __restrict__ vp_new, int Hkv, int Tp, float scale, float eps, float dn,
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
  const float ms = nk / dn;
  // P_tt = exp(s |K^_t|^2 - 1/s), |K^_t|^2 = dn ms / (ms + eps)
  const float ptt = __builtin_amdgcn_exp2f(LOG2E_F * (scale * dn * ms / (ms + eps) - 1.f / scale));
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
