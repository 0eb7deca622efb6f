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
//   lucid_bwd_prep_kernel          ndelta = -rowsum(dO * O), zero the chain counters
//   lucid_attn_bwd_dkdv_kernel     column sweep: dV' (summed over the GQA group), dK_attn
//   lucid_attn_bwd_dq_kernel       row sweep: dQ
//   lucid_precond_bwd_col_kernel   chained transposed solve -> dV, and the M^T K^ column sums
//   lucid_precond_bwd_row_kernel   M K^ row sums, RMSNorm backward, dK
#include <type_traits>

#include "lucid_common.h"

namespace lucid {

// delta[bhq][t] = -(dO_t . O_t) (stored negated); zero the chain counters.  Heads of the
// exact chains (row mass above kExactMass) take O as its bf16 pair O + olo (written by the
// attention forward).  seeds[bhq][t]: the two MFMA A-operand rows (8 bf16 each) that seed
// the column sweep's accumulators with the row terms, -lse2_t / c (c = s log2(e)) and
// -delta_t, each split into three bf16 terms (seed_a).  grid (T/64, B*Hq)
template <int D, bool F32 = false>
__global__ __launch_bounds__(256) void lucid_bwd_prep_kernel(const bf16* __restrict__ dout, Strides dos,
                                                             const bf16* __restrict__ o, Strides os,
                                                             const bf16* __restrict__ olo,
                                                             const float* __restrict__ mass, int Hq, int Hkv, int T,
                                                             float* __restrict__ delta, int* __restrict__ counters,
                                                             int BH, Lo lo, const float* __restrict__ lse,
                                                             float cinv, bf16* __restrict__ seeds) {
  constexpr int SEG = D / 4;
  const int blk = blockIdx.x, bhq = blockIdx.y;
  const int b = bhq / Hq, hq = bhq - b * Hq;
  const bool exact = mass[b * Hkv + hq / (Hq / Hkv)] > kExactMass;
  const int tid = threadIdx.x;
  const int row = tid >> 2, seg = tid & 3;
  const int t = blk * 64 + row;
  const bf16* dop = dout + b * dos.b + hq * dos.h + (int64_t)t * dos.t;
  const bf16* opp = o + b * os.b + hq * os.h + (int64_t)t * os.t;
  const bf16* olp = olo + ((int64_t)bhq * T + t) * D;
  float acc = 0.f;
  if constexpr (F32) {  // fp32 dO and O themselves
    const float* df = lo.dof + b * dos.b + hq * dos.h + (int64_t)t * dos.t + seg * SEG;
    const float* of = lo.o + b * os.b + hq * os.h + (int64_t)t * os.t + seg * SEG;
#pragma unroll
    for (int c = 0; c < SEG; c += 4) {
      const f32x4 a = *reinterpret_cast<const f32x4*>(df + c);
      const f32x4 x = *reinterpret_cast<const f32x4*>(of + c);
#pragma unroll
      for (int e = 0; e < 4; ++e) acc = fmaf(a[e], x[e], acc);
    }
  } else {
#pragma unroll
    for (int c = 0; c < SEG; c += 8) {
      const bf16x8 a = ld8(dop + seg * SEG + c);
      const bf16x8 bo = ld8(opp + seg * SEG + c);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc += (float)a[e] * (float)bo[e];
      if (exact) {
        const bf16x8 bl = ld8(olp + seg * SEG + c);
#pragma unroll
        for (int e = 0; e < 8; ++e) acc += (float)a[e] * (float)bl[e];
      }
    }
  }
  acc += __shfl_xor(acc, 1, 64);
  acc += __shfl_xor(acc, 2, 64);
  if (seg == 0) {
    const int64_t r = (int64_t)bhq * T + t;
    delta[r] = -acc;
    *reinterpret_cast<bf16x8*>(seeds + r * 16) = seed_a(-lse[r] * cinv, 0);
    *reinterpret_cast<bf16x8*>(seeds + r * 16 + 8) = seed_a(-acc, 0);
  }
  if (blk == 0 && tid == 0 && bhq < BH) counters[bhq] = 0;
}

// ---------------------------------------------------------------------------
// Column sweep for the attention part.  Workgroup = 128 keys of one kv head,
// wave w owns keys 32w..32w+31 (one n-tile, lane <-> key j); sweeps the G query
// heads of the group and every 64-row query tile at or below the diagonal.
// Each query tile (Q and dO rows, lse2, delta) is staged once per workgroup in
// LDS by direct global->LDS loads (three buffers, two tiles ahead, swizzled);
// Q^T and dO^T operands come from the same tiles through transposing LDS loads.
//   S[i][j] = Q_i . K_j, P = exp2(c S - lse2_i)
//   dV'^T[d][j] += dO^T[d][i] P[i][j];  dP[i][j] = dO_i . V'_j
//   dS = P (dP - delta_i);  dK^T[d][j] += Q^T[d][i] dS[i][j]
// At d = 64 two workgroups share a CU (<= 256 registers per lane).
// ---------------------------------------------------------------------------
template <int D, bool F32 = false>
struct DkdvSmem {
  static constexpr int NB = stage_bufs(D, F32);
  bf16 q[NB][64 * D];   // swizzled tiles (chunk c of row r at c ^ (r & 7))
  bf16 dO[NB][64 * D];
  bf16 ql[F32 ? NB : 1][F32 ? 64 * D : 8];   // lo tiles (fp32 inputs)
  bf16 dOl[F32 ? NB : 1][F32 ? 64 * D : 8];
  bf16 seed[NB][64][16];  // per row: the seed operands of -lse2 / c and -delta (seeds)
};

// F32 (fp32 inputs, head dim 64): the lo tiles of Q and dO are staged beside the hi tiles,
// K and V' carry their lo parts in registers, and every product (dV', dP, dK) takes
// three MFMAs (S = Q.K four, lo*lo included); P and dS are split into hi and lo.
// DA: the head-dim columns that can be nonzero (zero-padded rows of a smaller head dim; the
// products skip the k-steps and tiles that would only meet zero columns, whose outputs stay 0)
template <int D, bool F32 = false, int DA = D>
__global__ __launch_bounds__(256) LUCID_TWO_WAVES_IF(D == 64 && !F32) void lucid_attn_bwd_dkdv_kernel(
    const bf16* __restrict__ q, Strides qs, const bf16* __restrict__ k, Strides ks, const bf16* __restrict__ vpb,
    const bf16* __restrict__ dout, Strides dos, const bf16* __restrict__ seeds, float* __restrict__ dvp, float* __restrict__ dka, int Hq, int Hkv, int T, int BH, float scale, Lo lo,
    const bf16* __restrict__ vpbl) {
  static_assert(!F32 || D == 64 || D == 128, "fp32 inputs: head dim 64 or 128");
  constexpr int NDT = D / 32;
  constexpr int NKS = D / 16;
  constexpr int NDT_A = (DA + 31) / 32, NKS_A = DA / 16;
  static_assert(DA % 16 == 0 && DA <= D, "active head dim");
  // newest vector-memory ops of a step, per wave
  constexpr int STAGE_OPS = (F32 ? 4 : 2) * (64 * (D / 8) / 256);
  __shared__ __attribute__((aligned(16))) DkdvSmem<D, F32> sm;
  constexpr int NB = stage_bufs(D, F32);
  const int id = blockIdx.x;
  const int jb = id / BH, bh = id - (id / BH) * BH;
  const int b = bh / Hkv, h = bh - b * Hkv;
  const int G = Hq / Hkv;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int g = lane >> 5, l32 = lane & 31;
  const int jw = jb * 128 + w * 32;  // first key of this wave
  const int jrow = jw + l32;
  const bf16* kh = k + b * ks.b + h * ks.h;
  const float c = scale * LOG2E_F;

  bf16x8 kb[NKS], vb[NKS], kbl[NKS], vbl[NKS];
#pragma unroll
  for (int st = 0; st < NKS_A; ++st) {
    kb[st] = ld8(kh + (int64_t)jrow * ks.t + 16 * st + 8 * g);
    vb[st] = ld8(vpb + ((int64_t)bh * T + jrow) * D + 16 * st + 8 * g);
    if constexpr (F32) {
      kbl[st] = ld8(lo.k + b * ks.b + h * ks.h + (int64_t)jrow * ks.t + 16 * st + 8 * g);
      vbl[st] = ld8(vpbl + ((int64_t)bh * T + jrow) * D + 16 * st + 8 * g);
    }
  }
  f32x16 adv[NDT], adk[NDT];
#pragma unroll
  for (int t = 0; t < NDT; ++t) {
    adv[t] = zero16();
    adk[t] = zero16();
  }
  const int nt64 = T / 64;
  const int it_first = jb * 2;            // first query tile any wave needs
  const int ntile = nt64 - it_first;      // query tiles per query head
  const int nsteps = G * ntile;           // step s: query head s / ntile, tile it_first + s % ntile
  const int it_w = jw / 64;               // this wave's diagonal tile
  const int kloc = jw - it_w * 64 + l32;  // this lane's key inside its diagonal tile
  int plan_q[64 * (D / 8) / 256], plan_o[64 * (D / 8) / 256];
  // head dim 64: the conflict-free swizzle (every staged tile is read twice per wave, in rows
  // and transposed, so the LDS bandwidth matters here)
  constexpr int SW = D == 64 ? 1 : 0;
  dma_plan<64, D / 8, 256, SW>(qs.t, plan_q);
  dma_plan<64, D / 8, 256, SW>(dos.t, plan_o);
  auto stage = [&](int s) {
    const int gi = s / ntile, it = it_first + s - gi * ntile, buf = s % NB;
    const int hq = h * G + gi, bhq = b * Hq + hq, i0 = it * 64;
    if (w < 2) dma_1k(seeds + ((int64_t)bhq * T + i0 + 32 * w) * 16, &sm.seed[buf][32 * w][0]);  // 2 KB of seed rows
    dma_stage<64, D / 8>(plan_q, q + b * qs.b + hq * qs.h + (int64_t)i0 * qs.t, sm.q[buf]);
    dma_stage<64, D / 8>(plan_o, dout + b * dos.b + hq * dos.h + (int64_t)i0 * dos.t, sm.dO[buf]);
    if constexpr (F32) {
      dma_stage<64, D / 8>(plan_q, lo.q + b * qs.b + hq * qs.h + (int64_t)i0 * qs.t, sm.ql[buf]);
      dma_stage<64, D / 8>(plan_o, lo.dout + b * dos.b + hq * dos.h + (int64_t)i0 * dos.t, sm.dOl[buf]);
    }
  };
  stage(0);
  if (NB == 3 && nsteps > 1) {
    stage(1);
    dma_wait_but<STAGE_OPS>();
  } else {
    dma_wait();
  }
  __syncthreads();
  int tro[NDT], tro2[NDT], rdo[NKS];  // lane offsets of the transposing (two loads) and the row reads
#pragma unroll
  for (int t = 0; t < NDT; ++t) lds_tr_lane_offs<D / 8, SW>(t * 32, tro[t], tro2[t]);
#pragma unroll
  for (int st = 0; st < NKS; ++st) rdo[st] = swz_off<D / 8, SW>(l32, 2 * st + g);
  const bf16x8 ones = seed_ones(g);
  // one 64-row query tile in buffer buf (a compile-time index, so that every LDS operand
  // address is a lane offset plus an immediate); DIAG: the tile holding this wave's keys
  // (causal mask)
  auto tile = [&](auto bufc, const bool DIAG) __attribute__((always_inline)) {
    const int buf = bufc;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      if (DIAG && mt * 32 + 31 < kloc - l32) continue;  // rows all above this wave's keys
      // the per-row terms enter through the matrix cores: a rank-3 product with `ones`
      // seeds the score accumulator with -lse_i / c and the dP accumulator with -delta_i
      // (the three-term splits come staged from lucid_bwd_prep_kernel; no per-element row
      // reads and no VALU work here)
      f32x16 pv;
      bf16x8 pb0, pb1;
      {
        bf16x8 qa[NKS];
#pragma unroll
        for (int st = 0; st < NKS_A; ++st) qa[st] = ld8(sm.q[buf] + rdo[st] + mt * 32 * D);
        // (lanes 32..63 read the same row: they meet the zero rows of `ones`)
        f32x16 sc = mfma32(ld8(&sm.seed[buf][mt * 32 + l32][0]), ones, zero16());
#pragma unroll
        for (int st = 0; st < NKS_A; ++st) sc = mfma32(qa[st], kb[st], sc);
        if constexpr (F32) {
#pragma unroll
          for (int st = 0; st < NKS_A; ++st) {
            const bf16x8 qal = ld8(sm.ql[buf] + rdo[st] + mt * 32 * D);
            sc = mfma32(qa[st], kbl[st], sc);
            sc = mfma32(qal, kb[st], sc);
            sc = mfma32(qal, kbl[st], sc);
          }
        }
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          float p = __builtin_amdgcn_exp2f(sc[e] * c);
          if (DIAG && (mt * 32 + drow(e, g) < kloc)) p = 0.f;
          pv[e] = p;
        }
        pb0 = pack_b(pv, 0);
        pb1 = pack_b(pv, 1);
      }
#pragma unroll
      for (int t = 0; t < NDT_A; ++t) {
        const bf16x8 o0 = lds_tr_a_at2<D / 8>(sm.dO[buf], tro[t], tro2[t], mt * 32);
        const bf16x8 o1 = lds_tr_a_at2<D / 8>(sm.dO[buf], tro[t], tro2[t], mt * 32 + 16);
        adv[t] = mfma32(o0, pb0, adv[t]);
        adv[t] = mfma32(o1, pb1, adv[t]);
        if constexpr (F32) {
          adv[t] = mfma32(o0, pack_lo(pv, 0, pb0), adv[t]);
          adv[t] = mfma32(o1, pack_lo(pv, 1, pb1), adv[t]);
          adv[t] = mfma32(lds_tr_a_at2<D / 8>(sm.dOl[buf], tro[t], tro2[t], mt * 32), pb0, adv[t]);
          adv[t] = mfma32(lds_tr_a_at2<D / 8>(sm.dOl[buf], tro[t], tro2[t], mt * 32 + 16), pb1, adv[t]);
        }
      }
      f32x16 ds;
      {
        bf16x8 da[NKS];
#pragma unroll
        for (int st = 0; st < NKS_A; ++st) da[st] = ld8(sm.dO[buf] + rdo[st] + mt * 32 * D);
        // dP - delta: the accumulator starts at -delta (stored negated)
        f32x16 dp = mfma32(ld8(&sm.seed[buf][mt * 32 + l32][8]), ones, zero16());
#pragma unroll
        for (int st = 0; st < NKS_A; ++st) dp = mfma32(da[st], vb[st], dp);
        if constexpr (F32) {
#pragma unroll
          for (int st = 0; st < NKS_A; ++st) {
            dp = mfma32(da[st], vbl[st], dp);
            dp = mfma32(ld8(sm.dOl[buf] + rdo[st] + mt * 32 * D), vb[st], dp);
          }
        }
#pragma unroll
        for (int e = 0; e < 16; ++e) ds[e] = pv[e] * dp[e];
        pb0 = pack_b(ds, 0);
        pb1 = pack_b(ds, 1);
      }
#pragma unroll
      for (int t = 0; t < NDT_A; ++t) {
        const bf16x8 q0 = lds_tr_a_at2<D / 8>(sm.q[buf], tro[t], tro2[t], mt * 32);
        const bf16x8 q1 = lds_tr_a_at2<D / 8>(sm.q[buf], tro[t], tro2[t], mt * 32 + 16);
        adk[t] = mfma32(q0, pb0, adk[t]);
        adk[t] = mfma32(q1, pb1, adk[t]);
        if constexpr (F32) {
          adk[t] = mfma32(q0, pack_lo(ds, 0, pb0), adk[t]);
          adk[t] = mfma32(q1, pack_lo(ds, 1, pb1), adk[t]);
          adk[t] = mfma32(lds_tr_a_at2<D / 8>(sm.ql[buf], tro[t], tro2[t], mt * 32), pb0, adk[t]);
          adk[t] = mfma32(lds_tr_a_at2<D / 8>(sm.ql[buf], tro[t], tro2[t], mt * 32 + 16), pb1, adk[t]);
        }
      }
    }
  };
  // step s works on buffer s % NB: the loop is unrolled by NB so that it is a constant
  auto step = [&](auto bufc, const int s) __attribute__((always_inline)) {
    if (s + NB - 1 < nsteps) stage(s + NB - 1);
    const int it = it_first + s % ntile;
    if (it > it_w) tile(bufc, false);
    else if (it == it_w) tile(bufc, true);
    if (NB == 3 && s + 2 < nsteps) dma_wait_but<STAGE_OPS>();  // the step after next may stay in flight
    else dma_wait();
    __syncthreads();
  };
  for (int s = 0; s < nsteps; s += NB) {
    step(std::integral_constant<int, 0>{}, s);
    if (s + 1 < nsteps) step(std::integral_constant<int, 1>{}, s + 1);
    if constexpr (NB == 3) {
      if (s + 2 < nsteps) step(std::integral_constant<int, 2>{}, s + 2);
    }
  }
  float* ov = dvp + ((int64_t)bh * T + jrow) * D;
  float* ok = dka + ((int64_t)bh * T + jrow) * D;
#pragma unroll
  for (int t = 0; t < NDT; ++t)
#pragma unroll
    for (int qq = 0; qq < 4; ++qq) {
      f32x4 a, bq;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        a[u] = adv[t][4 * qq + u];
        bq[u] = adk[t][4 * qq + u] * scale;
      }
      *reinterpret_cast<f32x4*>(ov + t * 32 + 8 * qq + 4 * g) = a;
      *reinterpret_cast<f32x4*>(ok + t * 32 + 8 * qq + 4 * g) = bq;
    }
}

// ---------------------------------------------------------------------------
// Row sweep for dQ.  Workgroup = 256 query rows (heavy blocks first), wave w
// owns rows RW w .. RW w + RW - 1 (lane <-> row i): four waves of 64 rows, or at head
// dim 128 eight waves of 32 rows (two per SIMD; with 64 rows per wave the Q and dO
// operands and accumulators of a wave exceed the registers and spill).  Every key tile (K rows, V' rows) is
// staged once per workgroup in LDS by direct global->LDS loads (three buffers,
// two tiles ahead); K^T operands come through transposing LDS loads.
//   S^T[j][i] = K_j . Q_i, dP^T[j][i] = V'_j . dO_i, dS^T = P^T (dP^T - delta_i)
//   dQ^T[d][i] += K^T[d][j] dS^T[j][i]
// EXACT (heads whose row mass exceeds kExactMass, i.e. keys along a shared direction; each
// instance returns at once for the other heads): every row of dS sums to zero, so the
// shared key direction cancels out of dQ_i = s sum_j dS_ij K_j and the bf16 rounding of
// dS would leave it behind; dS enters as a hi/lo pair (K is exact in bf16).  dP = dO V'^T
// keeps the bf16 V' of the forward: delta_i = dO_i . O_i equals sum_j P_ij dP_ij only when
// both use the same V', and that identity is what cancels the shared direction.
// ---------------------------------------------------------------------------
template <int D>
struct DqSmem {
  bf16 k[3][64 * D];  // swizzled tiles (chunk c of row r at c ^ (r & 7))
  bf16 v[3][64 * D];
};
template <int D>
struct DqSmemF32 {  // fp32 inputs: the lo tiles of K and V' beside the hi tiles
  static constexpr int NB = stage_bufs(D, true);
  bf16 k[NB][64 * D];
  bf16 v[NB][64 * D];
  bf16 kl[NB][64 * D];
  bf16 vl[NB][64 * D];
};

// WGR: rows per workgroup (256; 128 for the fp32 instance at head dim 128, whose hi/lo
// operands need one wave per SIMD to stay in registers)
// DA: the head-dim columns that can be nonzero (as in lucid_attn_bwd_dkdv_kernel)
template <int D, bool EXACT, bool F32 = false, int RW = 64, int WGR = 256, int DA = D>
__global__ __launch_bounds__(64 * (WGR / RW)) LUCID_TWO_WAVES_IF((D == 64 || RW == 32) && !EXACT) void lucid_attn_bwd_dq_kernel(
    const bf16* __restrict__ q, Strides qs, const bf16* __restrict__ k, Strides ks, const bf16* __restrict__ vpb,
    const bf16* __restrict__ dout, Strides dos, const float* __restrict__ lse,
    const float* __restrict__ delta, const float* __restrict__ mass,
    std::conditional_t<F32, float, bf16>* __restrict__ dq, Strides dqs, int Hq, int Hkv, int T, int BHq,
    float scale, Lo lo, const bf16* __restrict__ vpbl) {
  static_assert(!F32 || EXACT, "fp32 inputs: exact instance");
  static_assert(RW == 64 || RW == 32, "rows per wave");
  constexpr int NDT = D / 32;
  constexpr int NKS = D / 16;
  constexpr int NDT_A = (DA + 31) / 32, NKS_A = DA / 16;
  static_assert(DA % 16 == 0 && DA <= D && (DA == D || RW == 32), "active head dim");
  constexpr int NT = RW / 32;           // 32-row n-tiles per wave
  constexpr int NTHR = 64 * (WGR / RW);  // WGR rows per workgroup
  __shared__ __attribute__((aligned(16))) std::conditional_t<F32, DqSmemF32<D>, DqSmem<D>> sm;
  constexpr int NB = stage_bufs(D, F32);
  const int nblk = (T + WGR - 1) / WGR;
  const int id = blockIdx.x;
  const int bhq = id % BHq;
  const int ib = nblk - 1 - id / BHq;
  const int b = bhq / Hq, hq = bhq - b * Hq;
  const int h = hq / (Hq / Hkv);
  const int bh = b * Hkv + h;
  if ((mass[bh] > kExactMass) != EXACT) return;  // the other instance handles this head
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int g = lane >> 5, l32 = lane & 31;
  const int r0 = ib * WGR;
  const int row0 = r0 + w * RW;
  const bf16* kh = k + b * ks.b + h * ks.h;
  const bf16* vh = vpb + (int64_t)bh * T * D;
  const float c = scale * LOG2E_F;

  bf16x8 qb[NT][NKS], db[NT][NKS], qbl[NT][NKS], dbl[NT][NKS];
  float li[NT], di[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int ir = min(row0 + nt * 32 + l32, T - 1);
#pragma unroll
    for (int st = 0; st < NKS_A; ++st) {
      qb[nt][st] = ld8(q + b * qs.b + hq * qs.h + (int64_t)ir * qs.t + 16 * st + 8 * g);
      db[nt][st] = ld8(dout + b * dos.b + hq * dos.h + (int64_t)ir * dos.t + 16 * st + 8 * g);
      if constexpr (F32) {
        qbl[nt][st] = ld8(lo.q + b * qs.b + hq * qs.h + (int64_t)ir * qs.t + 16 * st + 8 * g);
        dbl[nt][st] = ld8(lo.dout + b * dos.b + hq * dos.h + (int64_t)ir * dos.t + 16 * st + 8 * g);
      }
    }
    li[nt] = lse[(int64_t)bhq * T + ir];
    di[nt] = delta[(int64_t)bhq * T + ir];
  }
  f32x16 acc[NDT][NT];
#pragma unroll
  for (int t = 0; t < NDT; ++t)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) acc[t][nt] = zero16();
  const int ntile = (min(r0 + WGR, T) + 63) / 64;
  const int last_w = row0 / 64;
  const int roff = row0 - last_w * 64;  // this wave's first row within its diagonal tile
  // newest vector-memory ops of a step, per wave
  constexpr int PLAN = 64 * (D / 8) / NTHR;
  constexpr int STAGE_OPS = (F32 ? 4 : 2) * PLAN;
  int plan_k[PLAN], plan_v[PLAN];
  dma_plan<64, D / 8, NTHR>(ks.t, plan_k);
  dma_plan<64, D / 8, NTHR>(D, plan_v);
  auto stage = [&](int jt) {
    const int j0 = jt * 64, buf = jt % NB;
    dma_stage<64, D / 8, NTHR>(plan_k, kh + (int64_t)j0 * ks.t, sm.k[buf]);
    dma_stage<64, D / 8, NTHR>(plan_v, vh + (int64_t)j0 * D, sm.v[buf]);
    if constexpr (F32) {
      dma_stage<64, D / 8, NTHR>(plan_k, lo.k + b * ks.b + h * ks.h + (int64_t)j0 * ks.t, sm.kl[buf]);
      dma_stage<64, D / 8, NTHR>(plan_v, vpbl + (int64_t)bh * T * D + (int64_t)j0 * D, sm.vl[buf]);
    }
  };
  stage(0);
  if (NB == 3 && ntile > 1) {
    stage(1);
    dma_wait_but<STAGE_OPS>();
  } else {
    dma_wait();
  }
  __syncthreads();
  // lane offsets of the row reads (the transposing reads keep their per-read address
  // arithmetic here: with precomputed offsets the register-bound D = 128 instance of
  // this kernel returned NaN in dQ, unlike the same helper in the dK/dV sweep)
  int rdo[NKS];
#pragma unroll
  for (int st = 0; st < NKS; ++st) rdo[st] = swz_off<D / 8>(l32, 2 * st + g);
  // one 64-key tile in buffer buf (a compile-time index: LDS operand addresses are lane
  // offsets plus immediates); DIAG: the tile holding this wave's rows (causal mask)
  auto tile = [&](auto bufc, const bool DIAG) __attribute__((always_inline)) {
    const int buf = bufc;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      // the K and V' operands of this key half: held across the n-tiles, or (one n-tile)
      // read where they are used, which keeps the head-dim-128 instance within its registers
      bf16x8 ka[NT > 1 ? NKS : 1], va[NT > 1 ? NKS : 1];
      if constexpr (NT > 1) {
#pragma unroll
        for (int st = 0; st < NKS; ++st) {
          ka[st] = ld8(sm.k[buf] + rdo[st] + mt * 32 * D);
          va[st] = ld8(sm.v[buf] + rdo[st] + mt * 32 * D);
        }
      }
      auto kop = [&](int st) { return NT > 1 ? ka[st % (NT > 1 ? NKS : 1)] : ld8(sm.k[buf] + rdo[st] + mt * 32 * D); };
      auto vop = [&](int st) { return NT > 1 ? va[st % (NT > 1 ? NKS : 1)] : ld8(sm.v[buf] + rdo[st] + mt * 32 * D); };
      bf16x8 dsb[NT][2], dsl[NT][2];
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        f32x16 sc = zero16(), dp = zero16();
#pragma unroll
        for (int st = 0; st < NKS_A; ++st) {
          sc = mfma32(kop(st), qb[nt][st], sc);
          dp = mfma32(vop(st), db[nt][st], dp);
        }
        if constexpr (F32) {
#pragma unroll
          for (int st = 0; st < NKS_A; ++st) {
            const bf16x8 kl8 = ld8(sm.kl[buf] + rdo[st] + mt * 32 * D);
            const bf16x8 vl8 = ld8(sm.vl[buf] + rdo[st] + mt * 32 * D);
            sc = mfma32(kop(st), qbl[nt][st], sc);
            sc = mfma32(kl8, qb[nt][st], sc);
            sc = mfma32(kl8, qbl[nt][st], sc);
            dp = mfma32(vop(st), dbl[nt][st], dp);
            dp = mfma32(vl8, db[nt][st], dp);
          }
        }
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          float p = __builtin_amdgcn_exp2f(fmaf(sc[e], c, -li[nt]));
          if (DIAG && (mt * 32 + drow(e, g) > roff + nt * 32 + l32)) p = 0.f;
          sc[e] = p * (dp[e] + di[nt]);  // di holds -delta
        }
        dsb[nt][0] = pack_b(sc, 0);
        dsb[nt][1] = pack_b(sc, 1);
        if constexpr (EXACT) {
          dsl[nt][0] = pack_lo(sc, 0, dsb[nt][0]);
          dsl[nt][1] = pack_lo(sc, 1, dsb[nt][1]);
        }
      }
#pragma unroll
      for (int t = 0; t < NDT_A; ++t) {
        const bf16x8 a0 = lds_tr_a<D / 8>(sm.k[buf], mt * 32, t * 32);
        const bf16x8 a1 = lds_tr_a<D / 8>(sm.k[buf], mt * 32 + 16, t * 32);
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          acc[t][nt] = mfma32(a0, dsb[nt][0], acc[t][nt]);
          acc[t][nt] = mfma32(a1, dsb[nt][1], acc[t][nt]);
          if constexpr (EXACT) {
            acc[t][nt] = mfma32(a0, dsl[nt][0], acc[t][nt]);
            acc[t][nt] = mfma32(a1, dsl[nt][1], acc[t][nt]);
          }
          if constexpr (F32) {
            acc[t][nt] = mfma32(lds_tr_a<D / 8>(sm.kl[buf], mt * 32, t * 32), dsb[nt][0], acc[t][nt]);
            acc[t][nt] = mfma32(lds_tr_a<D / 8>(sm.kl[buf], mt * 32 + 16, t * 32), dsb[nt][1], acc[t][nt]);
          }
        }
      }
    }
  };
  // step jt works on buffer jt % 3: the bf16 instances unroll the loop by three so that it
  // is a constant
  auto step = [&](auto bufc, const int jt) __attribute__((always_inline)) {
    if (jt + 2 < ntile) stage(jt + 2);
    if (row0 < T) {
      if (jt < last_w) tile(bufc, false);
      else if (jt == last_w) tile(bufc, true);
    }
    if (jt + 2 < ntile) dma_wait_but<STAGE_OPS>();  // the step after next may stay in flight
    else dma_wait();
    __syncthreads();
  };
  if constexpr (EXACT) {  // the exact instances keep the rolled loop (registers)
    for (int jt = 0; jt < ntile; ++jt) {
      const int buf = jt % NB;
      if (jt + NB - 1 < ntile) stage(jt + NB - 1);
      if (row0 < T) {
        if (jt < last_w) tile(buf, false);
        else if (jt == last_w) tile(buf, true);
      }
      if (NB == 3 && jt + 2 < ntile) dma_wait_but<STAGE_OPS>();
      else dma_wait();
      __syncthreads();
    }
  } else {
    static_assert(EXACT || NB == 3, "the bf16 instances stage three deep");
    for (int jt = 0; jt < ntile; jt += 3) {
      step(std::integral_constant<int, 0>{}, jt);
      if (jt + 1 < ntile) step(std::integral_constant<int, 1>{}, jt + 1);
      if (jt + 2 < ntile) step(std::integral_constant<int, 2>{}, jt + 2);
    }
  }
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int irow = row0 + nt * 32 + l32;
    if (irow >= T) continue;
    auto* op = dq + b * dqs.b + hq * dqs.h + (int64_t)irow * dqs.t;
#pragma unroll
    for (int t = 0; t < NDT; ++t)
#pragma unroll
      for (int qq = 0; qq < 4; ++qq) {
        bf16x4 bb;
#pragma unroll
        for (int u = 0; u < 4; ++u) bb[u] = (bf16)(acc[t][nt][4 * qq + u] * scale);
        if constexpr (F32) {
          f32x4 x;
#pragma unroll
          for (int u = 0; u < 4; ++u) x[u] = acc[t][nt][4 * qq + u] * scale;
          *reinterpret_cast<f32x4*>(op + t * 32 + 8 * qq + 4 * g) = x;
        } else {
          *reinterpret_cast<bf16x4*>(op + t * 32 + 8 * qq + 4 * g) = bb;
        }
      }
  }
}

// ---------------------------------------------------------------------------
// Chained transposed solve dV = P^-T dV' (Lucid_Tril_Solver.backward :328-334)
// and the column sums C_J = sum_{I >= J} M_IJ^T K^_I, M = (dV V'^T) * P.
// Workgroup = 128 columns: sub-blocks A = J0..J0+63 and B = J0+64..J0+127.
// id -> (p = NP-1 - id/BH, bh = id % BH): ids grow as p falls, so a workgroup
// waits only on later blocks held by lower ids.  counters[bh] = n means the
// last n 64-blocks of dV are published.
// wave w owns columns J0 + 32w .. +32 (one n-tile, lane <-> column) and sweeps
// all 64 rows of every later row tile I, so its column accumulators need no
// cross-wave reduction.  Each later row tile (K^ rows in bf16, dV rows) is
// staged once in LDS by direct global->LDS loads (three buffers, two tiles
// ahead, swizzled, no registers); the transposed operands dV^T and K^^T are read
// from the same tiles with transposing LDS loads:
//   S[I][J] = K^_I . K_J, P = exp(s r_J S - 1/s), G[I][J] = dV_I . V'_J
//   acc^T[d][J] += dV^T[d][I] P[I][J];  C^T[d][J] += K^^T[d][I] (G P)[I][J]
// (acc starts at -dV'^T).  Only the swept rows' K^ is rounded to bf16: its rounding
// differs from row to row, so it does not add up over the sums over I, while the
// column's own key stays exact (scaled by r_J in fp32).  The EXACT instance stages raw
// K rows and 1/rms instead and scales by r_I r_J in fp32.  Then dV_B = X_B^T R_B, dV_A = X_A^T (R_A - P_BA^T dV_B),
// R = dV' - acc, and the diagonal-block terms of C.  The chain's critical path
// is the work after the last tile becomes visible, so dV' and both inverses
// are loaded earlier.  At
// d = 64 two workgroups share a CU (LDS <= 80 KB, <= 256 registers per lane).
//
// EXACT (heads whose row mass exceeds kExactMass; each instance returns at once for the
// other heads): dV is also kept as its bf16 residual (dvbl), the staged row tiles carry
// it, V'_J's residual (vpbl) is held beside V'_J, and every product that sums over rows
// is split into hi*hi + hi*lo + lo*hi: P^T dV, G = dV V'^T, M^T K (K is exact in bf16,
// so two terms) and the in-block P_BA^T dV_B.  One workgroup per CU.
// F32 (fp32 inputs, exact, head dim 64): K also comes as hi + lo (the lo row tiles staged
// beside the others, K_J's lo part in registers, K^T's lo copy ktl), so every product with
// K takes three terms as well (four for the K.K of P); dV is written in fp32.
// ---------------------------------------------------------------------------
template <int D, bool EXACT, bool F32 = false>
struct PcolSmem;
template <int D>
struct PcolSmem<D, false, false> {
  union {
    struct {
      bf16 k[3][64 * D];   // swizzled tiles (chunk c of row r at c ^ (r & 7))
      bf16 dv[3][64 * D];
      float r[3][64];
    } st;
    struct {
      float Rt[D][132];     // R^T for the 128 columns (0..63 = A, 64..127 = B), reductions
      float Xt[64][68];     // Xt[c][r] = (P_diag^-1)[r][c] of the sub-block being solved
      bf16 vT[D][128 + 8];  // dV^T of the block (bf16, T-perm within 16-groups)
    } fin;
  } u;
};
template <int D, bool F32>
struct PcolSmem<D, true, F32> {
  static constexpr int NB = stage_bufs(D, F32);
  union {
    struct {
      bf16 k[NB][64 * D];
      bf16 dv[NB][64 * D];
      bf16 dvl[NB][64 * D];  // lo part of dV
      bf16 kl[F32 ? NB : 1][F32 ? 64 * D : 8];  // lo part of K (fp32 inputs)
      float r[NB][64];
    } st;
    struct {
      float Rt[D][132];
      float Xt[64][68];
      bf16 vT[D][128 + 8];
      bf16 vTl[D][128 + 8];  // lo part of dV^T of the block
    } fin;
  } u;
};

// DA: the head-dim columns that can be nonzero (zero-padded rows of a smaller head dim): the
// sweeps' products skip the rest; the solve and the cross term stay full width (their padded
// columns are zero because dV' and V' are)
template <int D, bool EXACT, bool F32 = false, int DA = D>
__global__ __launch_bounds__(256) LUCID_TWO_WAVES_IF(D == 64 && !EXACT) void lucid_precond_bwd_col_kernel(
    const bf16* __restrict__ k, Strides ks, int Hkv, int T, int BH, const float* __restrict__ rinv,
    const bf16* __restrict__ khat, float scale, const bf16* __restrict__ kt, const bf16* __restrict__ vpb,
    const bf16* __restrict__ vpbl, const float* __restrict__ pinv, const float* __restrict__ mass,
    const float* __restrict__ dvp,
    bf16* __restrict__ dvb, bf16* __restrict__ dvbl, std::conditional_t<F32, float, bf16>* __restrict__ dv_out,
    Strides dvs, float* __restrict__ colsum, int* __restrict__ counters, Lo lo) {
  static_assert(!F32 || EXACT, "fp32 inputs: exact instance");
  constexpr int NDT = D / 32;
  constexpr int NKS = D / 16;
  constexpr int NDT_A = (DA + 31) / 32, NKS_A = DA / 16;
  static_assert(DA % 16 == 0 && DA <= D, "active head dim");
  __shared__ __attribute__((aligned(16))) PcolSmem<D, EXACT, F32> sm;
  constexpr int NB = stage_bufs(D, F32);

  const int NT = T / 64, NP = T / 128;
  const int id = blockIdx.x;
  const int p = NP - 1 - id / BH, bh = id - (id / BH) * BH;
  if ((mass[bh] > kExactMass) != EXACT) return;  // the other instance solves this head
  const int b = bh / Hkv, h = bh - b * Hkv;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int g = lane >> 5, l32 = lane & 31;
  const int cw = w * 32;  // this wave's columns J0 + cw .. +32
  const int J0 = p * 128;
  const bf16* kh = k + b * ks.b + h * ks.h;
  const float* rv = rinv + (int64_t)bh * T;
  const bf16* kth = kt + (int64_t)bh * D * T;
  const bf16* dvbh = dvb + (int64_t)bh * T * D;
  const bf16* dvblh = dvbl + (int64_t)bh * T * D;
  const bf16* vph = vpb + (int64_t)bh * T * D;
  int* cnt = counters + bh;
  const float sl2 = scale * LOG2E_F;
  const float c0 = LOG2E_F / scale;

  const bf16* klh = F32 ? lo.k + b * ks.b + h * ks.h : nullptr;
  const bf16* ktlh = F32 ? lo.kt + (int64_t)bh * D * T : nullptr;
  // bf16 chains: the sweep stages K^ tiles (khat, rounded to bf16 once per row) against the
  // column's raw key, so an MFMA times a_j = s log2(e) r_j gives the exponent E = s log2(e)
  // r_i r_j K_i.K_j; P = exp2(E - c0) = C exp2(E) with C = 2^-c0: the sweep takes exp2(E),
  // adv starts at -dV' / C, and adv and acs are multiplied by C after the sweep.  The exact
  // instance keeps raw K tiles and the fp32 factors r_i r_j.
  const bf16* khh = EXACT ? nullptr : khat + (int64_t)bh * T * D;
  const float invC = EXACT ? 1.f : __builtin_amdgcn_exp2f(c0);
  const int jc = J0 + cw + l32;
  const float aJ = sl2 * rv[jc];
  bf16x8 kbJ[NKS], vbJ[NKS], vbJl[NKS], kbJl[NKS];
#pragma unroll
  for (int st = 0; st < NKS_A; ++st) {
    kbJ[st] = ld8(kh + (int64_t)jc * ks.t + 16 * st + 8 * g);
    vbJ[st] = ld8(vph + (int64_t)jc * D + 16 * st + 8 * g);
    if constexpr (EXACT) vbJl[st] = ld8(vpbl + ((int64_t)bh * T + jc) * D + 16 * st + 8 * g);
    if constexpr (F32) kbJl[st] = ld8(klh + (int64_t)jc * ks.t + 16 * st + 8 * g);
  }
  f32x16 adv[NDT], acs[NDT];
  {
    const float* src = dvp + ((int64_t)bh * T + jc) * D;
#pragma unroll
    for (int t = 0; t < NDT; ++t) {
      acs[t] = zero16();
#pragma unroll
      for (int qq = 0; qq < 4; ++qq) {
        const f32x4 x = *reinterpret_cast<const f32x4*>(src + t * 32 + 8 * qq + 4 * g);
#pragma unroll
        for (int u = 0; u < 4; ++u) adv[t][4 * qq + u] = -x[u] * invC;
      }
    }
  }

  // ---- sweep over the later 64-row tiles, far (published first) to near ----
  const int first = NT - 1, last = 2 * p + 2;  // tiles first, first-1, ..., last
  int ready = 0;
  // step k of the sweep stages tile first - k into buffer k % NB; the newest
  // STAGE_OPS vector memory operations of a wave are the tiles of a step
  constexpr int STAGE_OPS = (F32 ? 4 : EXACT ? 3 : 2) * (64 * (D / 8) / 256);
  const int nsteps = first - last + 1;
  int plan_k[64 * (D / 8) / 256], plan_d[64 * (D / 8) / 256];
  dma_plan<64, D / 8>(ks.t, plan_k);
  dma_plan<64, D / 8>(D, plan_d);
  auto stage = [&](int k) {
    const int i0 = (first - k) * 64, buf = k % NB;
    if constexpr (EXACT) {
      if (w == 0) dma_f32x64(rv + i0, sm.u.st.r[buf]);
      dma_stage<64, D / 8>(plan_k, kh + (int64_t)i0 * ks.t, sm.u.st.k[buf]);
    } else {
      dma_stage<64, D / 8>(plan_d, khh + (int64_t)i0 * D, sm.u.st.k[buf]);
    }
    dma_stage<64, D / 8>(plan_d, dvbh + (int64_t)i0 * D, sm.u.st.dv[buf]);
    if constexpr (EXACT) dma_stage<64, D / 8>(plan_d, dvblh + (int64_t)i0 * D, sm.u.st.dvl[buf]);
    if constexpr (F32) dma_stage<64, D / 8>(plan_k, klh + (int64_t)i0 * ks.t, sm.u.st.kl[buf]);
  };
  // issue the steps up to `upto` whose tiles are already published (tile I is
  // published once the counter exceeds NT-1-I); never blocks
  int issued = 0;
  auto try_issue = [&](int upto) {
    if (issued <= upto && issued < nsteps) {
      const int need = NT - 1 - (first - issued);
      if (need >= ready) {
        const int seen = poll_counter(cnt);
        if (seen > need) {
          chain_acquire();
          ready = seen;
        }
      }
      if (need < ready) {
        stage(issued);
        ++issued;
      }
    }
  };
  // the two inverses X_A, X_B (2 x 64 x 64 fp32) into stg[0..7]: chunk u -> sub-block u >> 2
  const float* pinv_blk = pinv + ((int64_t)bh * NT + 2 * p) * 4096;
  f32x4 xr[8];
  auto xload = [&]() {
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int idx = tid + 256 * u;
      const int sb = idx >> 10, r = (idx >> 4) & 63, c4 = (idx & 15) * 4;
      xr[u] = *reinterpret_cast<const f32x4*>(pinv_blk + sb * 4096 + r * 64 + c4);
    }
  };
  auto xstore_t = [&](int sb) {
#pragma unroll
    for (int u = 4 * sb; u < 4 * sb + 4; ++u) {
      const int idx = tid + 256 * u;
      const int r = (idx >> 4) & 63, c4 = (idx & 15) * 4;
      const f32x4 x = xr[u];
#pragma unroll
      for (int e = 0; e < 4; ++e) sm.u.fin.Xt[c4 + e][r] = x[e];
    }
  };
  if (nsteps > 0) {
    ready = wait_counter_gt(cnt, NT - 1 - first);
    stage(0);
    issued = 1;
    if (NB == 3) try_issue(1);
    if (issued > 1) dma_wait_but<STAGE_OPS>();
    else dma_wait();
  } else {
    xload();
  }
  __syncthreads();

  auto sweep_tile = [&](int buf) {
#pragma unroll
    for (int rh = 0; rh < 2; ++rh) {
      bf16x8 ka[NKS], da[NKS];
#pragma unroll
      for (int st = 0; st < NKS_A; ++st) {
        ka[st] = ld8(swz<D / 8>(sm.u.st.k[buf], rh * 32 + l32, 2 * st + g));
        da[st] = ld8(swz<D / 8>(sm.u.st.dv[buf], rh * 32 + l32, 2 * st + g));
      }
      float rI[16];
      if constexpr (EXACT) lds_rows16(&sm.u.st.r[buf][rh * 32], g, rI);
      f32x16 sc = zero16(), gg = zero16();
#pragma unroll
      for (int st = 0; st < NKS_A; ++st) {
        sc = mfma32(ka[st], kbJ[st], sc);
        gg = mfma32(da[st], vbJ[st], gg);
      }
      if constexpr (EXACT) {
#pragma unroll
        for (int st = 0; st < NKS_A; ++st) {
          gg = mfma32(da[st], vbJl[st], gg);
          gg = mfma32(ld8(swz<D / 8>(sm.u.st.dvl[buf], rh * 32 + l32, 2 * st + g)), vbJ[st], gg);
        }
      }
      if constexpr (F32) {
#pragma unroll
        for (int st = 0; st < NKS_A; ++st) {
          const bf16x8 kal = ld8(swz<D / 8>(sm.u.st.kl[buf], rh * 32 + l32, 2 * st + g));
          sc = mfma32(ka[st], kbJl[st], sc);
          sc = mfma32(kal, kbJ[st], sc);
          sc = mfma32(kal, kbJl[st], sc);
        }
      }
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const float pe = __builtin_amdgcn_exp2f(EXACT ? fmaf(sc[e] * aJ, rI[e], -c0) : sc[e] * aJ);
        sc[e] = pe;
        gg[e] = EXACT ? gg[e] * pe * rI[e] : gg[e] * pe;
      }
      const bf16x8 pb0 = pack_b(sc, 0), pb1 = pack_b(sc, 1);
      const bf16x8 mb0 = pack_b(gg, 0), mb1 = pack_b(gg, 1);
      bf16x8 pl0, pl1, ml0, ml1;  // lo parts (EXACT)
      if constexpr (EXACT) {
        pl0 = pack_lo(sc, 0, pb0);
        pl1 = pack_lo(sc, 1, pb1);
        ml0 = pack_lo(gg, 0, mb0);
        ml1 = pack_lo(gg, 1, mb1);
      }
#pragma unroll
      for (int t = 0; t < NDT_A; ++t) {
        const bf16x8 a0 = lds_tr_a<D / 8>(sm.u.st.dv[buf], rh * 32, t * 32);
        const bf16x8 a1 = lds_tr_a<D / 8>(sm.u.st.dv[buf], rh * 32 + 16, t * 32);
        const bf16x8 k0 = lds_tr_a<D / 8>(sm.u.st.k[buf], rh * 32, t * 32);
        const bf16x8 k1 = lds_tr_a<D / 8>(sm.u.st.k[buf], rh * 32 + 16, t * 32);
        adv[t] = mfma32(a0, pb0, adv[t]);
        adv[t] = mfma32(a1, pb1, adv[t]);
        acs[t] = mfma32(k0, mb0, acs[t]);
        acs[t] = mfma32(k1, mb1, acs[t]);
        if constexpr (EXACT) {
          adv[t] = mfma32(a0, pl0, adv[t]);
          adv[t] = mfma32(a1, pl1, adv[t]);
          adv[t] = mfma32(lds_tr_a<D / 8>(sm.u.st.dvl[buf], rh * 32, t * 32), pb0, adv[t]);
          adv[t] = mfma32(lds_tr_a<D / 8>(sm.u.st.dvl[buf], rh * 32 + 16, t * 32), pb1, adv[t]);
          acs[t] = mfma32(k0, ml0, acs[t]);
          acs[t] = mfma32(k1, ml1, acs[t]);
        }
        if constexpr (F32) {
          acs[t] = mfma32(lds_tr_a<D / 8>(sm.u.st.kl[buf], rh * 32, t * 32), mb0, acs[t]);
          acs[t] = mfma32(lds_tr_a<D / 8>(sm.u.st.kl[buf], rh * 32 + 16, t * 32), mb1, acs[t]);
        }
      }
    }
  };
  // all steps but the last; the last one is peeled so that the inverses it
  // prefetches do not hold registers through the loop
  for (int ks_ = 0; ks_ + 1 < nsteps; ++ks_) {
    try_issue(ks_ + NB - 1);
    sweep_tile(ks_ % NB);
    if (issued == ks_ + 1) {  // the next tile was not published yet: wait for it
      ready = wait_counter_gt(cnt, NT - 1 - (first - issued));
      stage(issued);
      ++issued;
    }
    if (issued > ks_ + 2) dma_wait_but<STAGE_OPS>();  // the step after next may stay in flight
    else dma_wait();
    __syncthreads();
  }
  if (nsteps > 0) {
    xload();  // fetch the inverses while the last tile is processed
    sweep_tile((nsteps - 1) % NB);
    dma_wait();
    __syncthreads();
  }

  if constexpr (!EXACT) {  // the sweep's factor 1/C
    const float Cf = __builtin_amdgcn_exp2f(-c0);
#pragma unroll
    for (int t = 0; t < NDT; ++t)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        adv[t][e] *= Cf;
        acs[t][e] *= Cf;
      }
  }
  // ---- R = dV' - acc = -adv for this wave's columns; X^T of sub-block B ----
  float(*Rt)[132] = sm.u.fin.Rt;
#pragma unroll
  for (int t = 0; t < NDT; ++t)
#pragma unroll
    for (int e = 0; e < 16; ++e) Rt[t * 32 + drow(e, g)][cw + l32] = -adv[t][e];
  xstore_t(1);
  __syncthreads();

  // dV^T[d][c] = sum_r R^T[d][r] X[r][c] for sub-block sb (X lower: r >= c)
  auto diag_solve = [&](int sb) {
    for (int tile = w; tile < NDT * 2; tile += 4) {
      const int dt = tile >> 1, chh = tile & 1;
      f32x16 o = zero16();
      for (int st = chh ? 2 : 0; st < 4; ++st) {
        bf16x8 ah, al, bh8, bl;
        split8(&Rt[dt * 32 + l32][sb * 64 + 16 * st + 8 * g], ah, al);
        split8(&sm.u.fin.Xt[chh * 32 + l32][16 * st + 8 * g], bh8, bl);
        o = mfma32(ah, bh8, o);
        o = mfma32(ah, bl, o);
        o = mfma32(al, bh8, o);
      }
      const int cl = chh * 32 + l32;
      const int r = J0 + sb * 64 + cl;
      const int lslot = sb * 64 + ((cl & ~15) | jmap(cl & 15));
      bf16* ob = dvb + ((int64_t)bh * T + r) * D;
      auto* ou = dv_out + b * dvs.b + h * dvs.h + (int64_t)r * dvs.t;
#pragma unroll
      for (int qq = 0; qq < 4; ++qq) {
        const int d0 = dt * 32 + 8 * qq + 4 * g;
        bf16x4 bb, bl;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          bb[u] = (bf16)o[4 * qq + u];
          sm.u.fin.vT[d0 + u][lslot] = bb[u];
          if constexpr (EXACT) {
            bl[u] = (bf16)(o[4 * qq + u] - (float)bb[u]);
            sm.u.fin.vTl[d0 + u][lslot] = bl[u];
          }
        }
        *reinterpret_cast<bf16x4*>(ob + d0) = bb;
        if constexpr (F32) {
          f32x4 x;
#pragma unroll
          for (int u = 0; u < 4; ++u) x[u] = o[4 * qq + u];
          *reinterpret_cast<f32x4*>(ou + d0) = x;
        } else {
          *reinterpret_cast<bf16x4*>(ou + d0) = bb;
        }
        if constexpr (EXACT) *reinterpret_cast<bf16x4*>(dvbl + ((int64_t)bh * T + r) * D + d0) = bl;
      }
    }
  };
  diag_solve(1);
  publish_counter(cnt, NT - (2 * p + 1));

  // ---- R_A -= P_BA^T dV_B: wave -> (A columns half na, B rows half kb) ----
  {
    const int na = w & 1, kb = w >> 1;
    const int colA = J0 + na * 32 + l32;
    f32x16 sc = zero16();
#pragma unroll
    for (int st = 0; st < NKS; ++st) {
      const int64_t om = (int64_t)(J0 + 64 + kb * 32 + l32) * ks.t + 16 * st + 8 * g;
      const int64_t on = (int64_t)colA * ks.t + 16 * st + 8 * g;
      sc = mfma32(ld8(kh + om), ld8(kh + on), sc);
      if constexpr (F32) {
        sc = mfma32(ld8(kh + om), ld8(klh + on), sc);
        sc = mfma32(ld8(klh + om), ld8(kh + on), sc);
      }
    }
    const float aA = sl2 * rv[colA];
    float rB[16];
    load_rows16(rv + J0 + 64 + kb * 32, g, rB);
#pragma unroll
    for (int e = 0; e < 16; ++e) sc[e] = __builtin_amdgcn_exp2f(fmaf(sc[e] * aA, rB[e], -c0));
    const bf16x8 p0 = pack_b(sc, 0), p1 = pack_b(sc, 1);
    f32x16 cr[NDT];
#pragma unroll
    for (int t = 0; t < NDT; ++t) {
      const bf16x8 v0 = ld8(&sm.u.fin.vT[t * 32 + l32][64 + kb * 32 + 8 * g]);
      const bf16x8 v1 = ld8(&sm.u.fin.vT[t * 32 + l32][64 + kb * 32 + 16 + 8 * g]);
      cr[t] = mfma32(v0, p0, zero16());
      cr[t] = mfma32(v1, p1, cr[t]);
      if constexpr (EXACT) {
        cr[t] = mfma32(v0, pack_lo(sc, 0, p0), cr[t]);
        cr[t] = mfma32(v1, pack_lo(sc, 1, p1), cr[t]);
        cr[t] = mfma32(ld8(&sm.u.fin.vTl[t * 32 + l32][64 + kb * 32 + 8 * g]), p0, cr[t]);
        cr[t] = mfma32(ld8(&sm.u.fin.vTl[t * 32 + l32][64 + kb * 32 + 16 + 8 * g]), p1, cr[t]);
      }
    }
    const int col = na * 32 + l32;
    if (kb == 1) {
#pragma unroll
      for (int t = 0; t < NDT; ++t)
#pragma unroll
        for (int e = 0; e < 16; ++e) Rt[t * 32 + drow(e, g)][col] -= cr[t][e];
    }
    xstore_t(0);
    __syncthreads();
    if (kb == 0) {
#pragma unroll
      for (int t = 0; t < NDT; ++t)
#pragma unroll
        for (int e = 0; e < 16; ++e) Rt[t * 32 + drow(e, g)][col] -= cr[t][e];
    }
    __syncthreads();
  }
  diag_solve(0);
  publish_counter(cnt, NT - 2 * p);

  // ---- diagonal-block terms of the column sums (rows r >= columns c inside the workgroup) ----
  // wave w: its 32 columns (sub-block w >> 1) against rows of sub-blocks rb = w >> 1 .. 1
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) {
    if (rb < (w >> 1)) continue;
#pragma unroll
    for (int rh = 0; rh < 2; ++rh) {
      if (rb * 64 + rh * 32 + 31 < cw) continue;  // rows all above this wave's columns
      const int rbase = J0 + rb * 64 + rh * 32;
      bf16x8 ka[NKS], da[NKS];
#pragma unroll
      for (int st = 0; st < NKS_A; ++st) {
        ka[st] = ld8(kh + (int64_t)(rbase + l32) * ks.t + 16 * st + 8 * g);
        da[st] = ld8(dvbh + (int64_t)(rbase + l32) * D + 16 * st + 8 * g);
      }
      float rr[16];
      load_rows16(rv + rbase, g, rr);
      f32x16 sc = zero16(), gg = zero16();
#pragma unroll
      for (int st = 0; st < NKS_A; ++st) {
        sc = mfma32(ka[st], kbJ[st], sc);
        gg = mfma32(da[st], vbJ[st], gg);
      }
      if constexpr (EXACT) {
#pragma unroll
        for (int st = 0; st < NKS_A; ++st) {
          gg = mfma32(da[st], vbJl[st], gg);
          gg = mfma32(ld8(dvblh + (int64_t)(rbase + l32) * D + 16 * st + 8 * g), vbJ[st], gg);
        }
      }
      if constexpr (F32) {
#pragma unroll
        for (int st = 0; st < NKS_A; ++st) {
          const bf16x8 kal = ld8(klh + (int64_t)(rbase + l32) * ks.t + 16 * st + 8 * g);
          sc = mfma32(ka[st], kbJl[st], sc);
          sc = mfma32(kal, kbJ[st], sc);
          sc = mfma32(kal, kbJl[st], sc);
        }
      }
      // strictly below the diagonal: the diagonal terms M_jj K^_j lie along K^_j and are
      // added by the row kernel in closed form (they cancel in the RMSNorm backward)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int rloc = rb * 64 + rh * 32 + drow(e, g), cloc = cw + l32;
        const float pe = (rloc > cloc) ? __builtin_amdgcn_exp2f(fmaf(sc[e] * aJ, rr[e], -c0)) : 0.f;
        gg[e] = gg[e] * pe * rr[e];
      }
      const bf16x8 mb0 = pack_b(gg, 0), mb1 = pack_b(gg, 1);
#pragma unroll
      for (int t = 0; t < NDT_A; ++t) {
        const bf16* kp = kth + (int64_t)(t * 32 + l32) * T + rbase + 8 * g;
        acs[t] = mfma32(ld8(kp), mb0, acs[t]);
        acs[t] = mfma32(ld8(kp + 16), mb1, acs[t]);
        if constexpr (EXACT) {
          acs[t] = mfma32(ld8(kp), pack_lo(gg, 0, mb0), acs[t]);
          acs[t] = mfma32(ld8(kp + 16), pack_lo(gg, 1, mb1), acs[t]);
        }
        if constexpr (F32) {
          const bf16* kpl = ktlh + (int64_t)(t * 32 + l32) * T + rbase + 8 * g;
          acs[t] = mfma32(ld8(kpl), mb0, acs[t]);
          acs[t] = mfma32(ld8(kpl + 16), mb1, acs[t]);
        }
      }
    }
  }
  // ---- store the column sums of this wave's columns ----
  {
    float* dst = colsum + ((int64_t)bh * T + jc) * D;
#pragma unroll
    for (int t = 0; t < NDT; ++t)
#pragma unroll
      for (int qq = 0; qq < 4; ++qq) {
        f32x4 x;
#pragma unroll
        for (int u = 0; u < 4; ++u) x[u] = acs[t][4 * qq + u];
        *reinterpret_cast<f32x4*>(dst + t * 32 + 8 * qq + 4 * g) = x;
      }
  }
}

// ---------------------------------------------------------------------------
// The column chain with 256 columns per workgroup (head dim 64, bf16 chains; the default
// when T is a multiple of 256): eight waves, wave w owns columns J0 + 32w .. +32 of the
// four 64-column sub-blocks A..D (w >> 1), so every staged row tile (K^ rows, dV rows)
// serves twice the columns of lucid_precond_bwd_col_kernel and a head's tiles are
// fetched half as often.  The sweep body is that kernel's.  After the sweep over the
// rows below the block, the sub-blocks are solved from the last (D) to the first (A):
//   dV_s = X_s^T R_s  (R_s = dV'_s - acc_s, X_s = P_ss^-1), published as the head's next
//   64-row block; its dV rows (bf16, from the solve) and K^ rows are put in LDS in the
//   sweep layout, and the waves of the earlier sub-blocks take them as one more sweep
//   step (P^T dV and the M^T K^ column sums), while the two waves of sub-block s add the
//   strictly lower in-block terms of their column sums (rows r > c of the same block).
// So the in-block coupling needs no separate cross-term phase and a head has half as many
// hand-offs.  counters[bh] = n: the last n 64-row blocks of dV are published (as in
// lucid_precond_bwd_col_kernel).  Heads of the exact chains return at once.
// ---------------------------------------------------------------------------
template <int D>
struct PcolWideSmem {
  bf16 k[3][64 * D];  // staged row tiles, K^ and dV (swizzled, chunk c of row r at c ^ (r & 7))
  bf16 dv[3][64 * D];
  float Rt[D][68];    // R^T of the sub-block being solved
  float Xt[64][68];   // Xt[c][r] = X[r][c] of that sub-block
  bf16 sk[64 * D];    // the solved sub-block as a row tile: K^ rows, dV rows
  bf16 sdv[64 * D];
};

template <int D>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2))) void lucid_precond_bwd_col_wide_kernel(
    const bf16* __restrict__ k, Strides ks, int Hkv, int T, int BH, const float* __restrict__ rinv,
    const bf16* __restrict__ khat, float scale, const bf16* __restrict__ vpb, const float* __restrict__ pinv,
    const float* __restrict__ mass,
    const float* __restrict__ dvp, bf16* __restrict__ dvb, bf16* __restrict__ dv_out, Strides dvs,
    float* __restrict__ colsum, int* __restrict__ counters) {
  static_assert(D == 64, "wide column chain: head dim 64");
  constexpr int NDT = D / 32;
  constexpr int NKS = D / 16;
  constexpr int NTHR = 512;
  constexpr int SW = 0;  // (the conflict-free swizzle, SW = 1, costs more VALU address work here than it saves)
  __shared__ __attribute__((aligned(16))) PcolWideSmem<D> sm;

  const int NT = T / 64, NP = T / 256;
  const int id = blockIdx.x;
  const int p = NP - 1 - id / BH, bh = id - (id / BH) * BH;
  if (mass[bh] > kExactMass) return;  // the exact instance of the 128-column chain solves this head
  const int b = bh / Hkv, h = bh - b * Hkv;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int g = lane >> 5, l32 = lane & 31;
  const int sbw = w >> 1;         // this wave's sub-block
  const int J0 = p * 256;
  const int jc = J0 + 32 * w + l32;  // this lane's column
  const bf16* kh = k + b * ks.b + h * ks.h;
  const bf16* khh = khat + (int64_t)bh * T * D;
  const float* rv = rinv + (int64_t)bh * T;
  const bf16* dvbh = dvb + (int64_t)bh * T * D;
  const bf16* vph = vpb + (int64_t)bh * T * D;
  int* cnt = counters + bh;
  const float sl2 = scale * LOG2E_F;
  const float c0 = LOG2E_F / scale;

  // the staged K^_i rows (rounded to bf16 once per row) against the column's raw key: an
  // MFMA times aJ gives E = s log2(e) r_i r_j K_i.K_j, and P = exp2(E - c0) = C exp2(E) with
  // C = 2^-c0, so the sweep takes exp2(E) and the accumulators carry a factor 1/C (adv
  // starts at -dV' / C; both are multiplied by C where they are read)
  const float aJ = sl2 * rv[jc];
  const float Cf = __builtin_amdgcn_exp2f(-c0), invC = __builtin_amdgcn_exp2f(c0);
  bf16x8 kbJ[NKS], vbJ[NKS];
#pragma unroll
  for (int st = 0; st < NKS; ++st) {
    kbJ[st] = ld8(kh + (int64_t)jc * ks.t + 16 * st + 8 * g);
    vbJ[st] = ld8(vph + (int64_t)jc * D + 16 * st + 8 * g);
  }
  f32x16 adv[NDT], acs[NDT];
  {
    const float* src = dvp + ((int64_t)bh * T + jc) * D;
#pragma unroll
    for (int t = 0; t < NDT; ++t) {
      acs[t] = zero16();
#pragma unroll
      for (int qq = 0; qq < 4; ++qq) {
        const f32x4 x = *reinterpret_cast<const f32x4*>(src + t * 32 + 8 * qq + 4 * g);
#pragma unroll
        for (int u = 0; u < 4; ++u) adv[t][4 * qq + u] = -x[u] * invC;
      }
    }
  }

  // one 64-row tile (K^ rows, dV rows) against this wave's columns: acc^T += dV^T P,
  // C^T += K^^T (G P); DIAG: the rows of this wave's own sub-block, strictly below its
  // columns, C only
  auto sweep_rows = [&](const bf16* tk, const bf16* tdv, const bool DIAG) {
#pragma unroll
    for (int rh = 0; rh < 2; ++rh) {
      if (DIAG && rh * 32 + 31 <= (w & 1) * 32) continue;  // rows all at or above the columns
      bf16x8 ka[NKS], da[NKS];
#pragma unroll
      for (int st = 0; st < NKS; ++st) {
        ka[st] = ld8(swz<D / 8, SW>(tk, rh * 32 + l32, 2 * st + g));
        da[st] = ld8(swz<D / 8, SW>(tdv, rh * 32 + l32, 2 * st + g));
      }
      f32x16 sc = zero16(), gg = zero16();
#pragma unroll
      for (int st = 0; st < NKS; ++st) {
        sc = mfma32(ka[st], kbJ[st], sc);
        gg = mfma32(da[st], vbJ[st], gg);
      }
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        float pe = __builtin_amdgcn_exp2f(sc[e] * aJ);
        // strictly below the diagonal: the diagonal terms M_jj K^_j are added by the row
        // kernel in closed form
        if (DIAG && rh * 32 + drow(e, g) <= (w & 1) * 32 + l32) pe = 0.f;
        sc[e] = pe;
        gg[e] = gg[e] * pe;
      }
      const bf16x8 pb0 = pack_b(sc, 0), pb1 = pack_b(sc, 1);
      const bf16x8 mb0 = pack_b(gg, 0), mb1 = pack_b(gg, 1);
#pragma unroll
      for (int t = 0; t < NDT; ++t) {
        const bf16x8 k0 = lds_tr_a<D / 8, SW>(tk, rh * 32, t * 32);
        const bf16x8 k1 = lds_tr_a<D / 8, SW>(tk, rh * 32 + 16, t * 32);
        if (!DIAG) {
          const bf16x8 a0 = lds_tr_a<D / 8, SW>(tdv, rh * 32, t * 32);
          const bf16x8 a1 = lds_tr_a<D / 8, SW>(tdv, rh * 32 + 16, t * 32);
          adv[t] = mfma32(a0, pb0, adv[t]);
          adv[t] = mfma32(a1, pb1, adv[t]);
        }
        acs[t] = mfma32(k0, mb0, acs[t]);
        acs[t] = mfma32(k1, mb1, acs[t]);
      }
    }
  };

  // ---- sweep over the 64-row tiles below the block, far (published first) to near ----
  const int first = NT - 1, last = 4 * p + 4;
  int ready = 0;
  constexpr int PER = 64 * (D / 8) / NTHR;  // 16-byte loads per thread for a 64-row tile
  constexpr int STAGE_OPS = 2 * PER;
  const int nsteps = first - last + 1;
  int plan_d[PER];  // K^ and dV rows: row stride D
  dma_plan<64, D / 8, NTHR, SW>(D, plan_d);
  auto stage = [&](int kk) {
    const int i0 = (first - kk) * 64, buf = kk % 3;
    dma_stage<64, D / 8, NTHR>(plan_d, khh + (int64_t)i0 * D, sm.k[buf]);
    dma_stage<64, D / 8, NTHR>(plan_d, dvbh + (int64_t)i0 * D, sm.dv[buf]);
  };
  int issued = 0;
  auto try_issue = [&](int upto) {
    if (issued <= upto && issued < nsteps) {
      const int need = NT - 1 - (first - issued);
      if (need >= ready) {
        const int seen = poll_counter(cnt);
        if (seen > need) {
          chain_acquire();
          ready = seen;
        }
      }
      if (need < ready) {
        stage(issued);
        ++issued;
      }
    }
  };
  if (nsteps > 0) {
    ready = wait_counter_gt(cnt, NT - 1 - first);
    stage(0);
    issued = 1;
    try_issue(1);
    if (issued > 1) dma_wait_but<STAGE_OPS>();
    else dma_wait();
  }
  __syncthreads();
  for (int ks_ = 0; ks_ < nsteps; ++ks_) {
    try_issue(ks_ + 2);
    sweep_rows(sm.k[ks_ % 3], sm.dv[ks_ % 3], false);
    if (ks_ + 1 < nsteps && issued == ks_ + 1) {  // the next tile was not published yet: wait for it
      ready = wait_counter_gt(cnt, NT - 1 - (first - issued));
      stage(issued);
      ++issued;
    }
    if (issued > ks_ + 2) dma_wait_but<STAGE_OPS>();  // the step after next may stay in flight
    else dma_wait();
    __syncthreads();
  }

  // ---- the block's sub-blocks, last to first ----
  for (int s = 3; s >= 0; --s) {
    const int r0 = J0 + 64 * s;  // first row (= column) of sub-block s
    // its K^ rows into the solved-tile slot (read only after the barriers below)
    dma_stage<64, D / 8, NTHR>(plan_d, khh + (int64_t)r0 * D, sm.sk);
    // R^T of its columns (its two waves) and X^T
    if (sbw == s) {
#pragma unroll
      for (int t = 0; t < NDT; ++t)
#pragma unroll
        for (int e = 0; e < 16; ++e) sm.Rt[t * 32 + drow(e, g)][(w & 1) * 32 + l32] = -Cf * adv[t][e];
    }
    {
      const float* xb = pinv + ((int64_t)bh * NT + 4 * p + s) * 4096;
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int idx = tid + NTHR * u;  // 1024 chunks of 4
        const int r = idx >> 4, c4 = (idx & 15) * 4;
        const f32x4 x = *reinterpret_cast<const f32x4*>(xb + r * 64 + c4);
#pragma unroll
        for (int e = 0; e < 4; ++e) sm.Xt[c4 + e][r] = x[e];
      }
    }
    __syncthreads();
    // dV^T[d][c] = sum_r R^T[d][r] X[r][c] (X lower: r >= c): four 32x32 tiles, waves 0..3
    if (w < 4) {
      const int dt = w >> 1, chh = w & 1;
      f32x16 o = zero16();
      for (int st = chh ? 2 : 0; st < 4; ++st) {
        bf16x8 ah, al, bh8, bl;
        split8(&sm.Rt[dt * 32 + l32][16 * st + 8 * g], ah, al);
        split8(&sm.Xt[chh * 32 + l32][16 * st + 8 * g], bh8, bl);
        o = mfma32(ah, bh8, o);
        o = mfma32(ah, bl, o);
        o = mfma32(al, bh8, o);
      }
      const int cl = chh * 32 + l32;  // row of dV inside the sub-block
      const int r = r0 + cl;
      bf16* ob = dvb + ((int64_t)bh * T + r) * D;
      bf16* ou = dv_out + b * dvs.b + h * dvs.h + (int64_t)r * dvs.t;
#pragma unroll
      for (int qq = 0; qq < 4; ++qq) {
        const int d0 = dt * 32 + 8 * qq + 4 * g;
        bf16x4 bb;
#pragma unroll
        for (int u = 0; u < 4; ++u) bb[u] = (bf16)o[4 * qq + u];
        *reinterpret_cast<bf16x4*>(ob + d0) = bb;
        *reinterpret_cast<bf16x4*>(ou + d0) = bb;
        *reinterpret_cast<bf16x4*>(sm.sdv + swz_off<D / 8, SW>(cl, d0 >> 3) + (d0 & 7)) = bb;
      }
    }
    dma_wait();
    publish_counter(cnt, NT - (4 * p + s));  // waits for every wave's stores, then a barrier
    // the solved rows against the earlier sub-blocks' columns; the strictly lower in-block
    // column-sum terms for sub-block s's own columns
    if (sbw < s) sweep_rows(sm.sk, sm.sdv, false);
    else if (sbw == s) sweep_rows(sm.sk, sm.sdv, true);
    __syncthreads();  // before the next sub-block overwrites Rt, Xt and the solved-tile slots
  }
  // ---- the column sums of this wave's columns ----
  {
    float* dst = colsum + ((int64_t)bh * T + jc) * D;
#pragma unroll
    for (int t = 0; t < NDT; ++t)
#pragma unroll
      for (int qq = 0; qq < 4; ++qq) {
        f32x4 x;
#pragma unroll
        for (int u = 0; u < 4; ++u) x[u] = Cf * acs[t][4 * qq + u];
        *reinterpret_cast<f32x4*>(dst + t * 32 + 8 * qq + 4 * g) = x;
      }
  }
}

// ---------------------------------------------------------------------------
// Row sums R_I = sum_{J <= I} M_IJ K^_J, then dK^ = -s (R + C), the RMSNorm
// backward and the attention dK (dka; null for the preconditioner-only backward).
// No chain: every dV is known.
// Workgroup = 256 rows (heavy, late blocks first); wave w owns rows 64w .. +64
// (two 32-row n-tiles, lane <-> row) and sweeps both 32-key halves of every
// staged 64-key tile J (K^ rows in bf16, V' rows; direct global->LDS loads, three
// buffers, two tiles ahead; K^T operands through transposing LDS loads):
//   E^T[J][I] = s log2(e) r_I (K^_J . K_I), G^T[J][I] = V'_J . dV_I,
//   R^T[d][I] += K^^T[d][J] (G exp2(E))^T[J][I]   (P = exp2(E - c0) = 2^-c0 exp2(E): R is
//   multiplied by 2^-c0 after the sweep)
// Only the swept keys' K^ is rounded to bf16 (a rounding that differs from key to key and
// does not add up over the sum over J); the row's own key stays exact.
// Each wave finishes its own rows, so no cross-wave reduction is needed.
// EXACT (heads whose row mass exceeds kExactMass; each instance returns at once for the
// other heads): the exponents come from raw K tiles times fp32 factors r_I r_J, and
// G = V' dV^T and M K are split into hi*hi + hi*lo + lo*hi with the lo parts of V'
// (staged beside V') and dV (held beside dV); one workgroup per CU.
// ---------------------------------------------------------------------------
template <int D, bool EXACT, bool F32 = false>
struct ProwSmem {
  bf16 k[3][64 * D];  // swizzled K^ tiles (chunk c of row r at c ^ (r & 7))
  bf16 v[3][64 * D];
};
template <int D, bool F32>
struct ProwSmem<D, true, F32> {
  static constexpr int NB = stage_bufs(D, F32);
  bf16 k[NB][64 * D];
  bf16 v[NB][64 * D];
  bf16 vl[NB][64 * D];  // lo part of V'
  bf16 kl[F32 ? NB : 1][F32 ? 64 * D : 8];  // lo part of K (fp32 inputs)
  float r[NB][64];
};

// NT: 32-row n-tiles per wave (2: 256 rows per workgroup; 1: 128 rows, for the fp32 instance
// at head dim 128, whose hi/lo row operands of two n-tiles do not fit the registers)
template <int D, bool EXACT, bool F32 = false, int NT = 2>
__global__ __launch_bounds__(256) LUCID_TWO_WAVES_IF(D == 64 && !EXACT) void lucid_precond_bwd_row_kernel(
    const bf16* __restrict__ k, Strides ks, int Hkv, int T, int BH, const float* __restrict__ rinv,
    const bf16* __restrict__ khat, float scale, float dn, const bf16* __restrict__ vpb,
    const bf16* __restrict__ vpbl, const bf16* __restrict__ dvb,
    const bf16* __restrict__ dvbl, const float* __restrict__ mass, const float* __restrict__ colsum,
    const float* __restrict__ dka, std::conditional_t<F32, float, bf16>* __restrict__ dk_out, Strides dks, Lo lo) {
  static_assert(!F32 || EXACT, "fp32 inputs: exact instance");
  constexpr int NDT = D / 32;
  constexpr int NKS = D / 16;
  __shared__ __attribute__((aligned(16))) ProwSmem<D, EXACT, F32> sm;
  constexpr int NB = stage_bufs(D, F32);
  constexpr int WGR = 128 * NT;  // rows per workgroup
  const int nblk = (T + WGR - 1) / WGR;
  const int id = blockIdx.x;
  const int ib = nblk - 1 - id / BH, bh = id - (id / BH) * BH;  // heavy (late) blocks first
  if ((mass[bh] > kExactMass) != EXACT) return;  // the other instance handles this head
  const int b = bh / Hkv, h = bh - b * Hkv;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int g = lane >> 5, l32 = lane & 31;
  const int row0 = ib * WGR + w * 32 * NT;  // this wave's rows (T is a multiple of 128: all or none are < T)
  const bool active = row0 < T;
  const bf16* kh = k + b * ks.b + h * ks.h;
  const float* rv = rinv + (int64_t)bh * T;
  const bf16* vh = vpb + (int64_t)bh * T * D;
  const bf16* khh = EXACT ? nullptr : khat + (int64_t)bh * T * D;  // the exact instance reads raw K
  const float sl2 = scale * LOG2E_F;
  const float c0 = LOG2E_F / scale;

  const bf16* klh = F32 ? lo.k + b * ks.b + h * ks.h : nullptr;
  bf16x8 kbI[NT][NKS], dbI[NT][NKS], dbIl[NT][NKS], kbIl[NT][NKS];
  float aI[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int ir = active ? row0 + nt * 32 + l32 : 0;
    aI[nt] = sl2 * rv[ir];
#pragma unroll
    for (int st = 0; st < NKS; ++st) {
      kbI[nt][st] = ld8(kh + (int64_t)ir * ks.t + 16 * st + 8 * g);
      if constexpr (F32) kbIl[nt][st] = ld8(klh + (int64_t)ir * ks.t + 16 * st + 8 * g);
      dbI[nt][st] = ld8(dvb + ((int64_t)bh * T + ir) * D + 16 * st + 8 * g);
      if constexpr (EXACT) dbIl[nt][st] = ld8(dvbl + ((int64_t)bh * T + ir) * D + 16 * st + 8 * g);
    }
  }
  f32x16 acc[NDT][NT];
#pragma unroll
  for (int t = 0; t < NDT; ++t)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) acc[t][nt] = zero16();
  const int ntile = min((ib + 1) * (WGR / 64), T / 64);  // key tiles 0 .. ntile-1 (>= 2 since T >= 128)
  // newest vector-memory ops of a step, per wave
  constexpr int STAGE_OPS = (F32 ? 4 : EXACT ? 3 : 2) * (64 * (D / 8) / 256);
  int plan_k[64 * (D / 8) / 256], plan_v[64 * (D / 8) / 256];
  dma_plan<64, D / 8>(ks.t, plan_k);
  dma_plan<64, D / 8>(D, plan_v);
  auto stage = [&](int J) {
    const int j0 = J * 64, buf = J % NB;
    if constexpr (EXACT) {
      if (w == 0) dma_f32x64(rv + j0, sm.r[buf]);
      dma_stage<64, D / 8>(plan_k, kh + (int64_t)j0 * ks.t, sm.k[buf]);
    } else {
      dma_stage<64, D / 8>(plan_v, khh + (int64_t)j0 * D, sm.k[buf]);
    }
    dma_stage<64, D / 8>(plan_v, vh + (int64_t)j0 * D, sm.v[buf]);
    if constexpr (EXACT) dma_stage<64, D / 8>(plan_v, vpbl + (int64_t)bh * T * D + (int64_t)j0 * D, sm.vl[buf]);
    if constexpr (F32) dma_stage<64, D / 8>(plan_k, klh + (int64_t)j0 * ks.t, sm.kl[buf]);
  };
  stage(0);
  if (NB == 3) {  // ntile >= 2 (T >= 128)
    stage(1);
    dma_wait_but<STAGE_OPS>();
  } else {
    dma_wait();
  }
  __syncthreads();
  // this wave's rows are the 64-block row0 / 64; key tiles after it are fully masked
  const int last_w = row0 / 64;
  const int roff = row0 - last_w * 64;  // the wave's first row inside that block (32 at NT = 1 for odd waves)
  auto tile = [&](int buf, bool diag) {
#pragma unroll 1
    for (int jh = 0; jh < 2; ++jh) {
      bf16x8 ka[NKS], va[NKS];
#pragma unroll
      for (int st = 0; st < NKS; ++st) {
        ka[st] = ld8(swz<D / 8>(sm.k[buf], jh * 32 + l32, 2 * st + g));
        va[st] = ld8(swz<D / 8>(sm.v[buf], jh * 32 + l32, 2 * st + g));
      }
      float rJ[16];
      if constexpr (EXACT) lds_rows16(&sm.r[buf][jh * 32], g, rJ);
      bf16x8 mb[NT][2], ml[NT][2];
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        f32x16 sc = zero16(), gg = zero16();
#pragma unroll
        for (int st = 0; st < NKS; ++st) {
          sc = mfma32(ka[st], kbI[nt][st], sc);
          gg = mfma32(va[st], dbI[nt][st], gg);
        }
        if constexpr (EXACT) {
#pragma unroll
          for (int st = 0; st < NKS; ++st) {
            gg = mfma32(va[st], dbIl[nt][st], gg);
            gg = mfma32(ld8(swz<D / 8>(sm.vl[buf], jh * 32 + l32, 2 * st + g)), dbI[nt][st], gg);
          }
        }
        if constexpr (F32) {
#pragma unroll
          for (int st = 0; st < NKS; ++st) {
            const bf16x8 kal = ld8(swz<D / 8>(sm.kl[buf], jh * 32 + l32, 2 * st + g));
            sc = mfma32(ka[st], kbIl[nt][st], sc);
            sc = mfma32(kal, kbI[nt][st], sc);
            sc = mfma32(kal, kbIl[nt][st], sc);
          }
        }
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          float pe = __builtin_amdgcn_exp2f(EXACT ? fmaf(sc[e] * aI[nt], rJ[e], -c0) : sc[e] * aI[nt]);
          // j >= i masked: the diagonal term is added in closed form after the sweep
          if (diag && jh * 32 + drow(e, g) >= roff + nt * 32 + l32) pe = 0.f;
          gg[e] = EXACT ? gg[e] * pe * rJ[e] : gg[e] * pe;
        }
        mb[nt][0] = pack_b(gg, 0);
        mb[nt][1] = pack_b(gg, 1);
        if constexpr (EXACT) {
          ml[nt][0] = pack_lo(gg, 0, mb[nt][0]);
          ml[nt][1] = pack_lo(gg, 1, mb[nt][1]);
        }
      }
#pragma unroll
      for (int t = 0; t < NDT; ++t) {
        const bf16x8 k0 = lds_tr_a<D / 8>(sm.k[buf], jh * 32, t * 32);
        const bf16x8 k1 = lds_tr_a<D / 8>(sm.k[buf], jh * 32 + 16, t * 32);
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          acc[t][nt] = mfma32(k0, mb[nt][0], acc[t][nt]);
          acc[t][nt] = mfma32(k1, mb[nt][1], acc[t][nt]);
          if constexpr (EXACT) {
            acc[t][nt] = mfma32(k0, ml[nt][0], acc[t][nt]);
            acc[t][nt] = mfma32(k1, ml[nt][1], acc[t][nt]);
          }
          if constexpr (F32) {
            acc[t][nt] = mfma32(lds_tr_a<D / 8>(sm.kl[buf], jh * 32, t * 32), mb[nt][0], acc[t][nt]);
            acc[t][nt] = mfma32(lds_tr_a<D / 8>(sm.kl[buf], jh * 32 + 16, t * 32), mb[nt][1], acc[t][nt]);
          }
        }
      }
    }
  };
  for (int J = 0; J < ntile; ++J) {
    const int buf = J % NB;
    if (J + NB - 1 < ntile) stage(J + NB - 1);
    if (active) {
      if (J < last_w) tile(buf, false);
      else if (J == last_w) tile(buf, true);
    }
    if (NB == 3 && J + 2 < ntile) dma_wait_but<STAGE_OPS>();  // the step after next may stay in flight
    else dma_wait();
    __syncthreads();
  }
  if (!active) return;
  const float accf = EXACT ? 1.f : __builtin_amdgcn_exp2f(-c0);  // the bf16 sweep's 2^-c0
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int irow = row0 + nt * 32 + l32;
    const float ri = rv[irow];
    const float* cs = colsum + ((int64_t)bh * T + irow) * D;
    const float* da = dka + ((int64_t)bh * T + irow) * D;
    const bf16* kr = kh + (int64_t)irow * ks.t;
    const bf16* dvr = dvb + ((int64_t)bh * T + irow) * D;
    const bf16* vpr = vh + (int64_t)irow * D;
    float dkh[NDT][16], khat[NDT][16];
    float dotp = 0.f, kss = 0.f, gdot = 0.f;
#pragma unroll
    for (int t = 0; t < NDT; ++t)
#pragma unroll
      for (int qq = 0; qq < 4; ++qq) {
        const int d0 = t * 32 + 8 * qq + 4 * g;
        const f32x4 cv = *reinterpret_cast<const f32x4*>(cs + d0);
        const bf16x4 kv = *reinterpret_cast<const bf16x4*>(kr + d0);
        bf16x4 kvl;
        if constexpr (F32) kvl = *reinterpret_cast<const bf16x4*>(klh + (int64_t)irow * ks.t + d0);
        const bf16x4 dv4 = *reinterpret_cast<const bf16x4*>(dvr + d0);
        const bf16x4 vp4 = *reinterpret_cast<const bf16x4*>(vpr + d0);
        bf16x4 dv4l, vp4l;
        if constexpr (EXACT) {
          dv4l = *reinterpret_cast<const bf16x4*>(dvbl + ((int64_t)bh * T + irow) * D + d0);
          vp4l = *reinterpret_cast<const bf16x4*>(vpbl + ((int64_t)bh * T + irow) * D + d0);
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int e = 4 * qq + u;
          const float x = -scale * (accf * acc[t][nt][e] + cv[u]);
          const float kk = ri * ((float)kv[u] + (F32 ? (float)kvl[u] : 0.f));
          dkh[t][e] = x;
          khat[t][e] = kk;
          dotp += x * kk;
          kss += kk * kk;
          const float dvv = (float)dv4[u] + (EXACT ? (float)dv4l[u] : 0.f);
          const float vpv = (float)vp4[u] + (EXACT ? (float)vp4l[u] : 0.f);
          gdot = fmaf(dvv, vpv, gdot);
        }
      }
    dotp = wave_sum32(dotp);
    kss = wave_sum32(kss);
    gdot = wave_sum32(gdot);
    // dn <= 0: the keys arrived normalised (the Lucid_Tril_Solver seam): dK^ itself is the
    // output (r = 1, no RMSNorm backward)
    const bool knorm = dn > 0.f;
    const float f = knorm ? dotp / dn : 0.f;
    // The diagonal terms of M K^ + M^T K^ (excluded from both sums), -2 s M_ii K^_i with
    // M_ii = (dV_i . V'_i) P_ii, P_ii = exp(s |K^_i|^2 - 1/s), lie along K^_i, which the
    // RMSNorm backward keeps only to the fraction 1 - |K^_i|^2 / dn (= eps r_i^2): added here
    // as fd * K^_i rather than as two large terms that cancel down to that fraction.
    const float fd = -2.f * scale * gdot * __builtin_amdgcn_exp2f(fmaf(sl2, kss, -c0)) * (knorm ? 1.f - kss / dn : 1.f);
    auto* op = dk_out + b * dks.b + h * dks.h + (int64_t)irow * dks.t;
#pragma unroll
    for (int t = 0; t < NDT; ++t)
#pragma unroll
      for (int qq = 0; qq < 4; ++qq) {
        const int d0 = t * 32 + 8 * qq + 4 * g;
        f32x4 av = {0.f, 0.f, 0.f, 0.f};  // no attention part (preconditioner-only backward)
        if (dka) av = *reinterpret_cast<const f32x4*>(da + d0);
        f32x4 x;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int e = 4 * qq + u;
          x[u] = ri * (dkh[t][e] - khat[t][e] * f + khat[t][e] * fd) + av[u];
        }
        if constexpr (F32) {
          *reinterpret_cast<f32x4*>(op + d0) = x;
        } else {
          bf16x4 bb;
#pragma unroll
          for (int u = 0; u < 4; ++u) bb[u] = (bf16)x[u];
          *reinterpret_cast<bf16x4*>(op + d0) = bb;
        }
      }
  }
}

}  // namespace lucid
