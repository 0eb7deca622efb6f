// LUCID-Path backward on CDNA4 (gfx950) (parallel.py:78-177).
//
//   dV  = (I + L)^-T dO                       chained, last chunk first
//   dA  = -s (dV O^T) * L                     (strictly lower)
// and the path-attention backward driven by dA through the two-level transport
// (row sweep: queries carried down; column sweep: keys carried up; the d x d
// chunk products; the WY form), then the GQA reduction.
//
// Kernels (256 threads):
//   path_bwd_zero_kernel   zero chain counters and the atomic dHL / dHc accumulators
//   path_dv_kernel         chained transposed solve dV_J = Y_J^T (dO_J - sum_{I>J} L_IJ^T dV_I),
//                          plus the in-chunk dA_diag = -s (dV_J O_J^T) * L_diag
//   path_bwd_row_kernel    per query chunk: G scan over key chunks -> dq~, dHL, dHc
//   path_bwd_col_kernel    per key chunk: dk~ (same large chunk), dKL -> dk~, dSUF
//   path_products_bwd_kernel  per large chunk: dHc += SUF^T F, F <- F Hc^T + dSUF
//   path_wy_bwd_kernel     per chunk: backward of the WY form -> dq, dk, dw, dbeta
//   path_reduce_kernel     GQA sums and casts to the caller's bf16 gradients
#include "path_common.h"

namespace lucid {

// K: the kernels' head dim (64 or 128)
struct PathBwdWs {
  float* dvf;   // [BHq][T][K]        dV (fp32)
  bf16* dvb;    // [BHq][T][K]        dV rows (bf16)
  bf16* dvT;    // [BHq][K][T]        dV^T, T-perm (chain operand)
  float* dad;   // [BHq][NT][64][64]  dA_diag
  float* dqt;   // [BHq][T][K]        d q~
  float* dkt;   // [BHq][T][K]        d k~
  float* dsuf;  // [BHq][NT][K][K]    d SUF
  float* dhl;   // [BHq][NS][K][K]    d HL  (atomics)
  float* dhc;   // [BHq][NT][K][K]    d Hc  (atomics + products backward)
  float* dq;    // [BHq][T][K]
  float* dk;    // [BHq][T][K]        per query head, summed over the group at the end
  float* dw;    // [BHq][T][K]
  float* db;    // [BHq][T]
  int* counters;  // [BHq]
  float* delta; // [BHq][T]           PaTH softmax only: rowsum(dO * O)
  // fp32 inputs: element offsets of the lo planes of dvb, dvT (0 with bf16 inputs)
  int64_t lo_dvb, lo_dvT;
  // fp32 inputs: split copies (hi plane, lo plane at + lo_*) of the rows the sweeps stage
  // from the caller: xsp = dO [BHq][T][K] (PaTH softmax), ysp = O [BHq][T][K] (LUCID-Path)
  // or V [BH][T][K] (PaTH softmax)
  bf16* xsp;
  bf16* ysp;
  int64_t lo_xsp, lo_ysp;
};

// fp32 rows x [B][T][HH][K] (element strides xs: batch, head, time) -> bf16 hi and lo planes,
// contiguous [B][HH][T][K], the lo plane at dst + lo.  4 values per thread; grid
// (ceil(T K / 1024), B*HH)
__global__ __launch_bounds__(256) void path_split_kernel(const float* __restrict__ x, Strides xs, bf16* __restrict__ dst,
                                                         int64_t lo, int HH, int T, int K) {
  const int bhh = blockIdx.y, b = bhh / HH, hh = bhh - b * HH;
  const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (i >= (int64_t)T * K) return;
  const int t = (int)(i / K), c = (int)(i - (int64_t)t * K);
  const f32x4 v = *reinterpret_cast<const f32x4*>(x + b * xs.b + hh * xs.h + (int64_t)t * xs.t + c);
  bf16x4 h4, l4;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    h4[u] = (bf16)v[u];
    l4[u] = (bf16)(v[u] - (float)h4[u]);
  }
  bf16* d = dst + (int64_t)bhh * T * K + i;
  *reinterpret_cast<bf16x4*>(d) = h4;
  *reinterpret_cast<bf16x4*>(d + lo) = l4;
}

__global__ __launch_bounds__(256) void path_bwd_zero_kernel(int64_t n_hl, int64_t n_hc, int n_cnt, PathBwdWs bw) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * 256;
  for (int64_t j = i; j < n_hl; j += stride) bw.dhl[j] = 0.f;
  for (int64_t j = i; j < n_hc; j += stride) bw.dhc[j] = 0.f;
  if (i < n_cnt) bw.counters[i] = 0;
}

// ---------------------------------------------------------------------------
// Chained transposed solve (triangular_solve_bwd_dv_reuse.py:113-205), one
// workgroup per pair of 64-column chunks A = 2q, B = 2q + 1 (one large chunk holds
// both) of one query head; ids grow as q falls, so every wait is on a lower id.
// counters[bhq] = number of chunks of dV published from the end (B, then A).
// wave w owns columns 32w .. +32 of the pair (chunk A for w < 2, lane <-> column j)
// and all 64 rows of every later row tile I > B, so its sums need no cross-wave
// reduction:
//   S[I][J] = Qop_I . Kop_J, L = exp(s S - 1/s), acc^T[d][j] += dV^T[d][i] L[i][j]
// Row tiles beyond the large chunk share one query operand (QB) for both chunks and
// are swept in pairs, one barrier and one staging round per pair; the (at most PR - 2)
// row tiles inside the large chunk need a query slot per column chunk (QS) and are
// swept one per step with both slots staged.  Then dV_B = Y_B^T R_B (published),
// R_A -= L_BA^T dV_B, dV_A = Y_A^T R_A (published), R = dO - acc, and
// dA_diag = -s (dV_J O_J^T) * L_diag for both chunks on the matrix cores.  L_BA
// depends on the operands only and is computed before the sweep; the fp32 buffers
// of the final step reuse the staging space.
// ---------------------------------------------------------------------------
template <int KD, int NP>
struct DvSmem {
  union {
    struct {
      // [buffer][tile of the pair, or column chunk][plane], swizzled (chunk c of row r at c ^ (r & 7))
      bf16 q[2][2][NP][64 * KD];
      bf16 d[2][2][NP][KD * 64];
    } st;
    struct {
      float Rt[KD][132];    // R^T for the 128 columns (0..63 = A), then dV rows of one chunk
      float Yt[64][68];     // Yt[c][r] = Y[r][c] of the chunk being solved, then O rows
      bf16 dt[NP][KD][128 + 8];  // dV^T of both chunks, T-perm within 16-groups
    } fin;
  } u;
  bf16x8 lba[4][64][2 * NP];  // L_BA as MFMA B operands, per wave and lane ([2 + h]: lo)
};

// KD: head dim (64 or 128); at 128 a wave owns value tiles w >> 1 and (w >> 1) + 2 of the
// final solve, and dA_diag is summed over the two 64-column halves of dV and O
// F32: fp32 dO and O; every operand product is a 3-term split over hi / lo planes (mm3)
template <int KD, bool F32>
__global__ __launch_bounds__(256) LUCID_TWO_WAVES_IF(KD == 64 && !F32) void path_dv_kernel(
    const pin_t<F32>* __restrict__ dout, Strides dos, const pin_t<F32>* __restrict__ o, Strides os, int HQ, int H,
    int T, int BHq, float scale, PathFwdWs ws, PathBwdWs bw) {
  constexpr int NKS = KD / 16, NVT = KD / 32;  // k-steps of a logit product, 32-column value tiles
  constexpr int NP = F32 ? 2 : 1;
  __shared__ __attribute__((aligned(16))) DvSmem<KD, NP> sm;
  const int NT = T / PC, NS = (NT + PR - 1) / PR, NQ = (NT + 1) / 2;
  const int id = blockIdx.x;
  const int q = NQ - 1 - id / BHq, bhq = id - (id / BHq) * BHq;
  const int G = HQ / H;
  const int b = bhq / HQ, hq = bhq - b * HQ, bh = b * H + hq / G;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 5, l32 = lane & 31;
  const int A = 2 * q;
  const bool hasB = A + 1 < NT;
  const int last = hasB ? A + 1 : A;                     // last chunk of the workgroup
  const int sJ = A / PR, cb = sJ * PR, ceJ = min(cb + PR, NT) - 1;  // the large chunk holding A and B
  const int j0 = A * PC;
  const int wc = w >> 1;                                 // this wave's column chunk (0 = A, 1 = B)
  const bool mycols = wc == 0 || hasB;
  const int jc = j0 + (mycols ? w * 32 : (w & 1) * 32) + l32;  // this lane's column (a missing B reuses A's)
  int* cnt = bw.counters + bhq;
  const float sl2 = scale * LOG2E_F, cc0 = LOG2E_F / scale;

  bf16x8 kbs[NKS][NP], kbf[NKS][NP];
#pragma unroll
  for (int st = 0; st < NKS; ++st) {
    const bf16* ps = ws.kt + ((int64_t)bh * T + jc) * KD + 16 * st + 8 * g;
    const bf16* pf = ws.kl + ((int64_t)bh * T + jc) * KD + 16 * st + 8 * g;
    kbs[st][0] = ld8(ps);
    kbf[st][0] = ld8(pf);
    if constexpr (F32) {
      kbs[st][1] = ld8(ps + ws.lo_kt);
      kbf[st][1] = ld8(pf + ws.lo_kl);
    }
  }
  // accumulators start at -dO^T (R = dO - acc = -acc)
  f32x16 acc[NVT];
  {
    const pin_t<F32>* drow_ = dout + b * dos.b + hq * dos.h + (int64_t)jc * dos.t;
#pragma unroll
    for (int t = 0; t < NVT; ++t)
#pragma unroll
      for (int qq = 0; qq < 4; ++qq) {
        if constexpr (F32) {
          const f32x4 x = *reinterpret_cast<const f32x4*>(drow_ + t * 32 + 8 * qq + 4 * g);
#pragma unroll
          for (int u = 0; u < 4; ++u) acc[t][4 * qq + u] = -x[u];
        } else {
          const bf16x4 x = *reinterpret_cast<const bf16x4*>(drow_ + t * 32 + 8 * qq + 4 * g);
#pragma unroll
          for (int u = 0; u < 4; ++u) acc[t][4 * qq + u] = -(float)x[u];
        }
      }
  }
  // QS slot of column chunk c (relative to the large chunk) for row chunk I inside it
  auto qs_slot = [&](int c) { return ws.qs + ((int64_t)bhq * PR + (A + c - cb)) * T * KD; };
  // L_BA (rows of B half kb, columns of A half na): Qop = QS slot A - cb of B's rows, Kop_A = k~_A
  if (hasB) {
    const int na = w & 1, kb = w >> 1;
    const bf16* qr = qs_slot(0) + (int64_t)((A + 1) * PC + kb * 32 + l32) * KD;
    const bf16* kr = ws.kt + ((int64_t)bh * T + j0 + na * 32 + l32) * KD;
    f32x16 sc = zero16();
#pragma unroll
    for (int st = 0; st < NKS; ++st) {
      bf16x8 qa8[NP], ka8[NP];
      qa8[0] = ld8(qr + 16 * st + 8 * g);
      ka8[0] = ld8(kr + 16 * st + 8 * g);
      if constexpr (F32) {
        qa8[1] = ld8(qr + ws.lo_qs + 16 * st + 8 * g);
        ka8[1] = ld8(kr + ws.lo_kt + 16 * st + 8 * g);
      }
      sc = mm3<NP>(qa8, ka8, sc);
    }
#pragma unroll
    for (int e = 0; e < 16; ++e) sc[e] = __builtin_amdgcn_exp2f(fmaf(sc[e], sl2, -cc0));
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      sm.lba[w][lane][hh] = pack_b(sc, hh);
      if constexpr (F32) sm.lba[w][lane][2 + hh] = pack_lo(sc, hh, sm.lba[w][lane][hh]);
    }
  }
  // row tile k (k = 0 .. n-1) is chunk I = NT-1-k, published once the counter exceeds k.
  // Tiles k < nfar lie beyond the large chunk (swept in pairs); the rest one per step.
  const int n = NT - 1 - last, nfar = min(n, NT - 1 - ceJ);
  const int nfs = (nfar + 1) / 2, nsteps = nfs + (n - nfar);
  auto first_tile = [&](int s) { return s < nfs ? 2 * s : nfar + (s - nfs); };
  auto need = [&](int s) { return s < nfs ? min(2 * s + 1, nfar - 1) : first_tile(s); };
  int plan_q[64 * (KD / 8) / 256], plan_t[KD * 8 / 256];
  dma_plan<64, KD / 8>(KD, plan_q);
  dma_plan<KD, 8>(T, plan_t);
  auto stage = [&](int s) {
    const int buf = s & 1, k0 = first_tile(s);
    if (s < nfs) {
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int k = k0 + u;
        if (k < nfar) {
          const int I = NT - 1 - k;
#pragma unroll
          for (int pl = 0; pl < NP; ++pl) {
            dma_stage<64, KD / 8>(plan_q, ws.qb + pl * ws.lo_qb + (((int64_t)bhq * NS + sJ) * T + (int64_t)I * PC) * KD,
                                  sm.u.st.q[buf][u][pl]);
            dma_stage<KD, 8>(plan_t, bw.dvT + pl * bw.lo_dvT + (int64_t)bhq * KD * T + I * PC, sm.u.st.d[buf][u][pl]);
          }
        }
      }
    } else {
      const int I = NT - 1 - k0;
#pragma unroll
      for (int pl = 0; pl < NP; ++pl) {
#pragma unroll
        for (int c = 0; c < 2; ++c)
          if (c == 0 || hasB)
            dma_stage<64, KD / 8>(plan_q, qs_slot(c) + pl * ws.lo_qs + (int64_t)I * PC * KD, sm.u.st.q[buf][c][pl]);
        dma_stage<KD, 8>(plan_t, bw.dvT + pl * bw.lo_dvT + (int64_t)bhq * KD * T + I * PC, sm.u.st.d[buf][0][pl]);
      }
    }
  };
  // Y_A, Y_B (fp32) are fetched into registers during the last step
  f32x4 yr[8];
  auto yload = [&]() {
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int c = u >> 2;
      if (c == 0 || hasB)
        yr[u] = *reinterpret_cast<const f32x4*>(ws.y + ((int64_t)bhq * NT + A + c) * 4096 + 4 * (tid + 256 * (u & 3)));
    }
  };
  auto ystore_t = [&](int c) {
#pragma unroll
    for (int u = 4 * c; u < 4 * c + 4; ++u) {
      const int f = 4 * (tid + 256 * (u & 3)), r = f >> 6, c4 = f & 63;
#pragma unroll
      for (int e = 0; e < 4; ++e) sm.u.fin.Yt[c4 + e][r] = yr[u][e];
    }
  };
  // one staged 64-row tile (planes qt[pl], dtl[pl]) against this wave's 32 columns
  auto tile = [&](bf16* const* qt, bf16* const* dtl, bool same) {
#pragma unroll
    for (int rh = 0; rh < 2; ++rh) {
      f32x16 sc = zero16();
#pragma unroll
      for (int st = 0; st < NKS; ++st) {
        bf16x8 qa[NP];
#pragma unroll
        for (int pl = 0; pl < NP; ++pl) qa[pl] = ld8(swz<KD / 8>(qt[pl], rh * 32 + l32, 2 * st + g));
        sc = mm3<NP>(qa, same ? kbs[st] : kbf[st], sc);
      }
#pragma unroll
      for (int e = 0; e < 16; ++e) sc[e] = __builtin_amdgcn_exp2f(fmaf(sc[e], sl2, -cc0));
      bf16x8 p[2][NP];
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        p[hh][0] = pack_b(sc, hh);
        if constexpr (F32) p[hh][1] = pack_lo(sc, hh, p[hh][0]);
      }
#pragma unroll
      for (int t = 0; t < NVT; ++t)
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          bf16x8 da[NP];
#pragma unroll
          for (int pl = 0; pl < NP; ++pl) da[pl] = ld8(swz<8>(dtl[pl], t * 32 + l32, 4 * rh + 2 * hh + g));
          acc[t] = mm3<NP>(da, p[hh], acc[t]);
        }
    }
  };
  int ready = 0;
  if (nsteps > 0) {
    ready = wait_counter_gt(cnt, need(0));
    stage(0);
    dma_wait();
  } else {
    yload();
  }
  __syncthreads();
  for (int s = 0; s < nsteps; ++s) {
    const int buf = s & 1;
    const bool more = s + 1 < nsteps;
    bool early = false;
    if (more) {
      const int nd = need(s + 1);
      if (nd >= ready) {
        const int seen = poll_counter(cnt);
        if (seen > nd) {
          chain_acquire();
          ready = seen;
        }
      }
      early = nd < ready;
      if (early) stage(s + 1);
    } else {
      yload();
    }
    auto planes = [&](bf16 (*x)[KD * 64], bf16** out) {
#pragma unroll
      for (int pl = 0; pl < NP; ++pl) out[pl] = x[pl];
    };
    bf16* qp_[NP];
    bf16* dp_[NP];
    if (s < nfs) {
      planes(sm.u.st.q[buf][0], qp_);
      planes(sm.u.st.d[buf][0], dp_);
      tile(qp_, dp_, false);
      if (2 * s + 1 < nfar) {
        planes(sm.u.st.q[buf][1], qp_);
        planes(sm.u.st.d[buf][1], dp_);
        tile(qp_, dp_, false);
      }
    } else {
      planes(sm.u.st.q[buf][mycols ? wc : 0], qp_);
      planes(sm.u.st.d[buf][0], dp_);
      tile(qp_, dp_, true);
    }
    if (more && !early) {
      ready = wait_counter_gt(cnt, need(s + 1));
      stage(s + 1);
    }
    dma_wait();
    __syncthreads();
  }
  // ---- R^T = -acc (Rt columns = columns of the workgroup); Y_B^T to LDS ----
  float(*Rt)[132] = sm.u.fin.Rt;
  float(*Yt)[68] = sm.u.fin.Yt;
  if (mycols) {
#pragma unroll
    for (int t = 0; t < NVT; ++t)
#pragma unroll
      for (int e = 0; e < 16; ++e) Rt[t * 32 + drow(e, g)][w * 32 + l32] = -acc[t][e];
  }
  ystore_t(hasB ? 1 : 0);
  __syncthreads();
  // dV^T[d][c] = sum_r R^T[d][r] Y[r][c] for chunk cc (Y lower: r >= c); wave -> (d tiles
  // dt0 + 2 i, column half); returns the wave's tiles in D layout
  const int dt0 = w >> 1, chh = w & 1;
  auto diag_solve = [&](int cc, f32x16* dvs) {
#pragma unroll
   for (int i = 0; i < NVT / 2; ++i) {
    const int dt = dt0 + 2 * i;
    f32x16 dvo = zero16();
    for (int st = chh ? 2 : 0; st < 4; ++st) {
      bf16x8 ah, al, bh8, bl;
      split8(&Rt[dt * 32 + l32][cc * 64 + 16 * st + 8 * g], ah, al);
      split8(&Yt[chh * 32 + l32][16 * st + 8 * g], bh8, bl);
      dvo = mfma32(ah, bh8, dvo);
      dvo = mfma32(ah, bl, dvo);
      dvo = mfma32(al, bh8, dvo);
    }
    const int cl = chh * 32 + l32;
    const int r = j0 + cc * 64 + cl;
    const int lslot = cc * 64 + ((cl & ~15) | jmap(cl & 15));
    float* of = bw.dvf + ((int64_t)bhq * T + r) * KD;
    bf16* ob = bw.dvb + ((int64_t)bhq * T + r) * KD;
#pragma unroll
    for (int qq = 0; qq < 4; ++qq) {
      const int d0 = dt * 32 + 8 * qq + 4 * g;
      f32x4 f;
      bf16x4 bb, bl;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        f[u] = dvo[4 * qq + u];
        bb[u] = (bf16)f[u];
        sm.u.fin.dt[0][d0 + u][lslot] = bb[u];
        if constexpr (F32) {
          bl[u] = (bf16)(f[u] - (float)bb[u]);
          sm.u.fin.dt[NP - 1][d0 + u][lslot] = bl[u];
        }
      }
      *reinterpret_cast<f32x4*>(of + d0) = f;
      *reinterpret_cast<bf16x4*>(ob + d0) = bb;
      if constexpr (F32) *reinterpret_cast<bf16x4*>(ob + bw.lo_dvb + d0) = bl;
    }
    dvs[i] = dvo;
   }
  };
  // dV^T of chunk cc to the chain operand with 16-byte stores, then publish it
  auto publish_chunk = [&](int cc) {
    __syncthreads();
    for (int c = tid; c < KD * 8; c += 256) {
      const int dd = c >> 3, s8 = (c & 7) * 8;
      bf16* dst = bw.dvT + ((int64_t)bhq * KD + dd) * T + j0 + cc * 64 + s8;
      *reinterpret_cast<bf16x8*>(dst) = ld8(&sm.u.fin.dt[0][dd][cc * 64 + s8]);
      if constexpr (F32) *reinterpret_cast<bf16x8*>(dst + bw.lo_dvT) = ld8(&sm.u.fin.dt[NP - 1][dd][cc * 64 + s8]);
    }
    publish_counter(cnt, NT - (A + cc));
  };
  f32x16 dvoB[NVT / 2], dvoA[NVT / 2];
  if (hasB) {
    diag_solve(1, dvoB);
    publish_chunk(1);
    // ---- R_A -= L_BA^T dV_B: wave -> (A columns half na, B rows half kb); Y_A^T to LDS ----
    const int na = w & 1, kb = w >> 1;
    bf16x8 lb[2][NP];
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      lb[hh][0] = sm.lba[w][lane][hh];
      if constexpr (F32) lb[hh][1] = sm.lba[w][lane][2 + hh];
    }
    f32x16 cr[NVT];
#pragma unroll
    for (int t = 0; t < NVT; ++t) {
      cr[t] = zero16();
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        bf16x8 da[NP];
#pragma unroll
        for (int pl = 0; pl < NP; ++pl) da[pl] = ld8(&sm.u.fin.dt[pl][t * 32 + l32][64 + kb * 32 + 16 * hh + 8 * g]);
        cr[t] = mm3<NP>(da, lb[hh], cr[t]);
      }
    }
    const int col = na * 32 + l32;
    if (kb == 1) {
#pragma unroll
      for (int t = 0; t < NVT; ++t)
#pragma unroll
        for (int e = 0; e < 16; ++e) Rt[t * 32 + drow(e, g)][col] -= cr[t][e];
    }
    ystore_t(0);
    __syncthreads();
    if (kb == 0) {
#pragma unroll
      for (int t = 0; t < NVT; ++t)
#pragma unroll
        for (int e = 0; e < 16; ++e) Rt[t * 32 + drow(e, g)][col] -= cr[t][e];
    }
    __syncthreads();
  }
  diag_solve(0, dvoA);
  publish_chunk(0);
  // ---- dA_diag = -s (dV_J O_J^T) * L_diag per chunk (every read of Rt / Yt came before the last
  // barrier), summed over the 64-column halves of dV and O ----
  float(*Dr)[68] = reinterpret_cast<float(*)[68]>(&sm.u.fin.Rt[0][0]);  // dV rows of the chunk
  for (int cc = 0; cc < (hasB ? 2 : 1); ++cc) {
    f32x16 a = zero16();
#pragma unroll
    for (int i = 0; i < NVT / 2; ++i) {
      const f32x16 dvo = cc ? dvoB[i] : dvoA[i];
#pragma unroll
      for (int e = 0; e < 16; ++e) Dr[chh * 32 + l32][dt0 * 32 + drow(e, g)] = dvo[e];
      load_rows64_f32(Yt, o + b * os.b + hq * os.h + (int64_t)(j0 + cc * 64) * os.t + 64 * i, os.t);  // O rows
      __syncthreads();
      a = mgemm64<false, true>(Dr, Yt, a);
      if (i + 1 < NVT / 2) __syncthreads();
    }
    const float* ldp = ws.ld + ((int64_t)bhq * NT + A + cc) * 4096;
    float* dst = bw.dad + ((int64_t)bhq * NT + A + cc) * 4096;
    const int cl = dl_col();
    DL_FOR_E {
      const int rr = dl_row(e);
      dst[rr * 64 + cl] = -scale * a[e] * ldp[rr * 64 + cl];
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// Row sweep (parallel_path_bwd_inter_dqh.py, parallel_path_bwd_intra.py): per pair
// of query chunks I1 = 2*blockIdx.x, I2 = I1 + 1 (one large chunk), key chunks J
// ascending.  G accumulates d(query operand):
//   G^T[d][i] += Kop^T[d][j] dA^T[j][i]
// and at every change of query operand X (large-chunk boundary: X = QB^(s), M = HL_s;
// inside the large chunk: X = QS^(c), M = Hc_c):  dM += X^T G,  G <- G M^T
// (X^T from transposing LDS reads of the staged X rows).
// Finally d q~ = G.  Wave w owns rows 32w..32w+31 of the pair (chunk I1 + w/2,
// lane <-> row i) and all 64 keys of every key tile; key-operand and O rows are
// staged by direct global->LDS loads (double buffered), Kop^T comes through
// transposing LDS reads.  The pair's dM contributions are summed over its 128 rows
// before the atomic adds.  grid (B*HQ, ceil(NT/2)), late (long) pairs first
// The dA rule is the template argument: LUCID-Path (SM = false) dA = -s (X_I Y_J^T) L
// with X = dV, Y = O (rows of the same query head); PaTH softmax (SM = true)
// dA = s P (X_I Y_J^T - delta_i), P = exp2(s' S - lse_i), X = dO, Y = V (kv head).
// ---------------------------------------------------------------------------
template <int KD, int NP>
struct RowSmem {
  bf16 k[2][NP][64 * KD];  // [buffer][plane], swizzled (chunk c of row r at c ^ (r & 7))
  bf16 o[2][NP][64 * KD];
  // G rows of the pair at a transport step as bf16 hi and lo planes, swizzled (chunk c of
  // row r at c ^ (r & 7)): split once when stored, read directly by both transition products
  bf16 gs[2][128 * KD];
};

// KD: head dim (64 or 128); the KD x KD transport matrices and their gradients are row-major.
// F32: X and Y rows are bf16 hi planes with their lo planes at xsrc + x_lo, ysrc + y_lo, and
// every operand product is a 3-term split (mm3)
template <bool SM, int KD, bool F32>
__global__ __launch_bounds__(256) LUCID_TWO_WAVES_IF(KD == 64 && !F32) void path_bwd_row_kernel(
    const bf16* __restrict__ xsrc, Strides xs, int64_t x_lo, const bf16* __restrict__ ysrc, Strides ys, int64_t y_lo,
    int HQ, int H, int T, float scale, PathFwdWs ws, PathBwdWs bw) {
  constexpr int NKS = KD / 16, NVT = KD / 32, CPR = KD / 8;  // k-steps, 32-column tiles, 16-byte chunks per row
  constexpr int NP = F32 ? 2 : 1;
  __shared__ __attribute__((aligned(16))) RowSmem<KD, NP> sm;
  const int NT = T / PC, NS = (NT + PR - 1) / PR;
  const int I1 = 2 * ((int)gridDim.y - 1 - (int)blockIdx.y), bhq = blockIdx.x;  // heaviest pairs of all heads first
  const int G_ = HQ / H;
  const int b = bhq / HQ, hq = bhq - b * HQ, bh = b * H + hq / G_;
  const bf16* yh = ysrc + b * ys.b + (SM ? hq / G_ : hq) * ys.h;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 5, l32 = lane & 31;
  const int Iw = I1 + (w >> 1);                     // this wave's query chunk
  const bool pair = I1 + 1 < NT;                    // NT odd: the last pair has one chunk
  const int sI = I1 / PR, cb = sI * PR;
  const int iw0 = min(Iw, NT - 1) * PC + (w & 1) * 32;  // first row of this wave
  const int nJ = pair ? I1 + 1 : I1;                // key tiles needed by the pair
  const float sl2 = scale * LOG2E_F, cc0 = LOG2E_F / scale;

  bf16x8 dvr[NKS][NP];
  {
    const bf16* xrow = xsrc + b * xs.b + hq * xs.h + (int64_t)(iw0 + l32) * xs.t;
#pragma unroll
    for (int st = 0; st < NKS; ++st) {
      dvr[st][0] = ld8(xrow + 16 * st + 8 * g);
      if constexpr (F32) dvr[st][1] = ld8(xrow + x_lo + 16 * st + 8 * g);
    }
  }
  // exponent offset and delta of this lane's row (LUCID-Path: the constant 1/s, no delta)
  const float ci = SM ? ws.lse[(int64_t)bhq * T + iw0 + l32] : cc0;
  const float di = SM ? bw.delta[(int64_t)bhq * T + iw0 + l32] : 0.f;
  // dA = F dP exp2(sl2 S) (LUCID-Path, F = -s 2^-cc0) or F P (dP - delta) (PaTH softmax,
  // F = s): the constant F is carried out of the sweep by G (applied to dM and to d q~)
  const float F = SM ? scale : -scale * __builtin_amdgcn_exp2f(-cc0);
  f32x16 acc[NVT];
#pragma unroll
  for (int t = 0; t < NVT; ++t) acc[t] = zero16();

  int plan_k[64 * CPR / 256], plan_o[64 * CPR / 256];
  dma_plan<64, CPR>(KD, plan_k);
  dma_plan<64, CPR>(ys.t, plan_o);
  // ---- dM += X^T G over the pair's rows (atomic) and G <- G M^T for each wave's rows ----
  // X (rows of the query operand, row-major) is staged into the idle half of the double
  // buffer (tile J+1 is staged only after the transition); X^T comes from transposing reads
  bf16x8 qb[NKS][NP];  // this wave's rows of the current query operand (MFMA B operands)
  // the query operand of key tile J (QB^(J/PR) below the large chunk, QS slot J - cb inside
  // it), and whether a transport step precedes tile J (the operand differs from tile J - 1's)
  auto opnd = [&](int J) {
    return (J < cb) ? ws.qb + ((int64_t)bhq * NS + J / PR) * T * KD : ws.qs + ((int64_t)bhq * PR + (J - cb)) * T * KD;
  };
  auto opnd_lo = [&](int J) { return (J < cb) ? ws.lo_qb : ws.lo_qs; };
  auto trans_at = [&](int J) { return (J < cb) ? (J % PR == 0 && J > 0) : (sI > 0 || J > cb); };
  // KD = 64: a transition's X rows (the new operand's rows of chunks I1, I1 + 1) are fetched
  // into registers one key tile ahead, so that no transition waits for them; at KD = 128 they
  // are staged by direct loads in the transition (registers)
  constexpr bool XPRE = KD == 64;
  constexpr int XPT = XPRE ? 2 * 64 * CPR / 256 : 1;  // 16-byte chunks per thread and plane
  bf16x8 xr[NP][XPT];
  auto xprefetch = [&](int J) {
    const bf16* X = opnd(J) + (int64_t)I1 * PC * KD;
    const int64_t xlo = opnd_lo(J);
#pragma unroll
    for (int u = 0; u < XPT; ++u) {
      const int idx = tid + 256 * u, r = idx / CPR, c = idx - (idx / CPR) * CPR;
      if (r < 64 || pair) {
#pragma unroll
        for (int pl = 0; pl < NP; ++pl) xr[pl][u] = ld8(X + pl * xlo + (int64_t)r * KD + 8 * c);
      }
    }
  };
  // Ms: M as bf16 hi and lo planes (the lo plane KD * KD elements after the hi plane)
  auto transition = [&](int J, const bf16* Ms, float* dM) {
    const bool act = Iw < NT && J < Iw;
    // the M rows of this wave's G M^T (KD = 64; hi, lo), loaded before the barrier so that
    // their latency overlaps the dM products
    bf16x8 mv[XPRE ? NVT : 1][XPRE ? NKS : 1][2];
    if constexpr (XPRE) {
      if (act) {
#pragma unroll
        for (int bt = 0; bt < NVT; ++bt)
#pragma unroll
          for (int ks = 0; ks < NKS; ++ks)
#pragma unroll
            for (int hh = 0; hh < 2; ++hh)
              mv[bt][ks][hh] = ld8(Ms + hh * (KD * KD) + (bt * 32 + l32) * KD + 16 * ks + 8 * g);
      }
      // planes of the X rows of chunk I1 (in k) and I1 + 1 (in o), swizzled as the direct loads
#pragma unroll
      for (int u = 0; u < XPT; ++u) {
        const int idx = tid + 256 * u, r = idx / CPR, c = idx - (idx / CPR) * CPR, rr = r & 63;
        if (r < 64 || pair) {
#pragma unroll
          for (int pl = 0; pl < NP; ++pl)
            *reinterpret_cast<bf16x8*>((r < 64 ? sm.k[(J + 1) & 1][pl] : sm.o[(J + 1) & 1][pl]) + swz_off<CPR>(rr, c)) =
                xr[pl][u];
        }
      }
    } else {
      const bf16* X = opnd(J);
      const int64_t xlo = opnd_lo(J);
#pragma unroll
      for (int pl = 0; pl < NP; ++pl) {
        dma_stage<64, CPR>(plan_k, X + pl * xlo + (int64_t)I1 * PC * KD, sm.k[(J + 1) & 1][pl]);
        if (pair) dma_stage<64, CPR>(plan_k, X + pl * xlo + (int64_t)(I1 + 1) * PC * KD, sm.o[(J + 1) & 1][pl]);
      }
    }
#pragma unroll
    for (int t = 0; t < NVT; ++t)
#pragma unroll
      for (int qd = 0; qd < 4; ++qd) {  // elements 4 qd .. 4 qd + 3: columns t*32 + 8 qd + 4 g + u
        bf16x4 hi, lo;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const float x = act ? acc[t][4 * qd + u] : 0.f;
          hi[u] = (bf16)x;
          lo[u] = (bf16)(x - (float)hi[u]);
        }
        const int off = swz_off<CPR>(32 * w + l32, 4 * t + qd) + 4 * g;
        *reinterpret_cast<bf16x4*>(sm.gs[0] + off) = hi;
        *reinterpret_cast<bf16x4*>(sm.gs[1] + off) = lo;
      }
    if constexpr (!XPRE) dma_wait();
    __syncthreads();
#pragma unroll 1
    for (int tt = w; tt < NVT * NVT; tt += 4) {
      const int at = tt / NVT, bt = tt % NVT;  // dM tile (a rows, b cols)
      f32x16 dm = zero16();
      // rows of a chunk that has left the sweep are skipped: its X rows may be undefined
      const int ks0 = (J < I1) ? 0 : 4, ks1 = (pair && J < I1 + 1) ? 8 : 4;
      for (int ks = ks0; ks < ks1; ++ks) {
        const bf16x8 xa = lds_tr_a<CPR>(ks < 4 ? sm.k[(J + 1) & 1][0] : sm.o[(J + 1) & 1][0], 16 * (ks & 3), at * 32);
        // G rows 16 ks + jmap(slot), column bt * 32 + lane: the transposing read's slot order
        const bf16x8 gh = lds_tr_a<CPR>(sm.gs[0], 16 * ks, bt * 32);
        const bf16x8 gl = lds_tr_a<CPR>(sm.gs[1], 16 * ks, bt * 32);
        dm = mfma32(xa, gh, dm);
        dm = mfma32(xa, gl, dm);
        if constexpr (F32)
          dm = mfma32(lds_tr_a<CPR>(ks < 4 ? sm.k[(J + 1) & 1][1] : sm.o[(J + 1) & 1][1], 16 * (ks & 3), at * 32), gh,
                      dm);
      }
#pragma unroll
      for (int e = 0; e < 16; ++e) unsafeAtomicAdd(dM + (at * 32 + drow(e, g)) * KD + bt * 32 + l32, F * dm[e]);
    }
    if (act) {
#pragma unroll
      for (int bt = 0; bt < NVT; ++bt) {
        f32x16 gn = zero16();
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) {
          bf16x8 ah, al;
          if constexpr (XPRE) {
            ah = mv[bt][ks][0];
            al = mv[bt][ks][1];
          } else {
            ah = ld8(Ms + (bt * 32 + l32) * KD + 16 * ks + 8 * g);
            al = ld8(Ms + KD * KD + (bt * 32 + l32) * KD + 16 * ks + 8 * g);
          }
          const bf16x8 bh8 = ld8(swz<CPR>(sm.gs[0], 32 * w + l32, 2 * ks + g));
          const bf16x8 bl = ld8(swz<CPR>(sm.gs[1], 32 * w + l32, 2 * ks + g));
          gn = mfma32(ah, bh8, gn);
          gn = mfma32(ah, bl, gn);
          gn = mfma32(al, bh8, gn);
        }
        acc[bt] = gn;
      }
    }
    // this wave's rows of the new operand (the sweep's query registers), from the staged X
    {
#pragma unroll
      for (int st = 0; st < NKS; ++st)
#pragma unroll
        for (int pl = 0; pl < NP; ++pl)
          qb[st][pl] = ld8(swz<CPR>((pair && (w >> 1)) ? sm.o[(J + 1) & 1][pl] : sm.k[(J + 1) & 1][pl],
                                    (w & 1) * 32 + l32, 2 * st + g));
    }
    __syncthreads();
  };

  auto stage = [&](int J) {
    const int buf = J & 1;
    const bf16* kr = ((J < cb) ? ws.kl : ws.kt) + ((int64_t)bh * T + J * PC) * KD;
    const int64_t klo = (J < cb) ? ws.lo_kl : ws.lo_kt;
#pragma unroll
    for (int pl = 0; pl < NP; ++pl) {
      dma_stage<64, CPR>(plan_k, kr + pl * klo, sm.k[buf][pl]);
      dma_stage<64, CPR>(plan_o, yh + pl * y_lo + (int64_t)J * PC * ys.t, sm.o[buf][pl]);
    }
  };
  if (nJ > 0) stage(0);
  dma_wait();
  __syncthreads();
  for (int J = 0; J < nJ; ++J) {
    const int buf = J & 1;
    // transport step before the first tile that uses a new query operand (it also loads the
    // new operand's rows into qb)
    const bool tr = trans_at(J);
    if (tr) {
      if (J < cb) {
        const int s = J / PR;
        transition(J, ws.hls + ((int64_t)bh * NS + s) * (2 * KD * KD), bw.dhl + ((int64_t)bhq * NS + s) * (KD * KD));
      } else {
        transition(J, ws.hcs + ((int64_t)bh * NT + J) * (2 * KD * KD), bw.dhc + ((int64_t)bhq * NT + J) * (KD * KD));
      }
    }
    if (J + 1 < nJ) stage(J + 1);
    if (!tr && (J >= cb || J % PR == 0)) {  // the query operand changes without a transport step (J = 0)
      const bf16* qsrc = opnd(J);
      const int64_t qlo = opnd_lo(J);
#pragma unroll
      for (int st = 0; st < NKS; ++st) {
        qb[st][0] = ld8(qsrc + (int64_t)(iw0 + l32) * KD + 16 * st + 8 * g);
        if constexpr (F32) qb[st][1] = ld8(qsrc + qlo + (int64_t)(iw0 + l32) * KD + 16 * st + 8 * g);
      }
    }
    if constexpr (XPRE) {
      if (J + 1 < nJ && trans_at(J + 1)) xprefetch(J + 1);  // in flight during this tile's sweep
    }
    if (Iw < NT && J < Iw) {
#pragma unroll
      for (int jh = 0; jh < 2; ++jh) {
        f32x16 sc = zero16(), dp = zero16();
#pragma unroll
        for (int st = 0; st < NKS; ++st) {
          bf16x8 ka[NP], oa[NP];
#pragma unroll
          for (int pl = 0; pl < NP; ++pl) {
            ka[pl] = ld8(swz<CPR>(sm.k[buf][pl], jh * 32 + l32, 2 * st + g));
            oa[pl] = ld8(swz<CPR>(sm.o[buf][pl], jh * 32 + l32, 2 * st + g));
          }
          sc = mm3<NP>(ka, qb[st], sc);
          dp = mm3<NP>(oa, dvr[st], dp);
        }
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const float ex = __builtin_amdgcn_exp2f(SM ? fmaf(sc[e], sl2, -ci) : sc[e] * sl2);
          sc[e] = SM ? ex * (dp[e] - di) : dp[e] * ex;
        }
        bf16x8 dd[2][NP];
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          dd[hh][0] = pack_b(sc, hh);
          if constexpr (F32) dd[hh][1] = pack_lo(sc, hh, dd[hh][0]);
        }
#pragma unroll
        for (int t = 0; t < NVT; ++t)
#pragma unroll
          for (int hh = 0; hh < 2; ++hh) {
            bf16x8 ka[NP];
#pragma unroll
            for (int pl = 0; pl < NP; ++pl) ka[pl] = lds_tr_a<CPR>(sm.k[buf][pl], jh * 32 + 16 * hh, t * 32);
            acc[t] = mm3<NP>(ka, dd[hh], acc[t]);
          }
      }
    }
    dma_wait();
    __syncthreads();
  }
  if (Iw < NT) {
    float* dst = bw.dqt + ((int64_t)bhq * T + iw0 + l32) * KD;
#pragma unroll
    for (int t = 0; t < NVT; ++t)
#pragma unroll
      for (int qq = 0; qq < 4; ++qq) {
        f32x4 v;
#pragma unroll
        for (int u = 0; u < 4; ++u) v[u] = F * acc[t][4 * qq + u];
        *reinterpret_cast<f32x4*>(dst + t * 32 + 8 * qq + 4 * g) = v;
      }
  }
}

// ---------------------------------------------------------------------------
// Column sweep (parallel_path_bwd_inter_dkv.py, parallel_path_bwd_intra.py): per
// pair of key chunks J1 = 2*blockIdx.x, J2 = J1 + 1 (one large chunk), query chunks
// I > J.  Wave w owns keys 32w .. 32w+31 of the pair (chunk Jw = J1 + w/2, lane <->
// key j) and sweeps all 64 rows of every query tile, so its accumulators need no
// cross-wave reduction.
//   S[i][j] = Qop_I . Kop_J, dP[i][j] = dV_I . O_J, dA = -s dP * exp(s S - 1/s)
//   dKop^T[d][j] += Qop^T[d][i] dA[i][j]   (Kop = k~_J for I in J's large chunk, else KL_J)
// Query tiles (the shared QB^(s) rows for later large chunks, or QS^(J1), QS^(J2)
// rows inside the large chunk) and dV rows are staged by direct global->LDS loads
// (three buffers, two tiles ahead); Qop^T comes through transposing LDS reads.
// Then d k~_J = dk~(same) + dKL SUF_J and dSUF_J = dKL^T k~_J.  grid (B*HQ, ceil(NT/2)),
// early (long) pairs first
// Template argument SM as in the row sweep; in PaTH softmax mode the rows' lse and
// delta are staged beside each query tile, and dV_J^T[d][j] += dO_I^T[d][i] P[i][j]
// is accumulated too and added to the diagonal block's part in dvf.
// ---------------------------------------------------------------------------
template <bool SM, int KD, int NP>
struct ColSmem {
  union {
    struct {
      bf16 qa[3][NP][64 * KD];  // [buffer][plane], swizzled (chunk c of row r at c ^ (r & 7))
      bf16 qb[3][NP][64 * KD];
      bf16 dv[3][NP][64 * KD];
    } st;
    struct {  // 64-column halves at KD = 128
      float a[KD / 64][64][68];  // d k~ (same large chunk), then the result
      float f[KD / 64][64][68];  // dKL
      float m[KD / 64][64][68];  // SUF_J blocks, then k~_J
    } fin;
  } u;
  float lse[SM ? 3 : 1][64];  // softmax: lse and delta of the staged query rows
  float dl[SM ? 3 : 1][64];
};

// The column sweep's last step at KD = 128, per chunk J of the pair, on 64 x 64 fp32 LDS
// blocks (a, f: 64-column halves of d k~ (same) and dKL; m: operand blocks):
//   d k~_J[:, c] = d k~(same)[:, c] + sum_k dKL[:, k] SUF_J(k, c)   (block (k, c) of SUF_J)
//   dSUF_J(r, c) = dKL[:, r]^T k~_J[:, c]
// Softmax mode: the same-chunk part was parked in dkt and dKL is in as_.
template <bool SM>
__device__ __forceinline__ void col_finish128(float (*a)[64][68], float (*f)[64][68], float (*m)[64][68],
                                              const f32x16 (&as_)[4], const f32x16 (&af)[4], float F, int J1, int NT,
                                              int T, int bh, int bhq, const PathFwdWs& ws, const PathBwdWs& bw) {
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 5, l32 = lane & 31;
  const int cl = dl_col();
  for (int half = 0; half < 2; ++half) {
    const int J = J1 + half;
    if (J >= NT) break;
    if ((w >> 1) == half) {
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int r = (w & 1) * 32 + l32, c = (t & 1) * 32 + drow(e, g);
          if (!SM) a[t >> 1][r][c] = F * as_[t][e];
          f[t >> 1][r][c] = F * (SM ? as_[t][e] : af[t][e]);
        }
    }
    const float* suf = ws.suf + ((int64_t)bh * NT + J) * (128 * 128);
    float* dkt = bw.dkt + ((int64_t)bhq * T + J * PC) * 128;
#pragma unroll 1
    for (int ch = 0; ch < 2; ++ch) {
      load_blk(m[0], suf + 64 * ch, 128);
      load_blk(m[1], suf + 64 * 128 + 64 * ch, 128);
      __syncthreads();
      f32x16 r = mgemm64<false, false>(f[0], m[0], zero16());
      r = mgemm64<false, false>(f[1], m[1], r);
      DL_FOR_E {
        const int rr = dl_row(e);
        float* p = dkt + (int64_t)rr * 128 + 64 * ch + cl;
        *p = r[e] + (SM ? *p : a[ch][rr][cl]);
      }
      __syncthreads();
    }
    load_rows64_f32(m[0], ws.kt + ((int64_t)bh * T + J * PC) * 128, 128);
    load_rows64_f32(m[1], ws.kt + ((int64_t)bh * T + J * PC) * 128 + 64, 128);
    __syncthreads();
    float* dsuf = bw.dsuf + ((int64_t)bhq * NT + J) * (128 * 128);
#pragma unroll 1
    for (int blk = 0; blk < 4; ++blk) {
      const int ra = blk >> 1, cb_ = blk & 1;
      const f32x16 r = mgemm64<true, false>(f[ra], m[cb_], zero16());
      DL_FOR_E dsuf[(int64_t)(64 * ra + dl_row(e)) * 128 + 64 * cb_ + cl] = r[e];
    }
    __syncthreads();
  }
}

// KD: head dim (64 or 128).  F32: X and Y rows are bf16 hi planes with their lo planes at
// xsrc + x_lo, ysrc + y_lo, and every operand product is a 3-term split (mm3)
template <bool SM, int KD, bool F32>
__global__ __launch_bounds__(256) LUCID_TWO_WAVES_IF(KD == 64 && !F32) void path_bwd_col_kernel(
    const bf16* __restrict__ xsrc, Strides xs, int64_t x_lo, const bf16* __restrict__ ysrc, Strides ys, int64_t y_lo,
    int HQ, int H, int T, float scale, PathFwdWs ws, PathBwdWs bw) {
  constexpr int NKS = KD / 16, NVT = KD / 32, CPR = KD / 8;  // k-steps, 32-column tiles, 16-byte chunks per row
  constexpr int NP = F32 ? 2 : 1;
  constexpr int PT = NP * 64 * CPR / 256;  // direct loads per wave for one staged tile (all planes)
  __shared__ __attribute__((aligned(16))) ColSmem<SM, KD, NP> sm;
  const int NT = T / PC, NS = (NT + PR - 1) / PR;
  const int J1 = 2 * blockIdx.y, bhq = blockIdx.x;  // heaviest (earliest) key pairs of all heads first
  const int G_ = HQ / H;
  const int b = bhq / HQ, hq = bhq - b * HQ, bh = b * H + hq / G_;
  const bf16* xh = xsrc + b * xs.b + hq * xs.h;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 5, l32 = lane & 31;
  const int Jw = J1 + (w >> 1);        // this wave's key chunk
  const bool live = Jw < NT;           // NT odd: the last pair has one chunk
  const int sJ = J1 / PR, cb = sJ * PR, ceJ = min(cb + PR, NT) - 1;
  const float sl2 = scale * LOG2E_F, cc0 = LOG2E_F / scale;
  // dA = F dP exp2(sl2 S) (LUCID-Path, F = -s 2^-cc0) or F P (dP - delta) (PaTH softmax,
  // F = s): the constant F is applied to the dK accumulators where the sweep hands them on
  const float F = SM ? scale : -scale * __builtin_amdgcn_exp2f(-cc0);

  bf16x8 kbs[NKS][NP], kbf[NKS][NP], ob[NKS][NP];
  {
    const int jr = min(J1 * PC + 32 * w + l32, T - 1);
    const bf16* yrow = ysrc + b * ys.b + (SM ? hq / G_ : hq) * ys.h + (int64_t)jr * ys.t;
#pragma unroll
    for (int st = 0; st < NKS; ++st) {
      const bf16* ps = ws.kt + ((int64_t)bh * T + jr) * KD + 16 * st + 8 * g;
      const bf16* pf = ws.kl + ((int64_t)bh * T + jr) * KD + 16 * st + 8 * g;
      kbs[st][0] = ld8(ps);
      kbf[st][0] = ld8(pf);
      ob[st][0] = ld8(yrow + 16 * st + 8 * g);
      if constexpr (F32) {
        kbs[st][1] = ld8(ps + ws.lo_kt);
        kbf[st][1] = ld8(pf + ws.lo_kl);
        ob[st][1] = ld8(yrow + y_lo + 16 * st + 8 * g);
      }
    }
  }
  f32x16 as_[NVT], af[NVT];
  f32x16 dva[SM ? NVT : 1];  // softmax: dV^T of this wave's keys
#pragma unroll
  for (int t = 0; t < NVT; ++t) {
    as_[t] = zero16();
    af[t] = zero16();
    if (SM) dva[t] = zero16();
  }

  // step k stages query tile I = J1 + 1 + k
  const int nsteps = NT - 1 - J1;
  // newest vector-memory ops of a step, per wave: 3 tiles inside J's large chunk, 2 beyond
  auto near = [&](int k) { return J1 + 1 + k <= ceJ; };
  int plan_r[PT], plan_x[PT];
  dma_plan<64, CPR>(KD, plan_r);
  if (SM) dma_plan<64, CPR>(xs.t, plan_x);
  auto stage = [&](int k) {
    const int I = J1 + 1 + k, buf = k % 3;
    const bool same = I <= ceJ;
    const bf16* q1 = same ? ws.qs + ((int64_t)bhq * PR + (J1 - cb)) * T * KD
                          : ws.qb + ((int64_t)bhq * NS + sJ) * T * KD;
    const int64_t qlo = same ? ws.lo_qs : ws.lo_qb;
#pragma unroll
    for (int pl = 0; pl < NP; ++pl) {
      dma_stage<64, CPR>(plan_r, q1 + pl * qlo + (int64_t)I * PC * KD, sm.u.st.qa[buf][pl]);
      dma_stage<64, CPR>(SM ? plan_x : plan_r, xh + pl * x_lo + (int64_t)I * PC * xs.t, sm.u.st.dv[buf][pl]);
      if (same)  // the second chunk of the pair has its own query operand inside the large chunk
        dma_stage<64, CPR>(plan_r,
                           ws.qs + pl * ws.lo_qs + ((int64_t)bhq * PR + (J1 + 1 - cb)) * T * KD + (int64_t)I * PC * KD,
                           sm.u.st.qb[buf][pl]);
    }
    if (SM) {  // one more load for waves 0 and 1
      if (w == 0) dma_f32x64(ws.lse + (int64_t)bhq * T + I * PC, sm.lse[buf]);
      if (w == 1) dma_f32x64(bw.delta + (int64_t)bhq * T + I * PC, sm.dl[buf]);
    }
  };
  // wait until the step after the next one is the only one in flight
  auto wait_next = [&](bool nr) {
    if (SM && w < 2) {
      if (nr) dma_wait_but<3 * PT + 1>();
      else dma_wait_but<2 * PT + 1>();
    } else {
      if (nr) dma_wait_but<3 * PT>();
      else dma_wait_but<2 * PT>();
    }
  };
  if (nsteps > 0) {
    stage(0);
    if (nsteps > 1) {
      stage(1);
      wait_next(near(1));
    } else {
      dma_wait();
    }
  }
  __syncthreads();
  // softmax (register budget): as_ holds d k~ (same large chunk) until the sweep leaves
  // J's large chunk, then it is parked in dkt and as_ collects dKL
  bool parked = false;
  auto park = [&]() {
    if (live) {
      float* dst = bw.dkt + ((int64_t)bhq * T + Jw * PC + (w & 1) * 32 + l32) * KD;
#pragma unroll
      for (int t = 0; t < NVT; ++t)
#pragma unroll
        for (int qq = 0; qq < 4; ++qq) {
          f32x4 x;
#pragma unroll
          for (int u = 0; u < 4; ++u) x[u] = F * as_[t][4 * qq + u];
          *reinterpret_cast<f32x4*>(dst + t * 32 + 8 * qq + 4 * g) = x;
        }
#pragma unroll
      for (int t = 0; t < NVT; ++t) as_[t] = zero16();
    }
    parked = true;
  };
  for (int k = 0; k < nsteps; ++k) {
    const int buf = k % 3;
    if (k + 2 < nsteps) stage(k + 2);
    const int I = J1 + 1 + k;
    if (SM && I == ceJ + 1) park();
    if (live && I > Jw) {
      const bool same = I <= ceJ;
      bf16 (*qt)[64 * KD] = (w >= 2 && same) ? sm.u.st.qb[buf] : sm.u.st.qa[buf];  // planes
#pragma unroll
      for (int rh = 0; rh < 2; ++rh) {
        f32x16 sc = zero16(), dp = zero16();
#pragma unroll
        for (int st = 0; st < NKS; ++st) {
          bf16x8 qa8[NP], da8[NP];
#pragma unroll
          for (int pl = 0; pl < NP; ++pl) {
            qa8[pl] = ld8(swz<CPR>(qt[pl], rh * 32 + l32, 2 * st + g));
            da8[pl] = ld8(swz<CPR>(sm.u.st.dv[buf][pl], rh * 32 + l32, 2 * st + g));
          }
          sc = mm3<NP>(qa8, same ? kbs[st] : kbf[st], sc);
          dp = mm3<NP>(da8, ob[st], dp);
        }
        if (SM) {
#pragma unroll
          for (int qq = 0; qq < 4; ++qq) {  // rows rh*32 + drow(4qq + u, g)
            const f32x4 c4 = *reinterpret_cast<const f32x4*>(sm.lse[buf] + rh * 32 + 8 * qq + 4 * g);
            const f32x4 d4 = *reinterpret_cast<const f32x4*>(sm.dl[buf] + rh * 32 + 8 * qq + 4 * g);
#pragma unroll
            for (int u = 0; u < 4; ++u) {
              const int e = 4 * qq + u;
              sc[e] = __builtin_amdgcn_exp2f(fmaf(sc[e], sl2, -c4[u]));  // P
              dp[e] = sc[e] * (dp[e] - d4[u]);                           // dA / F
            }
          }
          bf16x8 pp[2][NP];
#pragma unroll
          for (int hh = 0; hh < 2; ++hh) {
            pp[hh][0] = pack_b(sc, hh);
            if constexpr (F32) pp[hh][1] = pack_lo(sc, hh, pp[hh][0]);
          }
#pragma unroll
          for (int t = 0; t < NVT; ++t)
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
              bf16x8 xa[NP];
#pragma unroll
              for (int pl = 0; pl < NP; ++pl) xa[pl] = lds_tr_a<CPR>(sm.u.st.dv[buf][pl], rh * 32 + 16 * hh, t * 32);
              dva[t] = mm3<NP>(xa, pp[hh], dva[t]);
            }
#pragma unroll
          for (int e = 0; e < 16; ++e) sc[e] = dp[e];
        } else {
#pragma unroll
          for (int e = 0; e < 16; ++e) sc[e] = dp[e] * __builtin_amdgcn_exp2f(sc[e] * sl2);
        }
        bf16x8 dd[2][NP];
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          dd[hh][0] = pack_b(sc, hh);
          if constexpr (F32) dd[hh][1] = pack_lo(sc, hh, dd[hh][0]);
        }
#pragma unroll
        for (int t = 0; t < NVT; ++t) {
          bf16x8 a0[NP], a1[NP];
#pragma unroll
          for (int pl = 0; pl < NP; ++pl) {
            a0[pl] = lds_tr_a<CPR>(qt[pl], rh * 32, t * 32);
            a1[pl] = lds_tr_a<CPR>(qt[pl], rh * 32 + 16, t * 32);
          }
          if (same || SM) {  // softmax: one accumulator, the same-chunk part is parked in dkt
            as_[t] = mm3<NP>(a0, dd[0], as_[t]);
            as_[t] = mm3<NP>(a1, dd[1], as_[t]);
          } else {
            af[t] = mm3<NP>(a0, dd[0], af[t]);
            af[t] = mm3<NP>(a1, dd[1], af[t]);
          }
        }
      }
    }
    if (k + 2 < nsteps) {  // the step after next may stay in flight
      wait_next(near(k + 2));
    } else {
      dma_wait();
    }
    __syncthreads();
  }
  if (SM && !parked) park();
  if (SM && live) {  // dV_J rows: the diagonal block's part is already in dvf
    float* dst = bw.dvf + ((int64_t)bhq * T + Jw * PC + (w & 1) * 32 + l32) * KD;
#pragma unroll
    for (int t = 0; t < NVT; ++t)
#pragma unroll
      for (int qq = 0; qq < 4; ++qq) {
        f32x4* p = reinterpret_cast<f32x4*>(dst + t * 32 + 8 * qq + 4 * g);
        f32x4 x = *p;
#pragma unroll
        for (int u = 0; u < 4; ++u) x[u] += dva[t][4 * qq + u];
        *p = x;
      }
  }
  // ---- per chunk of the pair: d k~_J = dk~(same) + dKL SUF_J, dSUF_J = dKL^T k~_J ----
  if constexpr (KD == 128) {
    col_finish128<SM>(sm.u.fin.a, sm.u.fin.f, sm.u.fin.m, as_, af, F, J1, NT, T, bh, bhq, ws, bw);
  } else {
  const int r0 = (tid >> 4) * 4, c0 = (tid & 15) * 4;
  for (int half = 0; half < 2; ++half) {
    const int J = J1 + half;
    if (J >= NT) break;
    if ((w >> 1) == half) {
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          if (!SM) sm.u.fin.a[0][(w & 1) * 32 + l32][t * 32 + drow(e, g)] = F * as_[t][e];
          sm.u.fin.f[0][(w & 1) * 32 + l32][t * 32 + drow(e, g)] = F * (SM ? as_[t][e] : af[t][e]);
        }
    }
    load_mat64<false>(sm.u.fin.m[0], ws.suf + ((int64_t)bh * NT + J) * 4096);
    __syncthreads();
    float acc4[4][4];
    zero44(acc4);
    lds_gemm64<false, false>(sm.u.fin.f[0], sm.u.fin.m[0], acc4);  // dKL SUF
    {
      float* dst = bw.dkt + ((int64_t)bhq * T + J * PC) * 64;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        f32x4 v;
        if (SM) v = *reinterpret_cast<const f32x4*>(dst + (r0 + i) * 64 + c0);  // parked part
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = acc4[i][j] + (SM ? v[j] : sm.u.fin.a[0][r0 + i][c0 + j]);
        *reinterpret_cast<f32x4*>(dst + (r0 + i) * 64 + c0) = v;
      }
    }
    __syncthreads();
    if constexpr (F32)
      load_rows64_split(sm.u.fin.m[0], ws.kt + ((int64_t)bh * T + J * PC) * 64, 64, ws.lo_kt);
    else
      load_rows64_f32(sm.u.fin.m[0], ws.kt + ((int64_t)bh * T + J * PC) * 64, 64);
    __syncthreads();
    zero44(acc4);
    lds_gemm64<true, false>(sm.u.fin.f[0], sm.u.fin.m[0], acc4);  // dSUF = dKL^T k~
    {
      float* dst = bw.dsuf + ((int64_t)bhq * NT + J) * 4096;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        f32x4 v;
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = acc4[i][j];
        *reinterpret_cast<f32x4*>(dst + (r0 + i) * 64 + c0) = v;
      }
    }
    __syncthreads();
  }
  }
}

// ---------------------------------------------------------------------------
// PaTH softmax backward of the diagonal blocks, per (chunk c, query head):
//   delta_i = dO_i . O_i,  P = exp2(s' A_diag - lse_i) (j <= i),
//   dA_diag = s P (dO V^T - delta_i),  dV_c = P^T dO_c   (the column sweep adds the rest)
// fp32 on LDS, dO and V rows as 64-column halves at KD = 128.  grid (NT, B*HQ)
// ---------------------------------------------------------------------------
template <int KD, bool F32>
__global__ __launch_bounds__(256) void path_softmax_diag_bwd_kernel(const pin_t<F32>* __restrict__ dout, Strides dos,
                                                                    const pin_t<F32>* __restrict__ o, Strides os,
                                                                    const pin_t<F32>* __restrict__ v, Strides vs,
                                                                    int HQ, int H, int T, float scale, PathFwdWs ws,
                                                                    PathBwdWs bw) {
  constexpr int NH = KD / 64;
  __shared__ __attribute__((aligned(16))) float Dm[NH][64][68];
  __shared__ __attribute__((aligned(16))) float Vm[NH][64][68];
  __shared__ __attribute__((aligned(16))) float Pm[64][68];
  __shared__ float dls[64], lss[64];
  const int NT = T / PC;
  const int c = blockIdx.x, bhq = blockIdx.y;
  const int G_ = HQ / H;
  const int b = bhq / HQ, hq = bhq - b * HQ, h = hq / G_;
  const int tid = threadIdx.x;
  const int r0 = (tid >> 4) * 4, c0 = (tid & 15) * 4;
  const int t0 = c * PC;
#pragma unroll
  for (int hh = 0; hh < NH; ++hh) {
    load_rows64_f32(Dm[hh], dout + b * dos.b + hq * dos.h + (int64_t)t0 * dos.t + 64 * hh, dos.t);
    load_rows64_f32(Vm[hh], v + b * vs.b + h * vs.h + (int64_t)t0 * vs.t + 64 * hh, vs.t);
  }
  {  // delta of row r: 4 threads x 16 columns per 64-column half
    const int r = tid >> 2, cc = (tid & 3) * 16;
    const pin_t<F32>* orow = o + b * os.b + hq * os.h + (int64_t)(t0 + r) * os.t + cc;
    const pin_t<F32>* drow_ = dout + b * dos.b + hq * dos.h + (int64_t)(t0 + r) * dos.t + cc;
    float acc = 0.f;
#pragma unroll
    for (int hh = 0; hh < 2 * NH; ++hh) {
      const int off = 64 * (hh >> 1) + 8 * (hh & 1);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc = fmaf((float)orow[off + e], (float)drow_[off + e], acc);
    }
    acc += __shfl_xor(acc, 1, 64);
    acc += __shfl_xor(acc, 2, 64);
    if ((tid & 3) == 0) {
      dls[r] = acc;
      bw.delta[(int64_t)bhq * T + t0 + r] = acc;
      lss[r] = ws.lse[(int64_t)bhq * T + t0 + r];
    }
  }
  __syncthreads();
  const float sl2 = scale * LOG2E_F;
  {
    const float* ad = ws.ld + ((int64_t)bhq * NT + c) * 4096;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const f32x4 x = *reinterpret_cast<const f32x4*>(ad + (r0 + i) * 64 + c0);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        Pm[r0 + i][c0 + j] = (c0 + j <= r0 + i) ? __builtin_amdgcn_exp2f(fmaf(x[j], sl2, -lss[r0 + i])) : 0.f;
    }
  }
  __syncthreads();
  float acc[4][4];
  zero44(acc);
#pragma unroll
  for (int hh = 0; hh < NH; ++hh) lds_gemm64<false, true>(Dm[hh], Vm[hh], acc);  // dP = dO V^T
  {
    float* dst = bw.dad + ((int64_t)bhq * NT + c) * 4096;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f32x4 x;
#pragma unroll
      for (int j = 0; j < 4; ++j) x[j] = scale * Pm[r0 + i][c0 + j] * (acc[i][j] - dls[r0 + i]);
      *reinterpret_cast<f32x4*>(dst + (r0 + i) * 64 + c0) = x;
    }
  }
#pragma unroll
  for (int hh = 0; hh < NH; ++hh) {
    zero44(acc);
    lds_gemm64<true, false>(Pm, Dm[hh], acc);  // dV_c = P^T dO
    float* dst = bw.dvf + ((int64_t)bhq * T + t0) * KD + 64 * hh;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f32x4 x;
#pragma unroll
      for (int j = 0; j < 4; ++j) x[j] = acc[i][j];
      *reinterpret_cast<f32x4*>(dst + (r0 + i) * KD + c0) = x;
    }
  }
}

// ---------------------------------------------------------------------------
// Products backward inside one large chunk (cumprod_householder_bwd.py:13-95):
//   F = dHL_s; for c from the bottom up: dHc_c += SUF_c^T F; F <- F Hc_c^T + dSUF_c
// grid (NS, B*HQ)
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void path_products_bwd_kernel(int HQ, int H, int T, PathFwdWs ws, PathBwdWs bw) {
  __shared__ __attribute__((aligned(16))) float F[64][68];
  __shared__ __attribute__((aligned(16))) float S[64][68];
  __shared__ __attribute__((aligned(16))) float Hs[64][68];
  const int NT = T / PC, NS = (NT + PR - 1) / PR;
  const int s = blockIdx.x, bhq = blockIdx.y;
  const int G_ = HQ / H;
  const int b = bhq / HQ, hq = bhq - b * HQ, bh = b * H + hq / G_;
  const int cb = s * PR, ce = min(cb + PR, NT) - 1;
  const int cl = dl_col();
  // products on the matrix cores (mgemm64, D layout); SUF_c and Hc_c of the next chunk
  // are fetched into registers while the current one is processed
  f32x4 ps[4], ph[4];
  mat_fetch(ps, ws.suf + ((int64_t)bh * NT + cb) * 4096);
  mat_fetch(ph, ws.hc + ((int64_t)bh * NT + cb) * 4096);
  load_mat64<false>(F, bw.dhl + ((int64_t)bhq * NS + s) * 4096);
  for (int c = cb; c <= ce; ++c) {
    mat_put(S, ps);
    mat_put(Hs, ph);
    __syncthreads();
    if (c < ce) {
      mat_fetch(ps, ws.suf + ((int64_t)bh * NT + c + 1) * 4096);
      mat_fetch(ph, ws.hc + ((int64_t)bh * NT + c + 1) * 4096);
    }
    {
      const f32x16 a = mgemm64<true, false>(S, F, zero16());  // dHc_c += SUF_c^T F
      float* dst = bw.dhc + ((int64_t)bhq * NT + c) * 4096;
      DL_FOR_E dst[dl_row(e) * 64 + cl] += a[e];
    }
    const f32x16 f = mgemm64<false, true>(F, Hs, zero16());  // F <- F Hc_c^T + dSUF_c
    __syncthreads();
    {
      const float* ds = bw.dsuf + ((int64_t)bhq * NT + c) * 4096;
      DL_FOR_E {
        const int r = dl_row(e);
        F[r][cl] = f[e] + ds[r * 64 + cl];
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Backward of the WY form of one chunk (intra_chunk_preprocess_bwd.py:14-110):
//   Wb = beta W, Tm = (I + stril(Wb W^T))^-1, W2 = Tm Wb, Hc = I - W^T W2,
//   q~ = q - QW W2 (QW = tril(q W^T)), k~ = k - TW^T W (TW = Tm stril(Wb k^T)),
//   A_diag = tril(q k^T - QW TW).
// Inputs d q~, d k~, dA_diag, dHc; outputs dq, dk, dw, dbeta (per query head, fp32).
// The 64x64 products run on the matrix cores (mgemm64, 3-term bf16 split, ~fp32
// accuracy); every wave keeps its 32x32 tile of each running result in MFMA D layout
// (rows dl_row(e), column dl_col()).  Operands live in 9 fp32 LDS buffers.
// grid (NT, B*HQ)
// ---------------------------------------------------------------------------
template <bool F32>
__global__ __launch_bounds__(256) void path_wy_bwd_kernel(const pin_t<F32>* __restrict__ q, Strides qs,
                                                          const pin_t<F32>* __restrict__ k, Strides ks,
                                                          const pin_t<F32>* __restrict__ w, Strides wst,
                                                          const pin_t<F32>* __restrict__ beta, Strides bst, int HQ,
                                                          int H, int T, PathFwdWs ws, PathBwdWs bw) {
  __shared__ __attribute__((aligned(16))) float W[64][68];
  __shared__ __attribute__((aligned(16))) float Wb[64][68];
  __shared__ __attribute__((aligned(16))) float Q[64][68];
  __shared__ __attribute__((aligned(16))) float K[64][68];
  __shared__ __attribute__((aligned(16))) float Tm[64][68];
  __shared__ __attribute__((aligned(16))) float S1[64][68];
  __shared__ __attribute__((aligned(16))) float S2[64][68];
  __shared__ __attribute__((aligned(16))) float S3[64][68];
  __shared__ __attribute__((aligned(16))) float S4[64][68];
  __shared__ float bsh[64];
  const int NT = T / PC;
  const int c = blockIdx.x, bhq = blockIdx.y;
  const int G_ = HQ / H;
  const int b = bhq / HQ, hq = bhq - b * HQ, h = hq / G_, bh = b * H + h;
  const int tid = threadIdx.x;
  const int t0 = c * PC;
  const f32x16 z = zero16();

  // The fp32 inputs go to registers first (16 values per thread each) so their
  // latency overlaps the WY recomputation; each is stored to LDS when its buffer frees.
  f32x4 pw2[4], pdh[4], pdq[4], pdk[4], pda[4];
  mat_fetch(pw2, ws.w2 + ((int64_t)bh * T + t0) * 64);
  mat_fetch(pdh, bw.dhc + ((int64_t)bhq * NT + c) * 4096);
  mat_fetch(pdq, bw.dqt + ((int64_t)bhq * T + t0) * 64);
  mat_fetch(pdk, bw.dkt + ((int64_t)bhq * T + t0) * 64);
  mat_fetch(pda, bw.dad + ((int64_t)bhq * NT + c) * 4096);
  load_rows64_f32(W, w + b * wst.b + h * wst.h + (int64_t)t0 * wst.t, wst.t);
  load_rows64_f32(Q, q + b * qs.b + hq * qs.h + (int64_t)t0 * qs.t, qs.t);
  load_rows64_f32(K, k + b * ks.b + h * ks.h + (int64_t)t0 * ks.t, ks.t);
  __syncthreads();
  {
    const int r = tid >> 2, cc = (tid & 3) * 16;
    const float bt = (float)beta[b * bst.b + h * bst.h + (int64_t)(t0 + r) * bst.t];
    if ((tid & 3) == 0) bsh[r] = bt;
#pragma unroll
    for (int e = 0; e < 16; ++e) Wb[r][cc + e] = bt * W[r][cc + e];
  }
  mat_put(S1, pw2);  // W2
  mat_put(S2, pdh);  // dHc
  __syncthreads();
  dl_store(Tm, mgemm64<false, true>(Wb, W, z), 2);
  __syncthreads();
  invert_unit_lower64(Tm);
  f32x16 aW = dl_neg(mgemm64<false, true>(S1, S2, z));   // -W2 dHc^T
  f32x16 aW2 = dl_neg(mgemm64<false, false>(W, S2, z));  // -W dHc
  dl_store(S3, mgemm64<false, true>(Q, W, z), 1);        // QW
  __syncthreads();
  mat_put(S2, pdq);  // d q~
  __syncthreads();
  f32x16 aq = dl_load(S2);
  f32x16 dQW = dl_neg(mgemm64<false, true>(S2, S1, z));  // -dq~ W2^T
  {
    const f32x16 t = mgemm64<true, false>(S3, S2, z);    // QW^T dq~
    DL_FOR_E aW2[e] -= t[e];
  }
  dl_store(S4, mgemm64<false, true>(Wb, K, z), 2);       // WBK
  __syncthreads();
  dl_store(S1, mgemm64<false, false>(Tm, S4, z), 0);     // TW
  mat_put(S2, pdk);                                       // d k~
  __syncthreads();
  f32x16 ak = dl_load(S2);
  f32x16 dTW = dl_neg(mgemm64<false, true>(W, S2, z));   // -W dk~^T
  {
    const f32x16 t = mgemm64<false, false>(S1, S2, z);   // TW dk~
    DL_FOR_E aW[e] -= t[e];
  }
  __syncthreads();
  mat_put(S2, pda);  // dA_diag
  __syncthreads();
  aq = mgemm64<false, false>(S2, K, aq);  // dq += dA K
  ak = mgemm64<true, false>(S2, Q, ak);   // dk += dA^T Q
  {
    const f32x16 t = mgemm64<false, true>(S2, S1, z);   // dA TW^T
    const f32x16 t5 = mgemm64<true, false>(S3, S2, z);  // QW^T dA
    DL_FOR_E {
      dQW[e] -= t[e];
      dTW[e] -= t5[e];
    }
  }
  __syncthreads();
  dl_store(S2, dQW, 1);
  dl_store(S1, dTW, 0);
  __syncthreads();
  aq = mgemm64<false, false>(S2, W, aq);         // dq += tril(dQW) W
  aW = mgemm64<true, false>(S2, Q, aW);          // dW += tril(dQW)^T q
  f32x16 dTm = mgemm64<false, true>(S1, S4, z);  // dTm = dTW WBK^T
  dl_store(S3, mgemm64<true, false>(Tm, S1, z), 2);  // dWBK = stril(Tm^T dTW)
  __syncthreads();
  f32x16 aWb = mgemm64<false, false>(S3, K, z);  // dWb = dWBK k
  ak = mgemm64<true, false>(S3, Wb, ak);         // dk += dWBK^T Wb
  dl_store(S2, aW2, 0);                          // dW2
  __syncthreads();
  dTm = mgemm64<false, true>(S2, Wb, dTm);  // dTm += dW2 Wb^T
  aWb = mgemm64<true, false>(Tm, S2, aWb);  // dWb += Tm^T dW2
  dl_store(S1, dTm, 0);
  __syncthreads();
  dl_store(S3, mgemm64<true, false>(Tm, S1, z), 0);  // Tm^T dTm
  __syncthreads();
  dl_store(S4, dl_neg(mgemm64<false, true>(S3, Tm, z)), 2);  // da = -stril((Tm^T dTm) Tm^T)
  __syncthreads();
  aWb = mgemm64<false, false>(S4, W, aWb);  // dWb += da W
  aW = mgemm64<true, false>(S4, Wb, aW);    // dW += da^T Wb
  // dW += beta dWb; dbeta_r = sum_c dWb[r][c] W[r][c] (row sums through S2)
  const int cl = dl_col();
  DL_FOR_E {
    const int r = dl_row(e);
    aW[e] += bsh[r] * aWb[e];
    S2[r][cl] = aWb[e] * W[r][cl];
  }
  const int64_t rowbase = ((int64_t)bhq * T + t0) * 64;
  DL_FOR_E {
    const int64_t off = rowbase + dl_row(e) * 64 + cl;
    bw.dq[off] = aq[e];
    bw.dk[off] = ak[e];
    bw.dw[off] = aW[e];
  }
  __syncthreads();
  {
    const int r = tid >> 2, cc = (tid & 3) * 16;
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 16; i += 4) {
      const f32x4 v = *reinterpret_cast<const f32x4*>(&S2[r][cc + i]);
      s += (v[0] + v[1]) + (v[2] + v[3]);
    }
    s += __shfl_xor(s, 1, 64);
    s += __shfl_xor(s, 2, 64);
    if ((tid & 3) == 0) bw.db[(int64_t)bhq * T + t0 + r] = s;
  }
}

// ---------------------------------------------------------------------------
// GQA sums over the query heads of each kv head (parallel.py:165-171) and casts
// to the caller's bf16 gradients.  grid (T/4, B*H), thread = (row, column), KD / 64 columns
// per thread (KD: head dim of the fp32 rows)
// ---------------------------------------------------------------------------
template <bool F32>
__global__ __launch_bounds__(256) void path_reduce_kernel(int HQ, int H, int T, int KD, PathBwdWs bw,
                                                          pin_t<F32>* __restrict__ dq, Strides dqs,
                                                          pin_t<F32>* __restrict__ dk, Strides dks,
                                                          pin_t<F32>* __restrict__ dv, Strides dvs,
                                                          pin_t<F32>* __restrict__ dw, Strides dws,
                                                          pin_t<F32>* __restrict__ db, Strides dbs) {
  const int bh = blockIdx.y;
  const int b = bh / H, h = bh - b * H;
  const int G_ = HQ / H;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  for (int col = threadIdx.x & 63; col < KD; col += 64) {
    float sk = 0.f, sv = 0.f, sw = 0.f, sb = 0.f;
    for (int gi = 0; gi < G_; ++gi) {
      const int hq = h * G_ + gi;
      const int64_t bhq = (int64_t)b * HQ + hq;
      const int64_t off = (bhq * T + t) * KD + col;
      sk += bw.dk[off];
      sv += bw.dvf[off];
      sw += bw.dw[off];
      if (col == 0) sb += bw.db[bhq * T + t];
      dq[b * dqs.b + hq * dqs.h + (int64_t)t * dqs.t + col] = (pin_t<F32>)bw.dq[off];
    }
    dk[b * dks.b + h * dks.h + (int64_t)t * dks.t + col] = (pin_t<F32>)sk;
    dv[b * dvs.b + h * dvs.h + (int64_t)t * dvs.t + col] = (pin_t<F32>)sv;
    dw[b * dws.b + h * dws.h + (int64_t)t * dws.t + col] = (pin_t<F32>)sw;
    if (col == 0) db[b * dbs.b + h * dbs.h + (int64_t)t * dbs.t] = (pin_t<F32>)sb;
  }
}

}  // namespace lucid
