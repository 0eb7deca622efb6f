// LUCID-Path forward on CDNA4 (gfx950): O = (I + L)^-1 V,
//   L_ij = exp(s A_ij - 1/s) (j < i),  A_ij = q_i^T H_i ... H_{j+1} k_j,  H_t = I - beta_t w_t w_t^T
// (lucid_path/triton_code/parallel.py:27-76, triangular_solve_fwd.py:19-225).
//
// Two-level chunking (small chunk 64, large chunk PR = 16 small chunks, 1024 positions:
// 8 measured 5 % slower at config 4, 32 2 % slower): every inter-chunk logit block
// is ONE GEMM of a query carried down and a key carried up to a common boundary:
//   A_IJ = QB_I^(sJ) KL_J^T   (J in an earlier large chunk)
//   A_IJ = QS_I^(J)  k~_J^T   (J earlier in the same large chunk)
// so the chained solve has no per-pair Householder propagation (the reference
// propagates the query through every chunk pair, triangular_solve_fwd.py:170-196).
//
// Kernels (256 threads):
//   path_chunk_kernel      per (chunk, query head): WY form T_inv, W2, Hc = I - W^T W2,
//                          q~, k~, L_diag and Y = (I + L_diag)^-1   (fp32, LDS)
//   path_large_kernel      per (large chunk, kv head): SUF_c, HL_s and KL = k~ SUF^T
//   path_transport_kernel  per (pair of chunks, query head): QS and QB (MFMA, 3-term bf16 split)
//   path_solve_fwd_kernel  chained solve per query head (chain counters as in LUCID)
//   path_kcache_kernel     k_cache = keys carried to the sequence end (use_cache)
#include "path_common.h"

namespace lucid {

// K: the kernels' head dim (64 or 128); in-chunk C x C matrices are 64 x 64 at either
struct PathFwdWs {
  float* w2;    // [BH][T][K]         W2 = T_inv (beta W)
  float* hc;    // [BH][NT][K][K]     Hc = I - W^T W2
  bf16* kt;     // [BH][T][K]         k~ rows
  float* suf;   // [BH][NT][K][K]     SUF_c
  float* hl;    // [BH][NS][K][K]     HL_s
  bf16* hcs;    // [BH][NT][2][K][K]  Hc as bf16 hi and lo planes (the backward transport operand)
  bf16* hls;    // [BH][NS][2][K][K]  HL_s as bf16 hi and lo planes
  bf16* kl;     // [BH][T][K]         KL rows
  float* qt;    // [BHq][T][K]        q~
  float* ld;    // [BHq][NT][64][64]  L_diag (strictly lower)
  float* y;     // [BHq][NT][64][64]  (I + L_diag)^-1
  bf16* qs;     // [BHq][PR][T][K]    QS rows, slot = c - (first chunk of I's large chunk)
  bf16* qb;     // [BHq][NS][T][K]    QB rows
  bf16* oT;     // [BHq][K][T]        O^T, T-perm (chain operand)
  int* counters;  // [BHq]
  float* lse;   // [BHq][T]           PaTH softmax only: row log-sum-exp, exp2 domain (log2(l) + m)
  // fp32 inputs: element offsets of the lo planes of kt, kl, qs, qb, oT (0 with bf16 inputs)
  int64_t lo_kt, lo_kl, lo_qs, lo_qb, lo_oT;
  // fp32 inputs, PaTH softmax: split copy of V [BH][T][K] (hi plane, lo plane at + lo_vsp)
  bf16* vsp;
  int64_t lo_vsp;
};

// ---------------------------------------------------------------------------
// WY form and in-chunk transforms (triangular_solve_fwd.py:118-148, parallel.py:39-51)
// grid (NT, B*HQ).  kv-head outputs are written by the first query head of each group.
// ---------------------------------------------------------------------------
// F32: fp32 inputs; k~ is written as hi / lo planes
template <bool F32>
__global__ __launch_bounds__(256) void path_chunk_kernel(const pin_t<F32>* __restrict__ q, Strides qs,
                                                         const pin_t<F32>* __restrict__ k, Strides ks,
                                                         const pin_t<F32>* __restrict__ w, Strides wst,
                                                         const pin_t<F32>* __restrict__ beta, Strides bst, int HQ, int H,
                                                         int T, float scale, int softmax, PathFwdWs ws) {
  __shared__ __attribute__((aligned(16))) float Wm[64][68];
  __shared__ __attribute__((aligned(16))) float Wb[64][68];
  __shared__ __attribute__((aligned(16))) float Tm[64][68];
  __shared__ __attribute__((aligned(16))) float W2s[64][68];
  __shared__ __attribute__((aligned(16))) float Qs[64][68];
  __shared__ __attribute__((aligned(16))) float Ks[64][68];
  __shared__ __attribute__((aligned(16))) float X[64][68];
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

  load_rows64_f32(Wm, w + b * wst.b + h * wst.h + (int64_t)t0 * wst.t, wst.t);
  load_rows64_f32(Qs, q + b * qs.b + hq * qs.h + (int64_t)t0 * qs.t, qs.t);
  load_rows64_f32(Ks, k + b * ks.b + h * ks.h + (int64_t)t0 * ks.t, ks.t);
  __syncthreads();
  {
    const int r = tid >> 2, cc = (tid & 3) * 16;
    const float bt = (float)beta[b * bst.b + h * bst.h + (int64_t)(t0 + r) * bst.t];
#pragma unroll
    for (int e = 0; e < 16; ++e) Wb[r][cc + e] = bt * Wm[r][cc + e];
  }
  __syncthreads();
  // Products on the matrix cores (mgemm64); each wave keeps its 32x32 tile in D layout.
  // a = stril(beta W W^T) -> Tm, then T_inv = (I + a)^-1 in place
  dl_store(Tm, mgemm64<false, true>(Wb, Wm, z), 2);
  __syncthreads();
  invert_unit_lower64(Tm);
  // W2 = T_inv (beta W)
  {
    const f32x16 acc = mgemm64<false, false>(Tm, Wb, z);
    dl_store(W2s, acc, 0);
    if (kvw) {
      float* dst = ws.w2 + ((int64_t)bh * T + t0) * 64;
      DL_FOR_E dst[dl_row(e) * 64 + cl] = acc[e];
    }
  }
  __syncthreads();
  // Hc = I - W^T W2
  if (kvw) {
    const f32x16 acc = mgemm64<true, false>(Wm, W2s, z);
    float* dst = ws.hc + ((int64_t)bh * NT + c) * 4096;
    bf16* dsts = ws.hcs + ((int64_t)bh * NT + c) * 8192;
    DL_FOR_E {
      const int r = dl_row(e);
      const float x = (r == cl ? 1.f : 0.f) - acc[e];
      dst[r * 64 + cl] = x;
      put_split<2>(dsts, 4096, r * 64 + cl, x);
    }
  }
  // WBK = stril(beta W K^T) -> X
  dl_store(X, mgemm64<false, true>(Wb, Ks, z), 2);
  __syncthreads();
  // TW = T_inv WBK -> Wb (every read of beta W came before the last barrier)
  dl_store(Wb, mgemm64<false, false>(Tm, X, z), 0);
  __syncthreads();
  // k~ = K - TW^T W
  if (kvw) {
    const f32x16 acc = mgemm64<true, false>(Wb, Wm, z);
    bf16* dst = ws.kt + ((int64_t)bh * T + t0) * 64;
    DL_FOR_E {
      const int r = dl_row(e);
      put_split<F32 ? 2 : 1>(dst, ws.lo_kt, r * 64 + cl, Ks[r][cl] - acc[e]);
    }
  }
  // QW = tril(Q W^T) -> X (every read of WBK came before the last barrier)
  dl_store(X, mgemm64<false, true>(Qs, Wm, z), 1);
  __syncthreads();
  // q~ = Q - QW W2
  {
    const f32x16 acc = mgemm64<false, false>(X, W2s, z);
    float* dst = ws.qt + ((int64_t)bhq * T + t0) * 64;
    DL_FOR_E {
      const int r = dl_row(e);
      dst[r * 64 + cl] = Qs[r][cl] - acc[e];
    }
  }
  // A_diag = tril(Q K^T - QW TW); L_diag = stril(exp(s A - 1/s)) -> W2s, global
  // (PaTH softmax: the logits themselves, diagonal included; no inverse)
  const f32x16 qk = mgemm64<false, true>(Qs, Ks, z);
  const f32x16 qt = mgemm64<false, false>(X, Wb, z);
  float* dst = ws.ld + ((int64_t)bhq * NT + c) * 4096;
  if (softmax) {
    DL_FOR_E {
      const int r = dl_row(e);
      dst[r * 64 + cl] = cl <= r ? qk[e] - qt[e] : 0.f;
    }
    return;
  }
  __syncthreads();  // the q~ product above still reads W2s
  {
    const float sl2 = scale * LOG2E_F, cc0 = LOG2E_F / scale;
    DL_FOR_E {
      const int r = dl_row(e);
      const float v = cl < r ? __builtin_amdgcn_exp2f(fmaf(qk[e] - qt[e], sl2, -cc0)) : 0.f;
      W2s[r][cl] = v;
      dst[r * 64 + cl] = v;
    }
  }
  __syncthreads();
  invert_unit_lower64(W2s);
  {
    float* dy = ws.y + ((int64_t)bhq * NT + c) * 4096;
    for (int i = 0; i < 4; ++i) {
      const int f = 4 * (tid + 256 * i);
      *reinterpret_cast<f32x4*>(dy + f) = *reinterpret_cast<const f32x4*>(&W2s[f >> 6][f & 63]);
    }
  }
}

// ---------------------------------------------------------------------------
// Per large chunk: SUF_c (c from the top down), HL_s, KL = k~ SUF^T
// (cumprod_householder_fwd.py:13-79).  grid (NS, B*H)
// ---------------------------------------------------------------------------
template <bool F32>
__global__ __launch_bounds__(256) void path_large_kernel(int T, PathFwdWs ws) {
  __shared__ __attribute__((aligned(16))) float Sf[64][68];
  __shared__ __attribute__((aligned(16))) float Hs[64][68];
  __shared__ __attribute__((aligned(16))) float Kt[64][68];
  const int s = blockIdx.x, bh = blockIdx.y;
  const int NT = T / PC;
  const int tid = threadIdx.x;
  const int cb = s * PR, ce = min(cb + PR, NT) - 1;
  const int cl = dl_col();
  for (int idx = tid; idx < 4096; idx += 256) Sf[idx >> 6][idx & 63] = ((idx >> 6) == (idx & 63)) ? 1.f : 0.f;
  // products on the matrix cores (mgemm64, D layout); k~_c and Hc_c of the next chunk
  // are fetched into registers while the current one is processed
  const int kr = tid >> 2, kc = (tid & 3) * 16;
  bf16x8 pk[2], pl[2];
  f32x4 ph[4];
  auto fetch = [&](int c) {
    const bf16* src = ws.kt + ((int64_t)bh * T + c * PC + kr) * 64 + kc;
    pk[0] = ld8(src);
    pk[1] = ld8(src + 8);
    if constexpr (F32) {
      pl[0] = ld8(src + ws.lo_kt);
      pl[1] = ld8(src + ws.lo_kt + 8);
    }
    mat_fetch(ph, ws.hc + ((int64_t)bh * NT + c) * 4096);
  };
  fetch(ce);
  for (int c = ce; c >= cb; --c) {
#pragma unroll
    for (int hh = 0; hh < 2; ++hh)
#pragma unroll
      for (int e = 0; e < 8; ++e) Kt[kr][kc + 8 * hh + e] = (float)pk[hh][e] + (F32 ? (float)pl[hh][e] : 0.f);
    mat_put(Hs, ph);
    __syncthreads();
    if (c > cb) fetch(c - 1);
    {
      float* dst = ws.suf + ((int64_t)bh * NT + c) * 4096;
      for (int i = 0; i < 4; ++i) {
        const int f = 4 * (tid + 256 * i);
        *reinterpret_cast<f32x4*>(dst + f) = *reinterpret_cast<const f32x4*>(&Sf[f >> 6][f & 63]);
      }
    }
    // KL_c = k~_c SUF_c^T
    {
      const f32x16 a = mgemm64<false, true>(Kt, Sf, zero16());
      bf16* dst = ws.kl + ((int64_t)bh * T + c * PC) * 64;
      DL_FOR_E put_split<F32 ? 2 : 1>(dst, ws.lo_kl, dl_row(e) * 64 + cl, a[e]);
    }
    // SUF_{c-1} = SUF_c Hc_c
    const f32x16 sn = mgemm64<false, false>(Sf, Hs, zero16());
    __syncthreads();
    dl_store(Sf, sn, 0);
  }
  __syncthreads();
  float* dst = ws.hl + ((int64_t)bh * ((NT + PR - 1) / PR) + s) * 4096;
  bf16* dsts = ws.hls + ((int64_t)bh * ((NT + PR - 1) / PR) + s) * 8192;
  for (int i = 0; i < 4; ++i) {
    const int f = 4 * (tid + 256 * i);
    const f32x4 x = *reinterpret_cast<const f32x4*>(&Sf[f >> 6][f & 63]);
    *reinterpret_cast<f32x4*>(dst + f) = x;
#pragma unroll
    for (int u = 0; u < 4; ++u) put_split<2>(dsts, 4096, f + u, x[u]);
  }
}

// ---------------------------------------------------------------------------
// Query transport (transform_q.py:15-61): x = q~_I; QS slots for chunks of I's large
// chunk below I, then QB for every earlier large chunk.  One workgroup per pair of
// chunks A = 2p, B = 2p + 1 (one large chunk holds both) of one query head: B's
// sequence of transition matrices is A's with Hc_A in front, so after that one step
// the two 64-row blocks are carried together, each matrix loaded, transposed and
// synchronised once for 128 rows, and both blocks' rows (adjacent in T) emitted to
// the same slot.  grid (B*HQ, ceil(NT/2)): the work of a pair grows with p, so the
// late pairs of every head are dispatched first.
// ---------------------------------------------------------------------------
template <bool F32>
__global__ __launch_bounds__(256) void path_transport_kernel(int HQ, int H, int T, PathFwdWs ws) {
  __shared__ __attribute__((aligned(16))) float X[128][68];  // rows 0..63 = chunk A, 64..127 = chunk B
  // the step's transition matrix M as bf16 hi and lo planes, row-major, swizzled (chunk c of
  // row r at c ^ (r & 7)); its columns (the A operand of D^T = M^T X^T) come through
  // transposing reads
  __shared__ __attribute__((aligned(16))) bf16 Ms[2][64 * 64];
  const int p = (int)gridDim.y - 1 - (int)blockIdx.y, bhq = blockIdx.x;
  const int NT = T / PC, NS = (NT + PR - 1) / PR;
  const int G = HQ / H;
  const int b = bhq / HQ, hq = bhq - b * HQ, bh = b * H + hq / G;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, g = lane >> 5, l32 = lane & 31;
  const int A = 2 * p;
  const bool hasB = A + 1 < NT;
  const int sI = A / PR, cb = sI * PR;
  {
    const float* src = ws.qt + ((int64_t)bhq * T + A * PC) * 64;  // A's and B's rows are adjacent
    for (int idx = tid; idx < (hasB ? 8192 : 4096); idx += 256) X[idx >> 6][idx & 63] = src[idx];
  }
  __syncthreads();
  // rows r0 .. r0 + 64 * nblk of X -> bf16 rows at dst (row stride 64), and (F32) their
  // residuals at dst + lo
  auto emit = [&](bf16* dst, int64_t lo, int r0, int nblk) {
    const int cc = (tid & 3) * 16;
    for (int r = r0 + (tid >> 2); r < r0 + 64 * nblk; r += 64) {
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        bf16x8 v, vl;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          v[e] = (bf16)X[r][cc + 8 * hh + e];
          if constexpr (F32) vl[e] = (bf16)(X[r][cc + 8 * hh + e] - (float)v[e]);
        }
        *reinterpret_cast<bf16x8*>(dst + (int64_t)r * 64 + cc + 8 * hh) = v;
        if constexpr (F32) *reinterpret_cast<bf16x8*>(dst + lo + (int64_t)r * 64 + cc + 8 * hh) = vl;
      }
    }
  };
  // joint steps j = 0 .. nq-1 carry X through Hc_{A-1} .. Hc_cb (emitting QS), steps
  // nq .. nq+sI-1 through HL_{sI-1} .. HL_0 (emitting QB).  Each step emits X, then
  // multiplies it by the step's matrix; after the last emit X is not used, so the last step
  // only emits.  The matrix of the next step is loaded into registers while a step computes,
  // so no step waits for it.
  const int nq = A - cb, nsteps = nq + sI;
  auto mat = [&](int j) {  // hi plane (lo plane 4096 elements on); j = -1: Hc_A, B's own first step
    return (j < nq) ? ws.hcs + ((int64_t)bh * NT + (A - 1 - j)) * 8192
                    : ws.hls + ((int64_t)bh * NS + (sI - 1 - (j - nq))) * 8192;
  };
  auto slot = [&](int j) {  // destination of the rows emitted before step j (row 0 = chunk A's first row)
    return ((j < nq) ? ws.qs + (((int64_t)bhq * PR + (A - 1 - j - cb)) * T) * 64
                     : ws.qb + (((int64_t)bhq * NS + (sI - 1 - (j - nq))) * T) * 64) +
           (int64_t)A * PC * 64;
  };
  bf16x8 mr[4];  // thread t: plane u >> 1, 16-byte chunk q = t + 256 (u & 1) (row q >> 3, chunk q & 7)
  auto mload = [&](int j) {
    const bf16* M = mat(j);
#pragma unroll
    for (int u = 0; u < 4; ++u) mr[u] = ld8(M + (u >> 1) * 4096 + 8 * (tid + 256 * (u & 1)));
  };
  auto mstore = [&]() {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int q = tid + 256 * (u & 1);
      *reinterpret_cast<bf16x8*>(Ms[u >> 1] + swz_off<8>(q >> 3, q & 7)) = mr[u];
    }
  };
  const int dt = w >> 1, rt = w & 1;  // this wave's output tiles: (dt, rt) of A and (dt, rt + 2) of B
  // tile (dt, xr) of X M in D layout (m = column of the product, lane <-> row), 3-term split:
  // A operand = M^T rows = columns dt*32 + lane of M, k slots in the transposing read's order
  // (rows 16 st + jmap(slot)); B operand = the same k of X row xr*32 + lane
  auto xm_tile = [&](int xr) {
    f32x16 o = zero16();
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      const bf16x8 ah = lds_tr_a<8>(Ms[0], 16 * st, dt * 32);
      const bf16x8 al = lds_tr_a<8>(Ms[1], 16 * st, dt * 32);
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
  if (hasB) {
    // B's own first step: emit to QS slot A - cb, then X_B <- X_B Hc_A (if an emit follows)
    emit(ws.qs + (((int64_t)bhq * PR + (A - cb)) * T) * 64 + (int64_t)A * PC * 64, ws.lo_qs, 64, 1);
    if (nsteps > 0) {
      mload(-1);
      mstore();
      __syncthreads();
      if (nsteps > 1) mload(0);
      const f32x16 o = xm_tile(rt + 2);
      __syncthreads();
#pragma unroll
      for (int e = 0; e < 16; ++e) X[(rt + 2) * 32 + l32][dt * 32 + drow(e, g)] = o[e];
      if (nsteps > 1) mstore();
      __syncthreads();
    }
  } else if (nsteps > 1) {
    mload(0);
    mstore();
    __syncthreads();
  }
  const int nblk = hasB ? 2 : 1;
  for (int j = 0; j < nsteps; ++j) {
    emit(slot(j), (j < nq) ? ws.lo_qs : ws.lo_qb, 0, nblk);
    if (j + 1 == nsteps) break;
    if (j + 2 < nsteps) mload(j + 1);
    const f32x16 o0 = xm_tile(rt);
    f32x16 o1 = zero16();
    if (hasB) o1 = xm_tile(rt + 2);
    __syncthreads();
#pragma unroll
    for (int e = 0; e < 16; ++e) X[rt * 32 + l32][dt * 32 + drow(e, g)] = o0[e];
    if (hasB) {
#pragma unroll
      for (int e = 0; e < 16; ++e) X[(rt + 2) * 32 + l32][dt * 32 + drow(e, g)] = o1[e];
    }
    if (j + 2 < nsteps) mstore();
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// Chained solve (triangular_solve_fwd.py:99-225) per query head; one workgroup per
// pair of 64-row chunks A = 2p, B = 2p + 1 (one large chunk holds both); ids grow
// with p, so every wait is on a lower id.  counters[bhq] = number of chunks of O
// published (two at a time).
// The earlier key chunks are swept in pairs (J = 2pp, 2pp + 1, one large chunk), one
// barrier per pair, the next pair staged by direct global->LDS loads while this one
// is processed.  wave w: ih = w & 1 -> the rows of chunk A (ih = 0) or B (two 32-row
// n-tiles, lane <-> row), kh = w >> 1 -> key chunk 2pp + kh of every staged pair:
//   S^T[j][i] = Kop_J . Qop_I, L = exp(s S - 1/s), acc^T[d][i] += O^T[d][j] L^T[j][i]
// (the kh = 0 accumulators start at -V^T).  Then O_A = Y_A R_A and
// O_B = Y_B (R_B - L_BA O_A), R = V - acc, Y = (I + L_diag)^-1 applied through a 3-term
// bf16 split.  L_BA depends on the key operands only and is computed before the sweep.
// The fp32 buffers of the final step reuse the staging space.
// ---------------------------------------------------------------------------
// NP: bf16 planes per operand (2: fp32 inputs, hi and lo)
template <int KD, int NP>
struct SolveFwdSmem {
  union {
    struct {
      bf16 k[2][2][NP][64 * KD];  // [buffer][chunk of the pair][plane], swizzled (chunk c of row r at c ^ (r & 7))
      bf16 o[2][2][NP][KD * 64];
    } st;
    struct {
      float Rt[KD][132];    // R^T for the 128 rows (0..63 = A, 64..127 = B)
      float Ys[64][68];     // Y of the chunk being solved
      bf16 ot[NP][KD][128 + 8];  // O^T of both chunks, T-perm within 16-groups
    } fin;
  } u;
  bf16x8 lba[4][64][2 * NP];  // L_BA as MFMA B operands, per wave and lane ([2 + h]: lo)
};

// F32: fp32 V and O; every operand product is a 3-term split over hi / lo planes (mm3)
template <int KD, bool F32>
__global__ __launch_bounds__(256) LUCID_TWO_WAVES_IF(KD == 64 && !F32) void path_solve_fwd_kernel(
    const pin_t<F32>* __restrict__ v, Strides vs, pin_t<F32>* __restrict__ o, Strides os, int HQ, int H, int T, int BHq,
    float scale, PathFwdWs ws) {
  constexpr int NKS = KD / 16, NVT = KD / 32;  // k-steps of a logit product, 32-column value tiles
  constexpr int NP = F32 ? 2 : 1;
  __shared__ __attribute__((aligned(16))) SolveFwdSmem<KD, NP> sm;
  const int NT = T / PC, NS = (NT + PR - 1) / PR;
  const int id = blockIdx.x;
  const int p = id / BHq, bhq = id - (id / BHq) * BHq;
  const int G = HQ / H;
  const int b = bhq / HQ, hq = bhq - b * HQ, h = hq / G, bh = b * H + h;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 5, l32 = lane & 31;
  const int ih = w & 1, kh = w >> 1;
  const int A = 2 * p;
  const bool hasB = A + 1 < NT;
  const int cb = (A / PR) * PR;  // first chunk of the large chunk holding A and B
  const int i0 = A * PC;
  int* cnt = ws.counters + bhq;
  const float sl2 = scale * LOG2E_F, cc0 = LOG2E_F / scale;
  const bf16* oTh = ws.oT + (int64_t)bhq * KD * T;
  const int npair = p;  // key chunks 0 .. A - 1
  // this wave's rows (chunk A or B); a missing chunk B reads chunk A's rows, unused
  const bool myrows = ih == 0 || hasB;
  const int r0 = i0 + (myrows ? ih * 64 : 0);

  // accumulators: -V^T for the kh = 0 waves (R = V - acc = -(acc_0 + acc_1)), zero for the others
  f32x16 acc[NVT][2];
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    const pin_t<F32>* vrow = v + b * vs.b + h * vs.h + (int64_t)(r0 + nt * 32 + l32) * vs.t;
#pragma unroll
    for (int t = 0; t < NVT; ++t)
#pragma unroll
      for (int qq = 0; qq < 4; ++qq) {
        float vv[4];
        if constexpr (F32) {
          const f32x4 x = *reinterpret_cast<const f32x4*>(vrow + t * 32 + 8 * qq + 4 * g);
#pragma unroll
          for (int u = 0; u < 4; ++u) vv[u] = x[u];
        } else {
          const bf16x4 x = *reinterpret_cast<const bf16x4*>(vrow + t * 32 + 8 * qq + 4 * g);
#pragma unroll
          for (int u = 0; u < 4; ++u) vv[u] = (float)x[u];
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) acc[t][nt][4 * qq + u] = kh ? 0.f : -vv[u];
      }
  }
  // query operand of key chunk J for this wave's rows: QB^(J/PR) below the large chunk,
  // QS slot J - cb inside it
  auto qbase = [&](int J) {
    return (J < cb) ? ws.qb + ((int64_t)bhq * NS + J / PR) * T * KD : ws.qs + ((int64_t)bhq * PR + (J - cb)) * T * KD;
  };
  auto qlo = [&](int J) { return (J < cb) ? ws.lo_qb : ws.lo_qs; };  // lo plane offset of qbase(J)
  // L_BA (rows of B half nb, keys of A half ka): Kop_A = k~_A, Qop = QS slot A - cb of B's rows
  if (hasB) {
    const int nb = w & 1, ka = w >> 1;
    const bf16* kr = ws.kt + ((int64_t)bh * T + i0 + ka * 32 + l32) * KD;
    const bf16* qr = qbase(A) + (int64_t)(i0 + 64 + nb * 32 + l32) * KD;
    f32x16 sc = zero16();
#pragma unroll
    for (int st = 0; st < NKS; ++st) {
      bf16x8 ka8[NP], qa8[NP];
      ka8[0] = ld8(kr + 16 * st + 8 * g);
      qa8[0] = ld8(qr + 16 * st + 8 * g);
      if constexpr (F32) {
        ka8[1] = ld8(kr + ws.lo_kt + 16 * st + 8 * g);
        qa8[1] = ld8(qr + ws.lo_qs + 16 * st + 8 * g);
      }
      sc = mm3<NP>(ka8, qa8, sc);
    }
#pragma unroll
    for (int e = 0; e < 16; ++e) sc[e] = __builtin_amdgcn_exp2f(fmaf(sc[e], sl2, -cc0));
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      sm.lba[w][lane][hh] = pack_b(sc, hh);
      if constexpr (F32) sm.lba[w][lane][2 + hh] = pack_lo(sc, hh, sm.lba[w][lane][hh]);
    }
  }
  // below the large chunk the operand changes only every PR key chunks, so it stays in
  // registers across pairs; inside it every chunk has its own slot
  bf16x8 qop[2][NKS][NP];
  int qsrc = -1;
  auto load_q = [&](int J) {
    const int src = (J < cb) ? J / PR : NS + J;
    if (src == qsrc) return;
    qsrc = src;
    const bf16* base = qbase(J);
    const int64_t lo = qlo(J);
#pragma unroll
    for (int nt = 0; nt < 2; ++nt)
#pragma unroll
      for (int st = 0; st < NKS; ++st) {
        const bf16* p = base + (int64_t)(r0 + nt * 32 + l32) * KD + 16 * st + 8 * g;
        qop[nt][st][0] = ld8(p);
        if constexpr (F32) qop[nt][st][1] = ld8(p + lo);
      }
  };
  int plan_k[64 * (KD / 8) / 256], plan_t[KD * 8 / 256];
  dma_plan<64, KD / 8>(KD, plan_k);
  dma_plan<KD, 8>(T, plan_t);
  auto stage = [&](int pp) {  // key chunks 2pp, 2pp + 1 into buffer pp & 1
    const int buf = pp & 1;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int J = 2 * pp + u;
      const bf16* kp = ((J < cb) ? ws.kl : ws.kt) + ((int64_t)bh * T + J * PC) * KD;
      dma_stage<64, KD / 8>(plan_k, kp, sm.u.st.k[buf][u][0]);
      dma_stage<KD, 8>(plan_t, oTh + J * PC, sm.u.st.o[buf][u][0]);
      if constexpr (F32) {
        dma_stage<64, KD / 8>(plan_k, kp + ((J < cb) ? ws.lo_kl : ws.lo_kt), sm.u.st.k[buf][u][1]);
        dma_stage<KD, 8>(plan_t, oTh + ws.lo_oT + J * PC, sm.u.st.o[buf][u][1]);
      }
    }
  };
  // Y_A, Y_B (fp32) are fetched into registers during the last pair
  f32x4 yr[8];
  auto yload = [&]() {
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int c = u >> 2;
      if (c == 0 || hasB)
        yr[u] = *reinterpret_cast<const f32x4*>(ws.y + ((int64_t)bhq * NT + A + c) * 4096 + 4 * (tid + 256 * (u & 3)));
    }
  };
  auto ystore = [&](int c) {
#pragma unroll
    for (int u = 4 * c; u < 4 * c + 4; ++u) {
      const int f = 4 * (tid + 256 * (u & 3));
      *reinterpret_cast<f32x4*>(&sm.u.fin.Ys[f >> 6][f & 63]) = yr[u];
    }
  };
  auto sweep_pair = [&](int buf) {
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      bf16x8 ka[NKS][NP];
#pragma unroll
      for (int st = 0; st < NKS; ++st)
#pragma unroll
        for (int pl = 0; pl < NP; ++pl) ka[st][pl] = ld8(swz<KD / 8>(sm.u.st.k[buf][kh][pl], mt * 32 + l32, 2 * st + g));
      bf16x8 pb[2][2][NP];
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) {
        f32x16 sc = zero16();
#pragma unroll
        for (int st = 0; st < NKS; ++st) sc = mm3<NP>(ka[st], qop[nt][st], sc);
#pragma unroll
        for (int e = 0; e < 16; ++e) sc[e] = __builtin_amdgcn_exp2f(fmaf(sc[e], sl2, -cc0));
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          pb[nt][hh][0] = pack_b(sc, hh);
          if constexpr (F32) pb[nt][hh][1] = pack_lo(sc, hh, pb[nt][hh][0]);
        }
      }
#pragma unroll
      for (int t = 0; t < NVT; ++t) {
        bf16x8 va[2][NP];
#pragma unroll
        for (int pl = 0; pl < NP; ++pl) {
          va[0][pl] = ld8(swz<8>(sm.u.st.o[buf][kh][pl], t * 32 + l32, 4 * mt + g));
          va[1][pl] = ld8(swz<8>(sm.u.st.o[buf][kh][pl], t * 32 + l32, 4 * mt + 2 + g));
        }
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
          acc[t][nt] = mm3<NP>(va[0], pb[nt][0], acc[t][nt]);
          acc[t][nt] = mm3<NP>(va[1], pb[nt][1], acc[t][nt]);
        }
      }
    }
  };
  int ready = 0;
  if (npair > 0) {
    ready = wait_counter_gt(cnt, 1);
    stage(0);
    dma_wait();
  } else {
    yload();
  }
  __syncthreads();
  for (int pp = 0; pp < npair; ++pp) {
    const bool more = pp + 1 < npair;
    // the query operand is loaded before the next pair's staging so that waiting for
    // it does not wait for the staging loads
    load_q(2 * pp + kh);
    bool early = false;
    if (more) {
      const int nd = 2 * pp + 3;  // pair pp + 1 is complete once the counter exceeds this
      if (nd >= ready) {
        const int seen = poll_counter(cnt);
        if (seen > nd) {
          chain_acquire();
          ready = seen;
        }
      }
      early = nd < ready;
      if (early) stage(pp + 1);
    } else {
      yload();  // fetch Y_A, Y_B while the last pair is processed
    }
    sweep_pair(pp & 1);
    if (more && !early) {
      ready = wait_counter_gt(cnt, 2 * pp + 3);
      stage(pp + 1);
    }
    dma_wait();
    __syncthreads();
  }
  // ---- R^T = -(acc_0 + acc_1) (Rt columns = rows of the workgroup); Y_A to LDS ----
  float(*Rt)[132] = sm.u.fin.Rt;
  if (kh == 1 && myrows) {
#pragma unroll
    for (int t = 0; t < NVT; ++t)
#pragma unroll
      for (int nt = 0; nt < 2; ++nt)
#pragma unroll
        for (int e = 0; e < 16; ++e) Rt[t * 32 + drow(e, g)][ih * 64 + nt * 32 + l32] = acc[t][nt][e];
  }
  ystore(0);
  __syncthreads();
  if (kh == 0 && myrows) {
#pragma unroll
    for (int t = 0; t < NVT; ++t)
#pragma unroll
      for (int nt = 0; nt < 2; ++nt)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          float& x = Rt[t * 32 + drow(e, g)][ih * 64 + nt * 32 + l32];
          x = -(acc[t][nt][e] + x);
        }
  }
  __syncthreads();
  // O^T[d][r] = sum_c R^T[d][c] Y[r][c] for chunk c (Y lower triangular); wave w -> value
  // tiles dt = w >> 1 (+ 2, + 4 .. at KD > 64), row half rh = w & 1
  auto diag_solve = [&](int c) {
   const int rh = w & 1;
   for (int dt = w >> 1; dt < NVT; dt += 2) {
    f32x16 oo = zero16();
    for (int st = 0; st < (rh ? 4 : 2); ++st) {
      bf16x8 ah, al, bh8, bl;
      split8(&Rt[dt * 32 + l32][c * 64 + 16 * st + 8 * g], ah, al);
      split8(&sm.u.fin.Ys[rh * 32 + l32][16 * st + 8 * g], bh8, bl);
      oo = mfma32(ah, bh8, oo);
      oo = mfma32(ah, bl, oo);
      oo = mfma32(al, bh8, oo);
    }
    const int rl = rh * 32 + l32;
    const int lslot = c * 64 + ((rl & ~15) | jmap(rl & 15));
    pin_t<F32>* orow = o + b * os.b + hq * os.h + (int64_t)(i0 + c * 64 + rl) * os.t;
#pragma unroll
    for (int qq = 0; qq < 4; ++qq) {
      const int d0 = dt * 32 + 8 * qq + 4 * g;
      bf16x4 bb;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        bb[u] = (bf16)oo[4 * qq + u];
        sm.u.fin.ot[0][d0 + u][lslot] = bb[u];
        if constexpr (F32) sm.u.fin.ot[NP - 1][d0 + u][lslot] = (bf16)(oo[4 * qq + u] - (float)bb[u]);
      }
      if constexpr (F32) {
        f32x4 f;
#pragma unroll
        for (int u = 0; u < 4; ++u) f[u] = oo[4 * qq + u];
        *reinterpret_cast<f32x4*>(orow + d0) = f;
      } else {
        *reinterpret_cast<bf16x4*>(orow + d0) = bb;
      }
    }
   }
  };
  diag_solve(0);
  __syncthreads();
  if (hasB) {
    ystore(1);
    // ---- R_B -= L_BA O_A: wave -> (B rows half nb, A keys half ka) ----
    const int nb = w & 1, ka = w >> 1;
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
        bf16x8 oa[NP];
#pragma unroll
        for (int pl = 0; pl < NP; ++pl) oa[pl] = ld8(&sm.u.fin.ot[pl][t * 32 + l32][ka * 32 + 16 * hh + 8 * g]);
        cr[t] = mm3<NP>(oa, lb[hh], cr[t]);
      }
    }
    const int col = 64 + nb * 32 + l32;
    if (ka == 1) {
#pragma unroll
      for (int t = 0; t < NVT; ++t)
#pragma unroll
        for (int e = 0; e < 16; ++e) Rt[t * 32 + drow(e, g)][col] -= cr[t][e];
    }
    __syncthreads();
    if (ka == 0) {
#pragma unroll
      for (int t = 0; t < NVT; ++t)
#pragma unroll
        for (int e = 0; e < 16; ++e) Rt[t * 32 + drow(e, g)][col] -= cr[t][e];
    }
    __syncthreads();
    diag_solve(1);
    __syncthreads();
  }
  // O^T of the workgroup's chunks to the chain operand with 16-byte stores
  const int nch = hasB ? 2 : 1;
  for (int c = tid; c < KD * 8 * nch; c += 256) {
    const int dd = c / (8 * nch), s8 = (c - dd * 8 * nch) * 8;
    bf16* dst = ws.oT + ((int64_t)bhq * KD + dd) * T + i0 + s8;
    *reinterpret_cast<bf16x8*>(dst) = ld8(&sm.u.fin.ot[0][dd][s8]);
    if constexpr (F32) *reinterpret_cast<bf16x8*>(dst + ws.lo_oT) = ld8(&sm.u.fin.ot[NP - 1][dd][s8]);
  }
  publish_counter(cnt, A + nch);
}

// ---------------------------------------------------------------------------
// PaTH softmax attention forward: the in-chunk pass of intra_chunk_preprocess_fwd.py:71-115
// and the inter-chunk online softmax of parallel_path_fwd.py:54-124 in one kernel, on the
// same two-level logit blocks as the solve above:
//   O_i = sum_{j <= i} exp2(s' A_ij - lse_i) v_j,  s' = s log2(e)
// Per group of four query chunks I1 = 4p .. I1 + 3 (one large chunk); wave w owns chunk
// Iw = I1 + w (two 32-row n-tiles, lane <-> row, both lane halves hold the same row and
// half of the keys), so every staged key tile serves 256 rows.  The diagonal block reads
// the in-chunk logits; key chunks J < Iw give S^T[j][i] = Kop_J . Qop_I^(J).
// O^T[d][i] += V^T[d][j] P^T[j][i] with V^T from transposing LDS reads.  Key-operand and V
// rows are staged by direct global->LDS loads (double buffered).  The row log-sum-exp
// (exp2 domain) is kept for the backward.  grid (B*HQ, ceil(NT/4)), the groups with the
// most key chunks (of all heads) first.
// ---------------------------------------------------------------------------
template <int KD, int NP>
struct SoftmaxFwdSmem {
  bf16 k[2][NP][64 * KD];   // [buffer][plane], swizzled (chunk c of row r at c ^ (r & 7))
  bf16 v[2][NP][64 * KD];
  bf16 vd[4][NP][64 * KD];  // V rows of the group's own chunks (diagonal blocks)
};

// KD: head dim (64 or 128).  F32: v is the hi plane of a split fp32 V (lo plane at v + v_lo),
// o is fp32, and every product is a 3-term split (mm3)
template <int KD, bool F32>
__global__ __launch_bounds__(256) LUCID_TWO_WAVES_IF(KD == 64 && !F32) void path_softmax_fwd_kernel(
    const bf16* __restrict__ v, Strides vs, int64_t v_lo, pin_t<F32>* __restrict__ o, Strides os, int HQ, int H, int T,
    float scale, PathFwdWs ws) {
  constexpr int NKS = KD / 16, NVT = KD / 32, CPR = KD / 8;  // k-steps, 32-column tiles, 16-byte chunks per row
  constexpr int NP = F32 ? 2 : 1;
  __shared__ __attribute__((aligned(16))) SoftmaxFwdSmem<KD, NP> sm;
  const int NT = T / PC, NS = (NT + PR - 1) / PR, NQ = (NT + 3) / 4;
  const int I1 = 4 * (NQ - 1 - (int)blockIdx.y), bhq = blockIdx.x;  // heaviest groups of all heads first
  const int G_ = HQ / H;
  const int b = bhq / HQ, hq = bhq - b * HQ, h = hq / G_, bh = b * H + h;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 5, l32 = lane & 31;
  const int Iw = I1 + w;
  const bool live = Iw < NT;
  const int sI = I1 / PR, cb = sI * PR;
  const int iw0 = min(Iw, NT - 1) * PC;         // first row of this wave
  const int nJ = min(I1 + 3, NT - 1);           // key tiles needed by the group
  const float sl2 = scale * LOG2E_F;
  const bf16* vh = v + b * vs.b + h * vs.h;

  int plan_k[64 * CPR / 256], plan_v[64 * CPR / 256];
  dma_plan<64, CPR>(KD, plan_k);
  dma_plan<64, CPR>(vs.t, plan_v);
  auto stage = [&](int J) {
    const int buf = J & 1;
    const bf16* kp = ((J < cb) ? ws.kl : ws.kt) + ((int64_t)bh * T + J * PC) * KD;
    dma_stage<64, CPR>(plan_k, kp, sm.k[buf][0]);
    dma_stage<64, CPR>(plan_v, vh + (int64_t)J * PC * vs.t, sm.v[buf][0]);
    if constexpr (F32) {
      dma_stage<64, CPR>(plan_k, kp + ((J < cb) ? ws.lo_kl : ws.lo_kt), sm.k[buf][1]);
      dma_stage<64, CPR>(plan_v, vh + v_lo + (int64_t)J * PC * vs.t, sm.v[buf][1]);
    }
  };
#pragma unroll
  for (int c = 0; c < 4; ++c)
    if (I1 + c < NT) {
#pragma unroll
      for (int pl = 0; pl < NP; ++pl)
        dma_stage<64, CPR>(plan_v, vh + pl * v_lo + (int64_t)(I1 + c) * PC * vs.t, sm.vd[c][pl]);
    }
  if (nJ > 0) stage(0);

  f32x16 acc[2][NVT];
  float m[2] = {0.f, 0.f}, l[2] = {0.f, 0.f};
  dma_wait();
  __syncthreads();
  // the diagonal block first, one n-tile at a time: in-chunk logits of row rl, keys
  // j = 32 jh + drow(e, g); keys j > rl are masked
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
#pragma unroll
    for (int t = 0; t < NVT; ++t) acc[nt][t] = zero16();
    if (!live) continue;
    const int rl = nt * 32 + l32;
    const float* ad = ws.ld + ((int64_t)bhq * NT + Iw) * 4096 + rl * 64;
    f32x16 sd[2];
#pragma unroll
    for (int jh = 0; jh < 2; ++jh)
#pragma unroll
      for (int qq = 0; qq < 4; ++qq) {
        const f32x4 x = *reinterpret_cast<const f32x4*>(ad + jh * 32 + 8 * qq + 4 * g);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int j = jh * 32 + 8 * qq + 4 * g + u;
          sd[jh][4 * qq + u] = (j <= rl) ? x[u] * sl2 : -INFINITY;
        }
      }
    float mx = -INFINITY;
#pragma unroll
    for (int jh = 0; jh < 2; ++jh)
#pragma unroll
      for (int e = 0; e < 16; ++e) mx = fmaxf(mx, sd[jh][e]);
    m[nt] = wave_max32(mx);  // finite: the diagonal key is always present
#pragma unroll
    for (int jh = 0; jh < 2; ++jh) {
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        sd[jh][e] = __builtin_amdgcn_exp2f(sd[jh][e] - m[nt]);
        l[nt] += sd[jh][e];
      }
      bf16x8 p[2][NP];
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        p[hh][0] = pack_b(sd[jh], hh);
        if constexpr (F32) p[hh][1] = pack_lo(sd[jh], hh, p[hh][0]);
      }
#pragma unroll
      for (int t = 0; t < NVT; ++t)
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          bf16x8 va[NP];
#pragma unroll
          for (int pl = 0; pl < NP; ++pl) va[pl] = lds_tr_a<CPR>(sm.vd[w][pl], jh * 32 + 16 * hh, t * 32);
          acc[nt][t] = mm3<NP>(va, p[hh], acc[nt][t]);
        }
    }
  }
  bf16x8 qb[2][NKS][NP];
  for (int J = 0; J < nJ; ++J) {
    const int buf = J & 1;
    if (J + 1 < nJ) stage(J + 1);
    if (J >= cb || J % PR == 0) {  // the query operand changes
      const bf16* qsrc = (J < cb) ? ws.qb + ((int64_t)bhq * NS + J / PR) * T * KD
                                  : ws.qs + ((int64_t)bhq * PR + (J - cb)) * T * KD;
      const int64_t qlo = (J < cb) ? ws.lo_qb : ws.lo_qs;
#pragma unroll
      for (int nt = 0; nt < 2; ++nt)
#pragma unroll
        for (int st = 0; st < NKS; ++st) {
          const bf16* p = qsrc + (int64_t)(iw0 + nt * 32 + l32) * KD + 16 * st + 8 * g;
          qb[nt][st][0] = ld8(p);
          if constexpr (F32) qb[nt][st][1] = ld8(p + qlo);
        }
    }
    if (live && J < Iw) {
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) {
        f32x16 sc[2];
#pragma unroll
        for (int jh = 0; jh < 2; ++jh) {
          sc[jh] = zero16();
#pragma unroll
          for (int st = 0; st < NKS; ++st) {
            bf16x8 ka[NP];
#pragma unroll
            for (int pl = 0; pl < NP; ++pl) ka[pl] = ld8(swz<CPR>(sm.k[buf][pl], jh * 32 + l32, 2 * st + g));
            sc[jh] = mm3<NP>(ka, qb[nt][st], sc[jh]);
          }
        }
        float mx = -INFINITY;
#pragma unroll
        for (int jh = 0; jh < 2; ++jh)
#pragma unroll
          for (int e = 0; e < 16; ++e) mx = fmaxf(mx, sc[jh][e]);
        mx = wave_max32(mx);
        const float mn = fmaxf(m[nt], mx * sl2);
        const float alpha = __builtin_amdgcn_exp2f(m[nt] - mn);
        m[nt] = mn;
        l[nt] *= alpha;
#pragma unroll
        for (int t = 0; t < NVT; ++t)
#pragma unroll
          for (int e = 0; e < 16; ++e) acc[nt][t][e] *= alpha;
#pragma unroll
        for (int jh = 0; jh < 2; ++jh) {
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            sc[jh][e] = __builtin_amdgcn_exp2f(fmaf(sc[jh][e], sl2, -mn));
            l[nt] += sc[jh][e];
          }
          bf16x8 p[2][NP];
#pragma unroll
          for (int hh = 0; hh < 2; ++hh) {
            p[hh][0] = pack_b(sc[jh], hh);
            if constexpr (F32) p[hh][1] = pack_lo(sc[jh], hh, p[hh][0]);
          }
#pragma unroll
          for (int t = 0; t < NVT; ++t)
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
              bf16x8 va[NP];
#pragma unroll
              for (int pl = 0; pl < NP; ++pl) va[pl] = lds_tr_a<CPR>(sm.v[buf][pl], jh * 32 + 16 * hh, t * 32);
              acc[nt][t] = mm3<NP>(va, p[hh], acc[nt][t]);
            }
        }
      }
    }
    dma_wait();
    __syncthreads();
  }
  if (live) {
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      const float ls = wave_sum32(l[nt]);
      const float inv = 1.f / ls;
      const int i = iw0 + nt * 32 + l32;
      pin_t<F32>* orow = o + b * os.b + hq * os.h + (int64_t)i * os.t;
#pragma unroll
      for (int t = 0; t < NVT; ++t)
#pragma unroll
        for (int qq = 0; qq < 4; ++qq) {
          if constexpr (F32) {
            f32x4 f;
#pragma unroll
            for (int u = 0; u < 4; ++u) f[u] = acc[nt][t][4 * qq + u] * inv;
            *reinterpret_cast<f32x4*>(orow + t * 32 + 8 * qq + 4 * g) = f;
          } else {
            bf16x4 bb;
#pragma unroll
            for (int u = 0; u < 4; ++u) bb[u] = (bf16)(acc[nt][t][4 * qq + u] * inv);
            *reinterpret_cast<bf16x4*>(orow + t * 32 + 8 * qq + 4 * g) = bb;
          }
        }
      if (g == 0) ws.lse[(int64_t)bhq * T + i] = m[nt] + log2f(ls);
    }
  }
}

// ---------------------------------------------------------------------------
// k_cache_j = keys carried to the sequence end (prepare_k_cache.py:12-74):
// x = KL_J; x <- x HL_s^T for every later large chunk.  grid (NT, B*H)
// ---------------------------------------------------------------------------
template <bool F32>
__global__ __launch_bounds__(256) void path_kcache_kernel(int T, pin_t<F32>* __restrict__ kc, Strides kcs, int H,
                                                          PathFwdWs ws) {
  __shared__ __attribute__((aligned(16))) float X[64][68];
  __shared__ __attribute__((aligned(16))) float MT[64][68];
  const int J = blockIdx.x, bh = blockIdx.y;
  const int b = bh / H, h = bh - b * H;
  const int NT = T / PC, NS = (NT + PR - 1) / PR;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, g = lane >> 5, l32 = lane & 31;
  if constexpr (F32)
    load_rows64_split(X, ws.kl + ((int64_t)bh * T + J * PC) * 64, 64, ws.lo_kl);
  else
    load_rows64_f32(X, ws.kl + ((int64_t)bh * T + J * PC) * 64, 64);
  __syncthreads();
  for (int s = J / PR + 1; s < NS; ++s) {
    load_mat64<false>(MT, ws.hl + ((int64_t)bh * NS + s) * 4096);  // (HL^T)^T = HL
    __syncthreads();
    const int dt = w >> 1, rt = w & 1;
    const f32x16 oo = mat_xM_tile(X, MT, dt, rt);
    __syncthreads();
#pragma unroll
    for (int e = 0; e < 16; ++e) X[rt * 32 + l32][dt * 32 + drow(e, g)] = oo[e];
    __syncthreads();
  }
  const int r = tid >> 2, cc = (tid & 3) * 16;
  pin_t<F32>* dst = kc + b * kcs.b + h * kcs.h + (int64_t)(J * PC + r) * kcs.t + cc;
#pragma unroll
  for (int hh = 0; hh < 2; ++hh) {
    if constexpr (F32) {
#pragma unroll
      for (int q4 = 0; q4 < 2; ++q4)
        *reinterpret_cast<f32x4*>(dst + 8 * hh + 4 * q4) = *reinterpret_cast<const f32x4*>(&X[r][cc + 8 * hh + 4 * q4]);
    } else {
      bf16x8 vv;
#pragma unroll
      for (int e = 0; e < 8; ++e) vv[e] = (bf16)X[r][cc + 8 * hh + e];
      *reinterpret_cast<bf16x8*>(dst + 8 * hh) = vv;
    }
  }
}

}  // namespace lucid
