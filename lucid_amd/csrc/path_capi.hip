// C ABI of the LUCID-Path kernels (declared in include/lucid_path.h).
#include <string>

#include "../../include/lucid_path.h"
#include "path_fwd.hip"
#include "path_wide.hip"  // includes path_bwd.hip
#include "chain_guard.h"
#include "profiling.h"

namespace {

thread_local std::string g_path_error;

int pfail(const std::string& msg) {
  g_path_error = msg;
  return 1;
}

int phip(const char* where) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    g_path_error = std::string(where) + ": " + hipGetErrorString(e);
    return 1000 + (int)e;
  }
  return 0;
}

size_t a256(size_t x) { return (x + 255) & ~size_t(255); }

// First step of the entry points that launch a chain kernel (lucid_path_fwd, lucid_path_bwd):
// set up the bounded waits on this device, report a wait that gave up in an earlier launch.
int pchain_check() {
  std::string what;
  if (int e = chain_guard::setup(&what)) {
    g_path_error = what + ": " + hipGetErrorString((hipError_t)e);
    return 1000 + e;
  }
  if (chain_guard::take_flag()) {
    g_path_error = "a chain wait gave up in an earlier launch (no progress within the wait bound); "
                   "the results of that launch are invalid";
    return 2;
  }
  return 0;
}

// softmax = true: the PaTH softmax layout (row log-sum-exp instead of the solve's
// diagonal inverses and O^T chain operand).  KD: the kernels' head dim (64 or 128): rows
// of KD values, KD x KD transport matrices, C x C (64 x 64) in-chunk matrices.  f32: fp32
// inputs, every bf16 operand buffer followed by its lo plane.
lucid::PathFwdWs carve_path_fwd(void* base, int B, int T, int H, int HQ, size_t* bytes, bool softmax = false,
                                int KD = 64, bool f32 = false) {
  const size_t NP = f32 ? 2 : 1;
  const size_t BH = (size_t)B * H, BHq = (size_t)B * HQ;
  const size_t NT = T / 64, NS = (NT + lucid::PR - 1) / lucid::PR, KK = (size_t)KD * KD;
  lucid::PathFwdWs w{};
  size_t off = 0;
  char* p = static_cast<char*>(base);
  auto take = [&](size_t n) {
    char* r = p ? p + off : nullptr;
    off += a256(n);
    return r;
  };
  w.w2 = reinterpret_cast<float*>(take(BH * T * KD * 4));
  w.hc = reinterpret_cast<float*>(take(BH * NT * KK * 4));
  // a bf16 operand buffer of n elements (and its lo plane, at element offset lo)
  auto take_b = [&](size_t n, int64_t& lo) {
    lo = f32 ? (int64_t)n : 0;
    return reinterpret_cast<bf16*>(take(n * 2 * NP));
  };
  w.kt = take_b(BH * T * KD, w.lo_kt);
  w.suf = reinterpret_cast<float*>(take(BH * NT * KK * 4));
  w.hl = reinterpret_cast<float*>(take(BH * NS * KK * 4));
  w.hcs = reinterpret_cast<bf16*>(take(BH * NT * KK * 2 * 2));
  w.hls = reinterpret_cast<bf16*>(take(BH * NS * KK * 2 * 2));
  w.kl = take_b(BH * T * KD, w.lo_kl);
  w.qt = reinterpret_cast<float*>(take(BHq * T * KD * 4));
  w.ld = reinterpret_cast<float*>(take(BHq * NT * 4096 * 4));
  if (!softmax) w.y = reinterpret_cast<float*>(take(BHq * NT * 4096 * 4));
  w.qs = take_b(BHq * lucid::PR * T * KD, w.lo_qs);
  w.qb = take_b(BHq * NS * T * KD, w.lo_qb);
  if (!softmax) w.oT = take_b(BHq * T * KD, w.lo_oT);
  if (softmax && f32) w.vsp = take_b(BH * T * KD, w.lo_vsp);
  w.counters = reinterpret_cast<int*>(take(BHq * 4));
  if (softmax) w.lse = reinterpret_cast<float*>(take(BHq * T * 4));
  if (bytes) *bytes = off;
  return w;
}

int pcheck(const char* name, const void* p, const int64_t* s) {
  if (!p) return pfail(std::string(name) + " is null");
  if (!s) return pfail(std::string(name) + " strides are null");
  if (reinterpret_cast<uintptr_t>(p) % 16) return pfail(std::string(name) + " must be 16-byte aligned");
  return 0;
}

int pcheck_vec(const char* name, const void* p, const int64_t* s) {
  if (int rc = pcheck(name, p, s)) return rc;
  for (int i = 0; i < 3; ++i)
    if (s[i] % 8) return pfail(std::string(name) + " strides must be multiples of 8 elements");
  return 0;
}

lucid::Strides PS(const int64_t* s) { return lucid::Strides{s[0], s[1], s[2]}; }

lucid::PathBwdWs carve_path_bwd(void* base, int B, int T, int HQ, size_t* bytes, bool softmax = false, int KD = 64,
                                bool f32 = false) {
  const size_t NP = f32 ? 2 : 1;
  const size_t BHq = (size_t)B * HQ;
  const size_t NT = T / 64, NS = (NT + lucid::PR - 1) / lucid::PR, KK = (size_t)KD * KD;
  lucid::PathBwdWs w{};
  size_t off = 0;
  char* p = static_cast<char*>(base);
  auto take = [&](size_t n) {
    char* r = p ? p + off : nullptr;
    off += a256(n);
    return r;
  };
  w.dvf = reinterpret_cast<float*>(take(BHq * T * KD * 4));
  if (!softmax) {
    w.lo_dvb = w.lo_dvT = f32 ? (int64_t)(BHq * T * KD) : 0;
    w.dvb = reinterpret_cast<bf16*>(take(BHq * T * KD * 2 * NP));
    w.dvT = reinterpret_cast<bf16*>(take(BHq * T * KD * 2 * NP));
  }
  w.dad = reinterpret_cast<float*>(take(BHq * NT * 4096 * 4));
  w.dqt = reinterpret_cast<float*>(take(BHq * T * KD * 4));
  w.dkt = reinterpret_cast<float*>(take(BHq * T * KD * 4));
  w.dsuf = reinterpret_cast<float*>(take(BHq * NT * KK * 4));
  w.dhl = reinterpret_cast<float*>(take(BHq * NS * KK * 4));
  w.dhc = reinterpret_cast<float*>(take(BHq * NT * KK * 4));
  w.dq = reinterpret_cast<float*>(take(BHq * T * KD * 4));
  w.dk = reinterpret_cast<float*>(take(BHq * T * KD * 4));
  w.dw = reinterpret_cast<float*>(take(BHq * T * KD * 4));
  w.db = reinterpret_cast<float*>(take(BHq * T * 4));
  w.counters = reinterpret_cast<int*>(take(BHq * 4));
  if (softmax) w.delta = reinterpret_cast<float*>(take(BHq * T * 4));
  if (f32) {  // split copies of the caller's rows the sweeps stage (O, or dO and V)
    w.lo_ysp = (int64_t)(BHq * T * KD);
    w.ysp = reinterpret_cast<bf16*>(take(BHq * T * KD * 2 * 2));
    if (softmax) {
      w.lo_xsp = (int64_t)(BHq * T * KD);
      w.xsp = reinterpret_cast<bf16*>(take(BHq * T * KD * 2 * 2));
    }
  }
  if (bytes) *bytes = off;
  return w;
}

int check_shapes(int B, int T, int H, int HQ, int K) {
  if (B <= 0 || T <= 0 || H <= 0 || HQ <= 0) return pfail("B, T, H and HQ must be positive");
  if (K != 64 && K != 128) return pfail("head_dim must be 64 or 128, got " + std::to_string(K));
  if (T % 64) return pfail("T must be a multiple of 64, got " + std::to_string(T));
  if (HQ % H) return pfail("the number of query heads must be a multiple of the key heads");
  return 0;
}

// shared by both forwards: WY form, large-chunk products, query transport (KD: the kernels'
// head dim; head dim 128 has bf16 kernels only)
template <bool F32>
int launch_front(const void* q, const int64_t* q_strides, const void* k, const int64_t* k_strides,
                 const void* w, const int64_t* w_strides, const void* beta, const int64_t* beta_strides,
                 int B, int T, int H, int HQ, float scale, int softmax, const lucid::PathFwdWs& ws, hipStream_t st,
                 int KD) {
  using TI = lucid::pin_t<F32>;
  const int NT = T / 64, NS = (NT + lucid::PR - 1) / lucid::PR;
  const int BH = B * H, BHq = B * HQ;
  if (KD == 128) {
    LUCID_TIMED_LAUNCH(phip, "path_chunk128_kernel", lucid::path_chunk128_kernel, dim3(NT, BHq), st, (const bf16*)q,
                       PS(q_strides), (const bf16*)k, PS(k_strides), (const bf16*)w, PS(w_strides), (const bf16*)beta,
                       PS(beta_strides), HQ, H, T, scale, softmax, ws);
    LUCID_TIMED_LAUNCH(phip, "path_large128_kernel", lucid::path_large128_kernel, dim3(NS, BH), st, T, ws);
    LUCID_TIMED_LAUNCH(phip, "path_transport128_kernel", lucid::path_transport128_kernel, dim3(BHq, (NT + 1) / 2), st,
                       HQ, H, T, ws);
    return 0;
  }
  LUCID_TIMED_LAUNCH(phip, "path_chunk_kernel", lucid::path_chunk_kernel<F32>, dim3(NT, BHq), st, (const TI*)q,
                     PS(q_strides), (const TI*)k, PS(k_strides), (const TI*)w, PS(w_strides), (const TI*)beta,
                     PS(beta_strides), HQ, H, T, scale, softmax, ws);
  LUCID_TIMED_LAUNCH(phip, "path_large_kernel", lucid::path_large_kernel<F32>, dim3(NS, BH), st, T, ws);
  LUCID_TIMED_LAUNCH(phip, "path_transport_kernel", lucid::path_transport_kernel<F32>, dim3(BHq, (NT + 1) / 2), st, HQ,
                     H, T, ws);
  return 0;
}

// the decode key cache
template <bool F32>
int launch_kcache(void* kcache, const int64_t* kcache_strides, int B, int T, int H, const lucid::PathFwdWs& ws,
                  hipStream_t st, int KD) {
  const int NT = T / 64;
  if (KD == 128) {
    LUCID_TIMED_LAUNCH(phip, "path_kcache128_kernel", lucid::path_kcache128_kernel, dim3(NT, B * H), st, T,
                       (bf16*)kcache, PS(kcache_strides), H, ws);
    return 0;
  }
  LUCID_TIMED_LAUNCH(phip, "path_kcache_kernel", lucid::path_kcache_kernel<F32>, dim3(NT, B * H), st, T,
                     (lucid::pin_t<F32>*)kcache, PS(kcache_strides), H, ws);
  return 0;
}

// fp32 rows [B][T][HH][K] (strides xs) -> bf16 hi / lo planes [B][HH][T][K] at dst, dst + lo
int launch_split(const void* x, const int64_t* xs, bf16* dst, int64_t lo, int B, int HH, int T, int K,
                 hipStream_t st) {
  const int64_t n = (int64_t)T * K / 4;
  LUCID_TIMED_LAUNCH(phip, "path_split_kernel", lucid::path_split_kernel, dim3((unsigned)((n + 255) / 256), B * HH), st,
                     (const float*)x, PS(xs), dst, lo, HH, T, K);
  return 0;
}
lucid::Strides split_strides(int HH, int T, int K) {
  return lucid::Strides{(int64_t)HH * T * K, (int64_t)T * K, (int64_t)K};
}

// the logit-gradient stages shared by both backwards (after dV, dA and the row/column
// sweeps): products, WY backward, GQA reduction
template <bool F32>
int launch_back(const void* q, const int64_t* q_strides, const void* k, const int64_t* k_strides, const void* w,
                const int64_t* w_strides, const void* beta, const int64_t* beta_strides, void* dq,
                const int64_t* dq_strides, void* dk, const int64_t* dk_strides, void* dv, const int64_t* dv_strides,
                void* dw, const int64_t* dw_strides, void* dbeta, const int64_t* dbeta_strides, int B, int T, int H,
                int HQ, const lucid::PathFwdWs& ws, const lucid::PathBwdWs& bw, hipStream_t st, int KD) {
  using TI = lucid::pin_t<F32>;
  const int NT = T / 64, NS = (NT + lucid::PR - 1) / lucid::PR;
  const int BH = B * H, BHq = B * HQ;
  if (KD == 128) {
    LUCID_TIMED_LAUNCH(phip, "path_products_bwd128_kernel", lucid::path_products_bwd128_kernel, dim3(NS, BHq), st, HQ,
                       H, T, ws, bw);
    LUCID_TIMED_LAUNCH(phip, "path_wy_bwd128_kernel", lucid::path_wy_bwd128_kernel, dim3(NT, BHq), st, (const bf16*)q,
                       PS(q_strides), (const bf16*)k, PS(k_strides), (const bf16*)w, PS(w_strides), (const bf16*)beta,
                       PS(beta_strides), HQ, H, T, ws, bw);
  } else {
    LUCID_TIMED_LAUNCH(phip, "path_products_bwd_kernel", lucid::path_products_bwd_kernel, dim3(NS, BHq), st, HQ, H, T,
                       ws, bw);
    LUCID_TIMED_LAUNCH(phip, "path_wy_bwd_kernel", lucid::path_wy_bwd_kernel<F32>, dim3(NT, BHq), st, (const TI*)q,
                       PS(q_strides), (const TI*)k, PS(k_strides), (const TI*)w, PS(w_strides), (const TI*)beta,
                       PS(beta_strides), HQ, H, T, ws, bw);
  }
  LUCID_TIMED_LAUNCH(phip, "path_reduce_kernel", lucid::path_reduce_kernel<F32>, dim3((T + 3) / 4, BH), st, HQ, H, T,
                     KD, bw, (TI*)dq, PS(dq_strides), (TI*)dk, PS(dk_strides), (TI*)dv, PS(dv_strides), (TI*)dw,
                     PS(dw_strides), (TI*)dbeta, PS(dbeta_strides));
  return 0;
}

// kernels' head dim for a call: 64, or 128 above 64 (bf16 only)
int path_kd(int K) { return K > 64 ? 128 : 64; }

// LUCID-Path (softmax = 0) or PaTH softmax (softmax = 1) forward; F32: fp32 tensors
template <bool F32>
int path_fwd_impl(int softmax, const void* q, const int64_t* q_strides, const void* k, const int64_t* k_strides,
                  const void* v, const int64_t* v_strides, const void* w, const int64_t* w_strides, const void* beta,
                  const int64_t* beta_strides, void* o, const int64_t* o_strides, void* kcache,
                  const int64_t* kcache_strides, void* fwd_ws, int B, int T, int H, int HQ, int K, float scale,
                  void* stream) {
  using TI = lucid::pin_t<F32>;
  g_path_error.clear();
  if (int rc = check_shapes(B, T, H, HQ, K)) return rc;
  if (F32 && K != 64) return pfail("fp32 inputs run at head_dim 64 (smaller head dims zero-padded), got " +
                                   std::to_string(K));
  if (int rc = pcheck_vec("q", q, q_strides)) return rc;
  if (int rc = pcheck_vec("k", k, k_strides)) return rc;
  if (int rc = pcheck_vec("v", v, v_strides)) return rc;
  if (int rc = pcheck_vec("w", w, w_strides)) return rc;
  if (int rc = pcheck("beta", beta, beta_strides)) return rc;
  if (int rc = pcheck_vec("o", o, o_strides)) return rc;
  if (kcache)
    if (int rc = pcheck_vec("kcache", kcache, kcache_strides)) return rc;
  if (!fwd_ws) return pfail("fwd_ws is null");
  if (reinterpret_cast<uintptr_t>(fwd_ws) % 256) return pfail("fwd_ws must be 256-byte aligned");
  if (!softmax)
    if (int rc = pchain_check()) return rc;
  const lucid::PathFwdWs ws = carve_path_fwd(fwd_ws, B, T, H, HQ, nullptr, softmax != 0, K, F32);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int NT = T / 64;
  const int BHq = B * HQ;
  if (int rc = launch_front<F32>(q, q_strides, k, k_strides, w, w_strides, beta, beta_strides, B, T, H, HQ, scale,
                                 softmax, ws, st, K))
    return rc;
  if (!softmax) {
    if (K == 128)
      LUCID_TIMED_LAUNCH(phip, "path_solve_fwd_kernel", (lucid::path_solve_fwd_kernel<128, false>),
                         dim3(((NT + 1) / 2) * BHq), st, (const bf16*)v, PS(v_strides), (bf16*)o, PS(o_strides), HQ,
                         H, T, BHq, scale, ws);
    else
      LUCID_TIMED_LAUNCH(phip, "path_solve_fwd_kernel", (lucid::path_solve_fwd_kernel<64, F32>),
                         dim3(((NT + 1) / 2) * BHq), st, (const TI*)v, PS(v_strides), (TI*)o, PS(o_strides), HQ, H, T,
                         BHq, scale, ws);
  } else {
    const bf16* vv = (const bf16*)v;
    lucid::Strides vst = PS(v_strides);
    int64_t vlo = 0;
    if (F32) {
      if (int rc = launch_split(v, v_strides, ws.vsp, ws.lo_vsp, B, H, T, K, st)) return rc;
      vv = ws.vsp;
      vst = split_strides(H, T, K);
      vlo = ws.lo_vsp;
    }
    if (K == 128)
      LUCID_TIMED_LAUNCH(phip, "path_softmax_fwd_kernel", (lucid::path_softmax_fwd_kernel<128, false>),
                         dim3(BHq, (NT + 3) / 4), st, vv, vst, vlo, (bf16*)o, PS(o_strides), HQ, H, T, scale, ws);
    else
      LUCID_TIMED_LAUNCH(phip, "path_softmax_fwd_kernel", (lucid::path_softmax_fwd_kernel<64, F32>),
                         dim3(BHq, (NT + 3) / 4), st, vv, vst, vlo, (TI*)o, PS(o_strides), HQ, H, T, scale, ws);
  }
  if (kcache)
    if (int rc = launch_kcache<F32>(kcache, kcache_strides, B, T, H, ws, st, K)) return rc;
  return 0;
}

// the row and column sweeps of one backward at head dim KD
template <bool SM, int KD, bool F32>
int launch_sweeps(const bf16* x, lucid::Strides xs, int64_t x_lo, const bf16* y, lucid::Strides ys, int64_t y_lo,
                  int B, int T, int HQ, int H, float scale, const lucid::PathFwdWs& ws, const lucid::PathBwdWs& bw,
                  hipStream_t st) {
  const int NT = T / 64, BHq = B * HQ;
  LUCID_TIMED_LAUNCH(phip, SM ? "path_softmax_bwd_row_kernel" : "path_bwd_row_kernel",
                     (lucid::path_bwd_row_kernel<SM, KD, F32>), dim3(BHq, (NT + 1) / 2), st, x, xs, x_lo, y, ys, y_lo,
                     HQ, H, T, scale, ws, bw);
  LUCID_TIMED_LAUNCH(phip, SM ? "path_softmax_bwd_col_kernel" : "path_bwd_col_kernel",
                     (lucid::path_bwd_col_kernel<SM, KD, F32>), dim3(BHq, (NT + 1) / 2), st, x, xs, x_lo, y, ys, y_lo,
                     HQ, H, T, scale, ws, bw);
  return 0;
}

// LUCID-Path (softmax = 0; v unused) or PaTH softmax (softmax = 1) backward; F32: fp32 tensors
template <bool F32>
int path_bwd_impl(int softmax, const void* dout, const int64_t* do_strides, const void* q, const int64_t* q_strides,
                  const void* k, const int64_t* k_strides, const void* v, const int64_t* v_strides, const void* w,
                  const int64_t* w_strides, const void* beta, const int64_t* beta_strides, const void* o,
                  const int64_t* o_strides, const void* fwd_ws, void* dq, const int64_t* dq_strides, void* dk,
                  const int64_t* dk_strides, void* dv, const int64_t* dv_strides, void* dw, const int64_t* dw_strides,
                  void* dbeta, const int64_t* dbeta_strides, void* bwd_ws, int B, int T, int H, int HQ, int K,
                  float scale, void* stream) {
  using TI = lucid::pin_t<F32>;
  g_path_error.clear();
  if (int rc = check_shapes(B, T, H, HQ, K)) return rc;
  if (F32 && K != 64) return pfail("fp32 inputs run at head_dim 64 (smaller head dims zero-padded), got " +
                                   std::to_string(K));
  if (int rc = pcheck_vec("dout", dout, do_strides)) return rc;
  if (int rc = pcheck_vec("q", q, q_strides)) return rc;
  if (int rc = pcheck_vec("k", k, k_strides)) return rc;
  if (softmax)
    if (int rc = pcheck_vec("v", v, v_strides)) return rc;
  if (int rc = pcheck_vec("w", w, w_strides)) return rc;
  if (int rc = pcheck("beta", beta, beta_strides)) return rc;
  if (int rc = pcheck_vec("o", o, o_strides)) return rc;
  if (int rc = pcheck("dq", dq, dq_strides)) return rc;
  if (int rc = pcheck("dk", dk, dk_strides)) return rc;
  if (int rc = pcheck("dv", dv, dv_strides)) return rc;
  if (int rc = pcheck("dw", dw, dw_strides)) return rc;
  if (int rc = pcheck("dbeta", dbeta, dbeta_strides)) return rc;
  if (!fwd_ws || !bwd_ws) return pfail("fwd_ws and bwd_ws must be non-null");
  if (reinterpret_cast<uintptr_t>(fwd_ws) % 256 || reinterpret_cast<uintptr_t>(bwd_ws) % 256)
    return pfail("fwd_ws and bwd_ws must be 256-byte aligned");
  if (!softmax)
    if (int rc = pchain_check()) return rc;
  const lucid::PathFwdWs ws = carve_path_fwd(const_cast<void*>(fwd_ws), B, T, H, HQ, nullptr, softmax != 0, K, F32);
  const lucid::PathBwdWs bw = carve_path_bwd(bwd_ws, B, T, HQ, nullptr, softmax != 0, K, F32);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int NT = T / 64, NS = (NT + lucid::PR - 1) / lucid::PR;
  const int BHq = B * HQ;
  const int64_t n_hl = (int64_t)BHq * NS * K * K, n_hc = (int64_t)BHq * NT * K * K;
  LUCID_TIMED_LAUNCH(phip, "path_bwd_zero_kernel", lucid::path_bwd_zero_kernel, dim3(1024), st, n_hl, n_hc, BHq, bw);
  if (!softmax) {
    // X = dV rows (workspace), Y = O rows (the caller's, or their split copy)
    const lucid::Strides dvs = split_strides(HQ, T, K);  // dV rows [B][HQ][T][K]
    const bf16* yo = (const bf16*)o;
    lucid::Strides ys = PS(o_strides);
    if (F32) {
      if (int rc = launch_split(o, o_strides, bw.ysp, bw.lo_ysp, B, HQ, T, K, st)) return rc;
      yo = bw.ysp;
      ys = split_strides(HQ, T, K);
    }
    if (K == 128) {
      LUCID_TIMED_LAUNCH(phip, "path_dv_kernel", (lucid::path_dv_kernel<128, false>), dim3(((NT + 1) / 2) * BHq), st,
                         (const bf16*)dout, PS(do_strides), (const bf16*)o, PS(o_strides), HQ, H, T, BHq, scale, ws,
                         bw);
      if (int rc = launch_sweeps<false, 128, false>(bw.dvb, dvs, 0, yo, ys, 0, B, T, HQ, H, scale, ws, bw, st))
        return rc;
    } else {
      LUCID_TIMED_LAUNCH(phip, "path_dv_kernel", (lucid::path_dv_kernel<64, F32>), dim3(((NT + 1) / 2) * BHq), st,
                         (const TI*)dout, PS(do_strides), (const TI*)o, PS(o_strides), HQ, H, T, BHq, scale, ws, bw);
      if (int rc = launch_sweeps<false, 64, F32>(bw.dvb, dvs, bw.lo_dvb, yo, ys, bw.lo_ysp, B, T, HQ, H, scale, ws,
                                                 bw, st))
        return rc;
    }
  } else {
    // X = dO rows, Y = V rows (the caller's, or their split copies)
    const bf16* xd = (const bf16*)dout;
    const bf16* yv = (const bf16*)v;
    lucid::Strides xs = PS(do_strides), ys = PS(v_strides);
    if (F32) {
      if (int rc = launch_split(dout, do_strides, bw.xsp, bw.lo_xsp, B, HQ, T, K, st)) return rc;
      if (int rc = launch_split(v, v_strides, bw.ysp, bw.lo_ysp, B, H, T, K, st)) return rc;
      xd = bw.xsp;
      yv = bw.ysp;
      xs = split_strides(HQ, T, K);
      ys = split_strides(H, T, K);
    }
    if (K == 128) {
      LUCID_TIMED_LAUNCH(phip, "path_softmax_diag_bwd_kernel", (lucid::path_softmax_diag_bwd_kernel<128, false>),
                         dim3(NT, BHq), st, (const bf16*)dout, PS(do_strides), (const bf16*)o, PS(o_strides),
                         (const bf16*)v, PS(v_strides), HQ, H, T, scale, ws, bw);
      if (int rc = launch_sweeps<true, 128, false>(xd, xs, 0, yv, ys, 0, B, T, HQ, H, scale, ws, bw, st)) return rc;
    } else {
      LUCID_TIMED_LAUNCH(phip, "path_softmax_diag_bwd_kernel", (lucid::path_softmax_diag_bwd_kernel<64, F32>),
                         dim3(NT, BHq), st, (const TI*)dout, PS(do_strides), (const TI*)o, PS(o_strides),
                         (const TI*)v, PS(v_strides), HQ, H, T, scale, ws, bw);
      if (int rc = launch_sweeps<true, 64, F32>(xd, xs, bw.lo_xsp, yv, ys, bw.lo_ysp, B, T, HQ, H, scale, ws, bw, st))
        return rc;
    }
  }
  return launch_back<F32>(q, q_strides, k, k_strides, w, w_strides, beta, beta_strides, dq, dq_strides, dk,
                          dk_strides, dv, dv_strides, dw, dw_strides, dbeta, dbeta_strides, B, T, H, HQ, ws, bw, st,
                          K);
}

}  // namespace

extern "C" {

int lucid_path_abi_version(void) { return 2; }

const char* lucid_path_last_error(void) { return g_path_error.c_str(); }

int lucid_path_chain_status(void) {
  g_path_error.clear();
  return pchain_check();
}

int lucid_path_set_chain_wait_limit(double seconds) {
  g_path_error.clear();
  if (!(seconds > 0.0)) return pfail("the chain wait limit must be positive");
  chain_guard::set_limit(seconds);
  return 0;
}

size_t lucid_path_fwd_workspace_bytes(int B, int T, int H, int HQ, int K) {
  size_t n = 0;
  carve_path_fwd(nullptr, B, T, H, HQ, &n, false, path_kd(K));
  return n;
}

int lucid_path_fwd(const void* q, const int64_t* q_strides, const void* k, const int64_t* k_strides,
                   const void* v, const int64_t* v_strides, const void* w, const int64_t* w_strides,
                   const void* beta, const int64_t* beta_strides, void* o, const int64_t* o_strides,
                   void* kcache, const int64_t* kcache_strides, void* fwd_ws, int B, int T, int H, int HQ,
                   int K, float scale, void* stream) {
  return path_fwd_impl<false>(0, q, q_strides, k, k_strides, v, v_strides, w, w_strides, beta, beta_strides, o,
                              o_strides, kcache, kcache_strides, fwd_ws, B, T, H, HQ, K, scale, stream);
}

size_t lucid_path_bwd_workspace_bytes(int B, int T, int H, int HQ, int K) {
  (void)H;
  size_t n = 0;
  carve_path_bwd(nullptr, B, T, HQ, &n, false, path_kd(K));
  return n;
}

int lucid_path_bwd(const void* dout, const int64_t* do_strides, const void* q, const int64_t* q_strides,
                   const void* k, const int64_t* k_strides, const void* w, const int64_t* w_strides,
                   const void* beta, const int64_t* beta_strides, const void* o, const int64_t* o_strides,
                   const void* fwd_ws, void* dq, const int64_t* dq_strides, void* dk, const int64_t* dk_strides,
                   void* dv, const int64_t* dv_strides, void* dw, const int64_t* dw_strides, void* dbeta,
                   const int64_t* dbeta_strides, void* bwd_ws, int B, int T, int H, int HQ, int K, float scale,
                   void* stream) {
  return path_bwd_impl<false>(0, dout, do_strides, q, q_strides, k, k_strides, nullptr, nullptr, w, w_strides, beta,
                              beta_strides, o, o_strides, fwd_ws, dq, dq_strides, dk, dk_strides, dv, dv_strides, dw,
                              dw_strides, dbeta, dbeta_strides, bwd_ws, B, T, H, HQ, K, scale, stream);
}

size_t lucid_path_softmax_fwd_workspace_bytes(int B, int T, int H, int HQ, int K) {
  size_t n = 0;
  carve_path_fwd(nullptr, B, T, H, HQ, &n, true, path_kd(K));
  return n;
}

int lucid_path_softmax_fwd(const void* q, const int64_t* q_strides, const void* k, const int64_t* k_strides,
                           const void* v, const int64_t* v_strides, const void* w, const int64_t* w_strides,
                           const void* beta, const int64_t* beta_strides, void* o, const int64_t* o_strides,
                           void* kcache, const int64_t* kcache_strides, void* fwd_ws, int B, int T, int H, int HQ,
                           int K, float scale, void* stream) {
  return path_fwd_impl<false>(1, q, q_strides, k, k_strides, v, v_strides, w, w_strides, beta, beta_strides, o,
                              o_strides, kcache, kcache_strides, fwd_ws, B, T, H, HQ, K, scale, stream);
}

size_t lucid_path_softmax_bwd_workspace_bytes(int B, int T, int H, int HQ, int K) {
  (void)H;
  size_t n = 0;
  carve_path_bwd(nullptr, B, T, HQ, &n, true, path_kd(K));
  return n;
}

int lucid_path_softmax_bwd(const void* dout, const int64_t* do_strides, const void* q, const int64_t* q_strides,
                           const void* k, const int64_t* k_strides, const void* v, const int64_t* v_strides,
                           const void* w, const int64_t* w_strides, const void* beta, const int64_t* beta_strides,
                           const void* o, const int64_t* o_strides, const void* fwd_ws, void* dq,
                           const int64_t* dq_strides, void* dk, const int64_t* dk_strides, void* dv,
                           const int64_t* dv_strides, void* dw, const int64_t* dw_strides, void* dbeta,
                           const int64_t* dbeta_strides, void* bwd_ws, int B, int T, int H, int HQ, int K,
                           float scale, void* stream) {
  return path_bwd_impl<false>(1, dout, do_strides, q, q_strides, k, k_strides, v, v_strides, w, w_strides, beta,
                              beta_strides, o, o_strides, fwd_ws, dq, dq_strides, dk, dk_strides, dv, dv_strides, dw,
                              dw_strides, dbeta, dbeta_strides, bwd_ws, B, T, H, HQ, K, scale, stream);
}

size_t lucid_path_fwd_f32_workspace_bytes(int B, int T, int H, int HQ, int K) {
  (void)K;
  size_t n = 0;
  carve_path_fwd(nullptr, B, T, H, HQ, &n, false, 64, true);
  return n;
}

int lucid_path_fwd_f32(const float* q, const int64_t* q_strides, const float* k, const int64_t* k_strides,
                       const float* v, const int64_t* v_strides, const float* w, const int64_t* w_strides,
                       const float* beta, const int64_t* beta_strides, float* o, const int64_t* o_strides,
                       float* kcache, const int64_t* kcache_strides, void* fwd_ws, int B, int T, int H, int HQ, int K,
                       float scale, void* stream) {
  return path_fwd_impl<true>(0, q, q_strides, k, k_strides, v, v_strides, w, w_strides, beta, beta_strides, o,
                             o_strides, kcache, kcache_strides, fwd_ws, B, T, H, HQ, K, scale, stream);
}

size_t lucid_path_bwd_f32_workspace_bytes(int B, int T, int H, int HQ, int K) {
  (void)H;
  (void)K;
  size_t n = 0;
  carve_path_bwd(nullptr, B, T, HQ, &n, false, 64, true);
  return n;
}

int lucid_path_bwd_f32(const float* dout, const int64_t* do_strides, const float* q, const int64_t* q_strides,
                       const float* k, const int64_t* k_strides, const float* w, const int64_t* w_strides,
                       const float* beta, const int64_t* beta_strides, const float* o, const int64_t* o_strides,
                       const void* fwd_ws, float* dq, const int64_t* dq_strides, float* dk, const int64_t* dk_strides,
                       float* dv, const int64_t* dv_strides, float* dw, const int64_t* dw_strides, float* dbeta,
                       const int64_t* dbeta_strides, void* bwd_ws, int B, int T, int H, int HQ, int K, float scale,
                       void* stream) {
  return path_bwd_impl<true>(0, dout, do_strides, q, q_strides, k, k_strides, nullptr, nullptr, w, w_strides, beta,
                             beta_strides, o, o_strides, fwd_ws, dq, dq_strides, dk, dk_strides, dv, dv_strides, dw,
                             dw_strides, dbeta, dbeta_strides, bwd_ws, B, T, H, HQ, K, scale, stream);
}

size_t lucid_path_softmax_fwd_f32_workspace_bytes(int B, int T, int H, int HQ, int K) {
  (void)K;
  size_t n = 0;
  carve_path_fwd(nullptr, B, T, H, HQ, &n, true, 64, true);
  return n;
}

int lucid_path_softmax_fwd_f32(const float* q, const int64_t* q_strides, const float* k, const int64_t* k_strides,
                               const float* v, const int64_t* v_strides, const float* w, const int64_t* w_strides,
                               const float* beta, const int64_t* beta_strides, float* o, const int64_t* o_strides,
                               float* kcache, const int64_t* kcache_strides, void* fwd_ws, int B, int T, int H,
                               int HQ, int K, float scale, void* stream) {
  return path_fwd_impl<true>(1, q, q_strides, k, k_strides, v, v_strides, w, w_strides, beta, beta_strides, o,
                             o_strides, kcache, kcache_strides, fwd_ws, B, T, H, HQ, K, scale, stream);
}

size_t lucid_path_softmax_bwd_f32_workspace_bytes(int B, int T, int H, int HQ, int K) {
  (void)H;
  (void)K;
  size_t n = 0;
  carve_path_bwd(nullptr, B, T, HQ, &n, true, 64, true);
  return n;
}

int lucid_path_softmax_bwd_f32(const float* dout, const int64_t* do_strides, const float* q,
                               const int64_t* q_strides, const float* k, const int64_t* k_strides, const float* v,
                               const int64_t* v_strides, const float* w, const int64_t* w_strides, const float* beta,
                               const int64_t* beta_strides, const float* o, const int64_t* o_strides,
                               const void* fwd_ws, float* dq, const int64_t* dq_strides, float* dk,
                               const int64_t* dk_strides, float* dv, const int64_t* dv_strides, float* dw,
                               const int64_t* dw_strides, float* dbeta, const int64_t* dbeta_strides, void* bwd_ws,
                               int B, int T, int H, int HQ, int K, float scale, void* stream) {
  return path_bwd_impl<true>(1, dout, do_strides, q, q_strides, k, k_strides, v, v_strides, w, w_strides, beta,
                             beta_strides, o, o_strides, fwd_ws, dq, dq_strides, dk, dk_strides, dv, dv_strides, dw,
                             dw_strides, dbeta, dbeta_strides, bwd_ws, B, T, H, HQ, K, scale, stream);
}

void lucid_path_profile_enable(int on) { lucid_prof::enabled() = on != 0; }

void lucid_path_profile_only(const char* name) { lucid_prof::only() = name ? name : ""; }

int lucid_path_profile_collect(void) { return lucid_prof::collect(); }

int lucid_path_profile_entry(int idx, char* name, int name_len, double* total_ms, long* count) {
  return lucid_prof::entry(idx, name, name_len, total_ms, count);
}

void lucid_path_profile_reset(void) { lucid_prof::reset(); }

}  // extern "C"
