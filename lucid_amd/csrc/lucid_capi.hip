// C ABI of the LUCID attention kernels (declared in include/lucid_amd.h).
// One translation unit: the kernel files are included so that every template
// instantiation lives next to its launcher.
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/lucid_amd.h"
#include "lucid_bwd.hip"
#include "lucid_decode.hip"
#include "lucid_fwd.hip"
#include "model_ops.hip"
#include "chain_guard.h"
#include "profiling.h"

namespace {

thread_local std::string g_last_error;

// Precision of the preconditioner chains (lucid_set_precision): LUCID_PRECISION_AUTO picks
// per head from its row mass (lucid_mass_kernel, kExactMass); the others force one kind.
// Per calling thread: a mode set on one thread never changes how another thread's calls run.
thread_local int g_precision = LUCID_PRECISION_AUTO;

// Forward schedule (lucid_set_fused_forward): the fused chain + attention kernel at head
// dim 64 with one query head per kv head, or the two-kernel sequence.  Per calling thread.
thread_local bool g_fused_fwd = true;

int fail(const std::string& msg) {
  g_last_error = msg;
  return LUCID_EINVAL;
}

int hip_status(const char* where) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    g_last_error = std::string(where) + ": " + hipGetErrorString(e);
    return LUCID_EHIP + (int)e;
  }
  return LUCID_OK;
}

size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

// First step of every entry point that launches a chain kernel: set up the bounded waits on
// this device and report a wait that gave up in an earlier launch.
int chain_check() {
  std::string what;
  if (int e = chain_guard::setup(&what)) {
    g_last_error = what + ": " + hipGetErrorString((hipError_t)e);
    return LUCID_EHIP + e;
  }
  if (chain_guard::take_flag()) {
    g_last_error = "a chain wait gave up in an earlier launch (no progress within the wait bound); "
                   "the results of that launch are invalid";
    return LUCID_ECHAIN;
  }
  return LUCID_OK;
}

// Forward workspace carve-out (all offsets 256-byte aligned).
struct FwdWs {
  float* rinv;   // [BH][T]
  bf16* kt;      // [BH][D][T]  K^T, T-perm
  bf16* khat;    // [BH][T][D]  K^ = r K rounded to bf16 (the bf16 chains' key tiles)
  bf16* vpb;     // [BH][T][D]  V' bf16
  bf16* vpt;     // [BH][D][T]  V'^T, T-perm
  float* pinv;   // [BH][T/64][64][64]  inverses of the diagonal blocks of P
  float* zx;     // [BH][T/128][64][64] -(X_B P_BA) per 128-row block, columns T-perm
  bf16* vpbl;    // [BH][T][D]  lo part of V' (exact heads)
  bf16* vptl;    // [BH][D][T]  lo part of V'^T, T-perm (exact heads)
  float* mass;   // [BH]        largest row mass sum_{j<i} P_ij^2 (sampled; selects the chain precision)
  bf16* olo;     // [BHq][T][D] lo part of O (exact heads)
  int* counters; // [BH]
  // fp32 inputs only: the bf16 pairs of Q and K ([BH][T][D] rows), K^T's lo part, the
  // mean key of each head (fp32 [BH][D]) and the pair of K - mean (the attention's keys)
  bf16 *qh, *ql, *kh, *kl, *ktl;
  float* kmean;
  bf16 *kch, *kcl;
  size_t bytes;
};

// Head dims other than 64 and 128 run on rows zero-padded to the next of the two (every
// [.., d] operand has padded_dim(D) columns, columns D.. zero in the inputs and written
// zero in the outputs); the RMS of K divides by D itself.
int padded_dim(int D) { return D <= 64 ? 64 : 128; }

// f32: the fp32-input copies as well (with_q: also those of Q and the attention's keys)
FwdWs carve_fwd(void* base, int B, int Hq, int Hkv, int T, int D, bool f32 = false, bool with_q = true) {
  D = padded_dim(D);
  const size_t BH = (size_t)B * Hkv, BHq = (size_t)B * Hq;
  FwdWs w{};
  size_t off = 0;
  char* p = static_cast<char*>(base);
  auto take = [&](size_t n) {
    char* r = p ? p + off : nullptr;
    off += align256(n);
    return r;
  };
  w.rinv = reinterpret_cast<float*>(take(BH * T * 4));
  w.kt = reinterpret_cast<bf16*>(take(BH * D * T * 2));
  w.khat = reinterpret_cast<bf16*>(take(BH * T * D * 2));
  w.vpb = reinterpret_cast<bf16*>(take(BH * T * D * 2));
  w.vpt = reinterpret_cast<bf16*>(take(BH * D * T * 2));
  w.pinv = reinterpret_cast<float*>(take(BH * (T / 64) * 4096 * 4));
  w.zx = reinterpret_cast<float*>(take(BH * (T / 128) * 4096 * 4));
  w.vpbl = reinterpret_cast<bf16*>(take(BH * T * D * 2));
  w.vptl = reinterpret_cast<bf16*>(take(BH * D * T * 2));
  w.mass = reinterpret_cast<float*>(take(BH * 4));
  w.olo = reinterpret_cast<bf16*>(take(BHq * T * D * 2));
  w.counters = reinterpret_cast<int*>(take(BH * 4));
  if (f32) {
    if (with_q) {
      w.qh = reinterpret_cast<bf16*>(take(BHq * T * D * 2));
      w.ql = reinterpret_cast<bf16*>(take(BHq * T * D * 2));
    }
    w.kh = reinterpret_cast<bf16*>(take(BH * T * D * 2));
    w.kl = reinterpret_cast<bf16*>(take(BH * T * D * 2));
    w.ktl = reinterpret_cast<bf16*>(take(BH * D * T * 2));
    if (with_q) {
      w.kmean = reinterpret_cast<float*>(take(BH * D * 4));
      w.kch = reinterpret_cast<bf16*>(take(BH * T * D * 2));
      w.kcl = reinterpret_cast<bf16*>(take(BH * T * D * 2));
    }
  }
  w.bytes = off;
  return w;
}

struct BwdWs {
  float* delta;  // [BHq][T]
  bf16* seeds;   // [BHq][T][16] the dK/dV' sweep's seed operands of -lse2 / c and -delta
  float* dvp;    // [BH][T][D]   dV' (summed over the group)
  float* dka;    // [BH][T][D]   dK from the softmax part (scaled)
  bf16* dvb;     // [BH][T][D]   dV bf16
  bf16* dvbl;    // [BH][T][D]   lo part of dV (exact heads)
  float* colsum; // [BH][T][D]   sum_I M_IJ^T K^_I
  int* counters; // [BH]
  bf16 *doh, *dol; // fp32 inputs only: the bf16 pair of dO ([BHq][T][D] rows)
  size_t bytes;
};

BwdWs carve_bwd(void* base, int B, int Hq, int Hkv, int T, int D, bool f32 = false) {
  D = padded_dim(D);
  const size_t BH = (size_t)B * Hkv, BHq = (size_t)B * Hq;
  BwdWs w{};
  size_t off = 0;
  char* p = static_cast<char*>(base);
  auto take = [&](size_t n) {
    char* r = p ? p + off : nullptr;
    off += align256(n);
    return r;
  };
  w.delta = reinterpret_cast<float*>(take(BHq * T * 4));
  w.seeds = reinterpret_cast<bf16*>(take(BHq * T * 32));
  w.dvp = reinterpret_cast<float*>(take(BH * T * D * 4));
  w.dka = reinterpret_cast<float*>(take(BH * T * D * 4));
  w.dvb = reinterpret_cast<bf16*>(take(BH * T * D * 2));
  w.dvbl = reinterpret_cast<bf16*>(take(BH * T * D * 2));
  w.colsum = reinterpret_cast<float*>(take(BH * T * D * 4));
  w.counters = reinterpret_cast<int*>(take(BH * 4));
  if (f32) {
    w.doh = reinterpret_cast<bf16*>(take(BHq * T * D * 2));
    w.dol = reinterpret_cast<bf16*>(take(BHq * T * D * 2));
  }
  w.bytes = off;
  return w;
}

int check_dims(int B, int Hq, int Hkv, int T, int D) {
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || T <= 0) return fail("B, Hq, Hkv and T must be positive");
  if (D < 1 || D > 128) return fail("head_dim must be in [1, 128], got " + std::to_string(D));
  if (T % 128 != 0) return fail("T must be a multiple of 128, got " + std::to_string(T));
  if (Hq % Hkv != 0) return fail("Hq must be a multiple of Hkv");
  if ((int64_t)B * Hq * (T / 128) > (int64_t)0x7fffffff) return fail("grid too large");
  return LUCID_OK;
}

// Workspaces hold the chain operands; their 64-row blocks must fill whole cache lines.
int check_ws(const char* name, const void* p) {
  if (reinterpret_cast<uintptr_t>(p) % 256) return fail(std::string(name) + " must be 256-byte aligned");
  return LUCID_OK;
}

int check_tensor(const char* name, const void* p, const int64_t* s) {
  if (!p) return fail(std::string(name) + " is null");
  if (!s) return fail(std::string(name) + " strides are null");
  if (reinterpret_cast<uintptr_t>(p) % 16) return fail(std::string(name) + " must be 16-byte aligned");
  for (int i = 0; i < 3; ++i)
    if (s[i] % 8) return fail(std::string(name) + " strides must be multiples of 8 elements");
  return LUCID_OK;
}

lucid::Strides S(const int64_t* s) { return lucid::Strides{s[0], s[1], s[2]}; }

#define LUCID_LAUNCH(NAME, KERNEL, GRID, ST, ...) LUCID_TIMED_LAUNCH(hip_status, NAME, KERNEL, GRID, ST, __VA_ARGS__)
#define LUCID_LAUNCH_B(NAME, KERNEL, GRID, BLOCK, ST, ...) \
  LUCID_TIMED_LAUNCH_B(hip_status, NAME, KERNEL, GRID, BLOCK, ST, __VA_ARGS__)

template <int D>
int launch_precond_fwd(const void* k, const int64_t* ks, const void* v, const int64_t* vs, float* vprime,
                       const FwdWs& w, int B, int Hkv, int T, float scale, float eps, float dn, hipStream_t st) {
  const int BH = B * Hkv;
  // a forced precision is written straight into the head masses (no mass pass)
  const float mass_init = g_precision == LUCID_PRECISION_EXACT ? 1e30f : 0.f;
  LUCID_LAUNCH("lucid_prep_kernel", lucid::lucid_prep_kernel<D>, dim3(T / 64, BH), st, (const bf16*)k, S(ks), Hkv,
               T, eps, dn, scale, w.rinv, w.kt, w.pinv, w.counters, w.mass, mass_init, lucid::Lo{}, nullptr,
               w.khat);
  // the in-block coupling of every 128-row chain block and (AUTO) the heads' row masses
  LUCID_LAUNCH("lucid_zx_kernel", lucid::lucid_zx_kernel<D>, dim3(T / 128, BH), st, (const bf16*)k, S(ks), Hkv, T,
               w.rinv, scale, w.pinv, w.zx, lucid::Lo{}, g_precision == LUCID_PRECISION_AUTO ? w.mass : nullptr);
  // both instances of the chain: each solves the heads of its precision and returns at
  // once for the others
  if (g_precision != LUCID_PRECISION_EXACT) {
    if (D == 128 && T % 256 == 0)  // 256 rows per workgroup: each staged pair serves twice the rows
      LUCID_LAUNCH_B("lucid_precond_fwd_wide_kernel", (lucid::lucid_precond_fwd_wide_kernel<128>),
                     dim3((T / 256) * BH), dim3(512), st, (const bf16*)k, S(ks), (const bf16*)v, S(vs), Hkv, T, BH,
                     w.rinv, w.khat, scale, vprime, w.vpb, w.vpt, w.pinv, w.zx, w.mass, w.counters);
    else if (D == 128)  // eight waves (two per SIMD) at head dim 128
      LUCID_LAUNCH_B("lucid_precond_fwd_kernel", (lucid::lucid_precond_fwd_kernel<128, false, false, 8>),
                     dim3((T / 128) * BH), dim3(512), st, (const bf16*)k, S(ks), (const bf16*)v, S(vs), Hkv, T, BH,
                     w.rinv, w.khat, scale, vprime, w.vpb, w.vpt, w.vpbl, w.vptl, w.pinv, w.zx, w.mass, w.counters,
                     lucid::Lo{});
    else
      LUCID_LAUNCH("lucid_precond_fwd_kernel", (lucid::lucid_precond_fwd_kernel<D, false>), dim3((T / 128) * BH),
                   st, (const bf16*)k, S(ks), (const bf16*)v, S(vs), Hkv, T, BH, w.rinv, w.khat, scale, vprime,
                   w.vpb, w.vpt, w.vpbl, w.vptl, w.pinv, w.zx, w.mass, w.counters, lucid::Lo{});
  }
  if (g_precision != LUCID_PRECISION_FAST)
    LUCID_LAUNCH("lucid_precond_fwd_exact_kernel", (lucid::lucid_precond_fwd_kernel<D, true>),
                 dim3((T / 128) * BH), st, (const bf16*)k, S(ks), (const bf16*)v, S(vs), Hkv, T, BH, w.rinv, w.khat,
                 scale, vprime, w.vpb, w.vpt, w.vpbl, w.vptl, w.pinv, w.zx, w.mass, w.counters, lucid::Lo{});
  return LUCID_OK;
}

// The head-dim columns the attention products run over: rows of a head
// dim in (64, 96] are zero-padded to 128 and only the first 80 (d <= 80) or 96 columns can
// be nonzero (k-steps of 16, value tiles of 32).  dn: the caller's head dim (<= 0: unknown,
// all of D).  Returns 80, 96 or D.
template <int D>
int active_dims(float dn) {
  if (D != 128 || !(dn > 0.f)) return D;
  return dn <= 80.f ? 80 : dn <= 96.f ? 96 : D;
}

// Causal attention on the V' operands of w (bf16): the 256-thread kernel at head dim 64,
// the eight-wave kernel at 128.
template <int D>
int launch_attn_fwd(const void* q, const int64_t* qs, const void* k, const int64_t* ks, void* o, const int64_t* os,
                    float* lse, const FwdWs& w, int B, int Hq, int Hkv, int T, float scale, float dn,
                    hipStream_t st) {
  const int BHq = B * Hq;
  if constexpr (D == 128) {
    // 128 keys per staged tile: half the barriers and row-max updates of 64 (1 % at config 5)
    auto wide = [&](auto dac) -> int {
      LUCID_LAUNCH_B("lucid_attn_fwd_wide_kernel", (lucid::lucid_attn_fwd_wide_kernel<D, 128, decltype(dac)::value>),
                     dim3(((T + 255) / 256) * BHq), dim3(512), st, (const bf16*)q, S(qs), (const bf16*)k, S(ks),
                     w.vpt, (bf16*)o, S(os), lse, w.mass, w.olo, Hq, Hkv, T, B * Hkv, scale);
      return LUCID_OK;
    };
    const int da = active_dims<D>(dn);
    if (da == 80) return wide(std::integral_constant<int, 80>{});
    if (da == 96) return wide(std::integral_constant<int, 96>{});
    return wide(std::integral_constant<int, D>{});
  } else {
    LUCID_LAUNCH("lucid_attn_fwd_kernel", lucid::lucid_attn_fwd_kernel<D>, dim3(((T + 255) / 256) * BHq), st,
                 (const bf16*)q, S(qs), (const bf16*)k, S(ks), w.vpt, (bf16*)o, S(os), lse, w.mass, w.olo, Hq, Hkv,
                 T, BHq, scale, lucid::Lo{}, nullptr, 0);
  }
  return LUCID_OK;
}

template <int D>
int launch_fwd(const void* q, const int64_t* qs, const void* k, const int64_t* ks, const void* v, const int64_t* vs,
               void* o, const int64_t* os, float* vprime, float* lse, const FwdWs& w, int B, int Hq, int Hkv, int T,
               float scale, float eps, float dn, hipStream_t st) {
  if constexpr (D == 64) {
    if (Hq == Hkv && g_fused_fwd) {
      const int BH = B * Hkv;
      const float mass_init = g_precision == LUCID_PRECISION_EXACT ? 1e30f : 0.f;
      LUCID_LAUNCH("lucid_prep_kernel", lucid::lucid_prep_kernel<D>, dim3(T / 64, BH), st, (const bf16*)k, S(ks),
                   Hkv, T, eps, dn, scale, w.rinv, w.kt, w.pinv, w.counters, w.mass, mass_init, lucid::Lo{}, nullptr,
                   w.khat);
      LUCID_LAUNCH("lucid_zx_kernel", lucid::lucid_zx_kernel<D>, dim3(T / 128, BH), st, (const bf16*)k, S(ks), Hkv,
                   T, w.rinv, scale, w.pinv, w.zx, lucid::Lo{}, g_precision == LUCID_PRECISION_AUTO ? w.mass : nullptr);
      if (g_precision != LUCID_PRECISION_EXACT)
        LUCID_LAUNCH("lucid_fused_fwd_kernel", lucid::lucid_fused_fwd_kernel<D>, dim3((T / 128) * BH), st,
                     (const bf16*)q, S(qs), (const bf16*)k, S(ks), (const bf16*)v, S(vs), Hkv, T, BH, w.rinv, scale,
                     vprime, w.vpb, w.vpt, w.pinv, w.zx, w.mass, w.counters, (bf16*)o, S(os), lse);
      if (g_precision != LUCID_PRECISION_FAST) {
        // heads of the exact chains: their chain, then their attention (skip_fast)
        LUCID_LAUNCH("lucid_precond_fwd_exact_kernel", (lucid::lucid_precond_fwd_kernel<D, true>),
                     dim3((T / 128) * BH), st, (const bf16*)k, S(ks), (const bf16*)v, S(vs), Hkv, T, BH, w.rinv,
                     w.khat, scale, vprime, w.vpb, w.vpt, w.vpbl, w.vptl, w.pinv, w.zx, w.mass, w.counters,
                     lucid::Lo{});
        LUCID_LAUNCH("lucid_attn_fwd_exact_kernel", lucid::lucid_attn_fwd_kernel<D>, dim3(((T + 255) / 256) * B * Hq),
                     st, (const bf16*)q, S(qs), (const bf16*)k, S(ks), w.vpt, (bf16*)o, S(os), lse, w.mass, w.olo,
                     Hq, Hkv, T, B * Hq, scale, lucid::Lo{}, nullptr, 1);
      }
      return LUCID_OK;
    }
  }
  if (int rc = launch_precond_fwd<D>(k, ks, v, vs, vprime, w, B, Hkv, T, scale, eps, dn, st)) return rc;
  return launch_attn_fwd<D>(q, qs, k, ks, o, os, lse, w, B, Hq, Hkv, T, scale, dn, st);
}

// The attention part of the backward: delta, dV' and the softmax dK (into w.dvp, w.dka)
// and dQ.  Reads f.vpb, f.olo and f.mass.
template <int D>
int launch_attn_bwd(const void* dout, const int64_t* dos, const void* q, const int64_t* qs, const void* k,
                    const int64_t* ks, const void* o, const int64_t* os, const float* lse, const FwdWs& f, void* dq,
                    const int64_t* dqs, const BwdWs& w, int B, int Hq, int Hkv, int T, float scale, float dn,
                    hipStream_t st) {
  const int BH = B * Hkv, BHq = B * Hq;
  const float cinv = 1.f / (scale * LOG2E_F);
  LUCID_LAUNCH("lucid_bwd_prep_kernel", lucid::lucid_bwd_prep_kernel<D>, dim3(T / 64, BHq), st, (const bf16*)dout,
               S(dos), (const bf16*)o, S(os), f.olo, f.mass, Hq, Hkv, T, w.delta, w.counters, BH, lucid::Lo{}, lse,
               cinv, w.seeds);
  // dQ: four waves of 64 rows at head dim 64, eight waves of 32 rows at 128; the exact
  // instance at 128: 128 rows per workgroup, one wave per SIMD (its hi/lo operands need the
  // registers).  DA: the active head-dim columns (zero-padded rows of a smaller head dim)
  constexpr int RW = D == 128 ? 32 : 64;
  constexpr int XWGR = D == 128 ? 128 : 256;
  auto sweeps = [&](auto dac) -> int {
    constexpr int DA = decltype(dac)::value;
    LUCID_LAUNCH("lucid_attn_bwd_dkdv_kernel", (lucid::lucid_attn_bwd_dkdv_kernel<D, false, DA>),
                 dim3((T / 128) * BH), st, (const bf16*)q, S(qs), (const bf16*)k, S(ks), f.vpb, (const bf16*)dout,
                 S(dos), w.seeds, w.dvp, w.dka, Hq, Hkv, T, BH, scale, lucid::Lo{}, nullptr);
    LUCID_LAUNCH_B("lucid_attn_bwd_dq_kernel", (lucid::lucid_attn_bwd_dq_kernel<D, false, false, RW, 256, DA>),
                   dim3(((T + 255) / 256) * BHq), dim3(64 * (256 / RW)), st, (const bf16*)q, S(qs), (const bf16*)k,
                   S(ks), f.vpb, (const bf16*)dout, S(dos), lse, w.delta, f.mass, (bf16*)dq, S(dqs), Hq, Hkv, T, BHq,
                   scale, lucid::Lo{}, nullptr);
    LUCID_LAUNCH_B("lucid_attn_bwd_dq_exact_kernel", (lucid::lucid_attn_bwd_dq_kernel<D, true, false, RW, XWGR, DA>),
                   dim3(((T + XWGR - 1) / XWGR) * BHq), dim3(64 * (XWGR / RW)), st, (const bf16*)q, S(qs),
                   (const bf16*)k, S(ks), f.vpb, (const bf16*)dout, S(dos), lse, w.delta, f.mass, (bf16*)dq, S(dqs),
                   Hq, Hkv, T, BHq, scale, lucid::Lo{}, nullptr);
    return LUCID_OK;
  };
  if constexpr (D == 128) {
    const int da = active_dims<D>(dn);
    if (da == 80) return sweeps(std::integral_constant<int, 80>{});
    if (da == 96) return sweeps(std::integral_constant<int, 96>{});
  }
  return sweeps(std::integral_constant<int, D>{});
}

// The preconditioner part: dV = P^-T dV' (w.dvp, counters zeroed), then dK with the softmax
// part w.dka added (null: none).  Reads the forward's K operands, V' and row masses.
template <int D>
int launch_precond_bwd(const void* k, const int64_t* ks, const FwdWs& f, void* dk, const int64_t* dks, void* dv,
                       const int64_t* dvs, const BwdWs& w, const float* dka, int B, int Hkv, int T, float scale,
                       float dn, hipStream_t st) {
  const int BH = B * Hkv;
  // each chain kernel in two instances (bf16 and exact), selected per head by the forward's
  // row mass; the precision forced at the forward call is recorded there
  // bf16 chains at head dim 64: 256 columns per workgroup when T allows it
  if (D == 64 && T % 256 == 0) {
    LUCID_LAUNCH_B("lucid_precond_bwd_col_wide_kernel", lucid::lucid_precond_bwd_col_wide_kernel<64>,
                   dim3((T / 256) * BH), dim3(512), st, (const bf16*)k, S(ks), Hkv, T, BH, f.rinv, f.khat, scale,
                   f.vpb, f.pinv, f.mass, w.dvp, w.dvb, (bf16*)dv, S(dvs), w.colsum, w.counters);
  }
  // the 128-column chains (bf16 unless the wide one ran, and the exact instance) over the
  // active head-dim columns
  auto col_chains = [&](auto dac) -> int {
    constexpr int DA = decltype(dac)::value;
    if (!(D == 64 && T % 256 == 0))
      LUCID_LAUNCH("lucid_precond_bwd_col_kernel", (lucid::lucid_precond_bwd_col_kernel<D, false, false, DA>),
                   dim3((T / 128) * BH), st, (const bf16*)k, S(ks), Hkv, T, BH, f.rinv, f.khat, scale, f.kt, f.vpb,
                   f.vpbl, f.pinv, f.mass, w.dvp, w.dvb, w.dvbl, (bf16*)dv, S(dvs), w.colsum, w.counters,
                   lucid::Lo{});
    LUCID_LAUNCH("lucid_precond_bwd_col_exact_kernel", (lucid::lucid_precond_bwd_col_kernel<D, true, false, DA>),
                 dim3((T / 128) * BH), st, (const bf16*)k, S(ks), Hkv, T, BH, f.rinv, f.khat, scale, f.kt, f.vpb,
                 f.vpbl, f.pinv, f.mass, w.dvp, w.dvb, w.dvbl, (bf16*)dv, S(dvs), w.colsum, w.counters, lucid::Lo{});
    return LUCID_OK;
  };
  int rc_col;
  if constexpr (D == 128) {
    const int da = active_dims<D>(dn);
    rc_col = da == 80   ? col_chains(std::integral_constant<int, 80>{})
             : da == 96 ? col_chains(std::integral_constant<int, 96>{})
                        : col_chains(std::integral_constant<int, D>{});
  } else {
    rc_col = col_chains(std::integral_constant<int, D>{});
  }
  if (rc_col) return rc_col;
  LUCID_LAUNCH("lucid_precond_bwd_row_kernel", (lucid::lucid_precond_bwd_row_kernel<D, false>),
               dim3(((T + 255) / 256) * BH), st, (const bf16*)k, S(ks), Hkv, T, BH, f.rinv, f.khat, scale, dn,
               f.vpb, f.vpbl, w.dvb, w.dvbl, f.mass, w.colsum, dka, (bf16*)dk, S(dks), lucid::Lo{});
  // the exact instance at head dim 128: one n-tile per wave (128 rows per workgroup), so that
  // its hi/lo row operands stay in registers
  constexpr int XNT = D == 128 ? 1 : 2;
  LUCID_LAUNCH("lucid_precond_bwd_row_exact_kernel", (lucid::lucid_precond_bwd_row_kernel<D, true, false, XNT>),
               dim3(((T + 128 * XNT - 1) / (128 * XNT)) * BH), st, (const bf16*)k, S(ks), Hkv, T, BH, f.rinv, f.khat,
               scale, dn, f.vpb, f.vpbl, w.dvb, w.dvbl, f.mass, w.colsum, dka, (bf16*)dk, S(dks), lucid::Lo{});
  return LUCID_OK;
}

template <int D>
int launch_bwd(const void* dout, const int64_t* dos, const void* q, const int64_t* qs, const void* k,
               const int64_t* ks, const void* o, const int64_t* os, const float* lse, const FwdWs& f, void* dq,
               const int64_t* dqs, void* dk, const int64_t* dks, void* dv, const int64_t* dvs, const BwdWs& w, int B,
               int Hq, int Hkv, int T, float scale, float dn, hipStream_t st) {
  if (int rc = launch_attn_bwd<D>(dout, dos, q, qs, k, ks, o, os, lse, f, dq, dqs, w, B, Hq, Hkv, T, scale, dn, st))
    return rc;
  return launch_precond_bwd<D>(k, ks, f, dk, dks, dv, dvs, w, w.dka, B, Hkv, T, scale, dn, st);
}

// ---- the two operator seams (get_v_prime / eager_lucid_attention_forward) ----

// Workspace of the attention on a caller's V': the operand copies of V', 1/rms of K,
// the row masses and O's lo part (the FwdWs fields the attention kernels read).
// (f32: the bf16 pairs of Q, K - mean and V' as well.)
FwdWs carve_attn_vp(void* base, int B, int Hq, int Hkv, int T, int D, bool f32 = false) {
  D = padded_dim(D);
  const size_t BH = (size_t)B * Hkv, BHq = (size_t)B * Hq;
  FwdWs w{};
  size_t off = 0;
  char* p = static_cast<char*>(base);
  auto take = [&](size_t n) {
    char* r = p ? p + off : nullptr;
    off += align256(n);
    return r;
  };
  w.rinv = reinterpret_cast<float*>(take(BH * T * 4));
  w.vpb = reinterpret_cast<bf16*>(take(BH * T * D * 2));
  w.vpt = reinterpret_cast<bf16*>(take(BH * D * T * 2));
  w.mass = reinterpret_cast<float*>(take(BH * 4));
  w.olo = reinterpret_cast<bf16*>(take(BHq * T * D * 2));
  if (f32) {
    w.qh = reinterpret_cast<bf16*>(take(BHq * T * D * 2));
    w.ql = reinterpret_cast<bf16*>(take(BHq * T * D * 2));
    w.kmean = reinterpret_cast<float*>(take(BH * D * 4));
    w.kch = reinterpret_cast<bf16*>(take(BH * T * D * 2));
    w.kcl = reinterpret_cast<bf16*>(take(BH * T * D * 2));
    w.vpbl = reinterpret_cast<bf16*>(take(BH * T * D * 2));
    w.vptl = reinterpret_cast<bf16*>(take(BH * D * T * 2));
  }
  w.bytes = off;
  return w;
}

// Backward scratch of one seam: the attention part needs delta, dV' and the softmax dK, the
// preconditioner part dV' (as fp32), dV and its lo part, the column sums and counters.
// (f32 with attn: the bf16 pair of dO as well.)
BwdWs carve_seam_bwd(void* base, int B, int Hq, int Hkv, int T, int D, bool attn, bool f32 = false) {
  D = padded_dim(D);
  const size_t BH = (size_t)B * Hkv, BHq = (size_t)B * Hq;
  BwdWs w{};
  size_t off = 0;
  char* p = static_cast<char*>(base);
  auto take = [&](size_t n) {
    char* r = p ? p + off : nullptr;
    off += align256(n);
    return r;
  };
  w.dvp = reinterpret_cast<float*>(take(BH * T * D * 4));
  if (attn) {
    w.delta = reinterpret_cast<float*>(take(BHq * T * 4));
    w.seeds = reinterpret_cast<bf16*>(take(BHq * T * 32));
    w.dka = reinterpret_cast<float*>(take(BH * T * D * 4));
    if (f32) {
      w.doh = reinterpret_cast<bf16*>(take(BHq * T * D * 2));
      w.dol = reinterpret_cast<bf16*>(take(BHq * T * D * 2));
    }
  } else {
    w.dvb = reinterpret_cast<bf16*>(take(BH * T * D * 2));
    w.dvbl = reinterpret_cast<bf16*>(take(BH * T * D * 2));
    w.colsum = reinterpret_cast<float*>(take(BH * T * D * 4));
  }
  w.counters = reinterpret_cast<int*>(take(BH * 4));
  w.bytes = off;
  return w;
}

template <int D>
int launch_attn_vp_fwd(const void* q, const int64_t* qs, const void* k, const int64_t* ks, const void* vp,
                       const int64_t* vs, int vp_f32, void* o, const int64_t* os, float* lse, const FwdWs& w, int B,
                       int Hq, int Hkv, int T, float scale, float eps, float dn, hipStream_t st) {
  const int BH = B * Hkv, BHq = B * Hq;
  const float mass_init = g_precision == LUCID_PRECISION_EXACT ? 1e30f : 0.f;
  if (vp_f32)
    LUCID_LAUNCH("lucid_vp_layout_kernel", (lucid::lucid_vp_layout_kernel<D, float>), dim3(T / 64, BH), st,
                 (const bf16*)k, S(ks), (const float*)vp, S(vs), Hkv, T, eps, dn, w.rinv, w.vpb, w.vpt, w.mass,
                 mass_init, nullptr, nullptr);
  else
    LUCID_LAUNCH("lucid_vp_layout_kernel", (lucid::lucid_vp_layout_kernel<D, bf16>), dim3(T / 64, BH), st,
                 (const bf16*)k, S(ks), (const bf16*)vp, S(vs), Hkv, T, eps, dn, w.rinv, w.vpb, w.vpt, w.mass,
                 mass_init, nullptr, nullptr);
  if (g_precision == LUCID_PRECISION_AUTO)
    LUCID_LAUNCH("lucid_mass_kernel", lucid::lucid_mass_kernel<D>, dim3(T / 64, BH), st, (const bf16*)k, S(ks),
                 Hkv, T, w.rinv, scale, w.mass);
  return launch_attn_fwd<D>(q, qs, k, ks, o, os, lse, w, B, Hq, Hkv, T, scale, dn, st);
}

template <int D>
int launch_attn_vp_bwd(const void* dout, const int64_t* dos, const void* q, const int64_t* qs, const void* k,
                       const int64_t* ks, const void* o, const int64_t* os, const float* lse, const FwdWs& f,
                       void* dq, const int64_t* dqs, void* dk, const int64_t* dks, void* dvp, const int64_t* dvps,
                       int dvp_f32, const BwdWs& w, int B, int Hq, int Hkv, int T, float scale, float dn,
                       hipStream_t st) {
  const int BH = B * Hkv;
  if (int rc = launch_attn_bwd<D>(dout, dos, q, qs, k, ks, o, os, lse, f, dq, dqs, w, B, Hq, Hkv, T, scale, dn, st))
    return rc;
  LUCID_LAUNCH("lucid_rows_out_kernel", (lucid::lucid_rows_out_kernel<D, bf16>), dim3(T / 64, BH), st, w.dka,
               (bf16*)dk, S(dks), Hkv, T, 1.f);
  if (dvp_f32)
    LUCID_LAUNCH("lucid_rows_out_kernel", (lucid::lucid_rows_out_kernel<D, float>), dim3(T / 64, BH), st, w.dvp,
                 (float*)dvp, S(dvps), Hkv, T, 1.f);
  else
    LUCID_LAUNCH("lucid_rows_out_kernel", (lucid::lucid_rows_out_kernel<D, bf16>), dim3(T / 64, BH), st, w.dvp,
                 (bf16*)dvp, S(dvps), Hkv, T, 1.f);
  return LUCID_OK;
}

template <int D>
int launch_precond_only_bwd(const void* k, const int64_t* ks, const void* dvp, const int64_t* dvps, int dvp_f32,
                            const FwdWs& f, void* dk, const int64_t* dks, void* dv, const int64_t* dvs,
                            const BwdWs& w, int B, int Hkv, int T, float scale, float dn, hipStream_t st) {
  const int BH = B * Hkv;
  if (dvp_f32)
    LUCID_LAUNCH("lucid_rows_in_kernel", (lucid::lucid_rows_in_kernel<D, float>), dim3(T / 64, BH), st,
                 (const float*)dvp, S(dvps), w.dvp, Hkv, T, w.counters);
  else
    LUCID_LAUNCH("lucid_rows_in_kernel", (lucid::lucid_rows_in_kernel<D, bf16>), dim3(T / 64, BH), st,
                 (const bf16*)dvp, S(dvps), w.dvp, Hkv, T, w.counters);
  return launch_precond_bwd<D>(k, ks, f, dk, dks, dv, dvs, w, nullptr, B, Hkv, T, scale, dn, st);
}

// ---- fp32 inputs (head dim 64) ----
// Q, K, dO (and a caller's V') are split into bf16 pairs (lucid_split_kernel) and every
// product of the path is taken on the pairs (lucid_common.h, struct Lo); V, O and dO enter
// as fp32 where they are summed directly (the chain's right-hand side, delta).  All heads
// run the exact chain instances (their row mass is forced above kExactMass); outputs are
// fp32.  The launchers mirror the bf16 ones above piece by piece.

constexpr float kForceExact = 1e30f;

// Element strides of the contiguous [B][H][T][D] rows of a split copy.
lucid::Strides rows_strides(int H, int T, int D) {
  return lucid::Strides{(int64_t)H * T * D, (int64_t)T * D, (int64_t)D};
}

template <int D>
int launch_split(const void* x, const int64_t* xs, int B, int H, int T, bf16* hi, bf16* lo, hipStream_t st,
                 const float* center = nullptr) {
  LUCID_LAUNCH("lucid_split_kernel", lucid::lucid_split_kernel<D>, dim3(T / 64, B * H), st, (const float*)x,
               S(xs), H, T, hi, lo, center);
  return LUCID_OK;
}

// The attention's keys: K - (mean key of the head) as a bf16 pair in w.kch / w.kcl.
template <int D>
int launch_centered_keys(const void* k, const int64_t* ks, const FwdWs& w, int B, int Hkv, int T, hipStream_t st) {
  LUCID_LAUNCH("lucid_key_mean_kernel", lucid::lucid_key_mean_kernel<D>, dim3(B * Hkv), st, (const float*)k,
               S(ks), Hkv, T, w.kmean);
  return launch_split<D>(k, ks, B, Hkv, T, w.kch, w.kcl, st, w.kmean);
}

// V' = P^-1 V from fp32 K and V (K split into w.kh / w.kl).
template <int D>
int launch_precond_fwd_f32(const void* k, const int64_t* ks, const void* v, const int64_t* vs, float* vprime,
                           const FwdWs& w, int B, int Hkv, int T, float scale, float eps, float dn,
                           hipStream_t st) {
  const int BH = B * Hkv;
  const lucid::Strides ck = rows_strides(Hkv, T, D);
  if (int rc = launch_split<D>(k, ks, B, Hkv, T, w.kh, w.kl, st)) return rc;
  lucid::Lo lo{};
  lo.k = w.kl;
  lo.kt = w.ktl;
  lo.v = static_cast<const float*>(v);
  LUCID_LAUNCH("lucid_prep_f32_kernel", (lucid::lucid_prep_kernel<D, true>), dim3(T / 64, BH), st, w.kh, ck, Hkv,
               T, eps, dn, scale, w.rinv, w.kt, w.pinv, w.counters, w.mass, kForceExact, lo, w.ktl, nullptr);
  LUCID_LAUNCH("lucid_zx_f32_kernel", (lucid::lucid_zx_kernel<D, true>), dim3(T / 128, BH), st, w.kh, ck, Hkv, T,
               w.rinv, scale, w.pinv, w.zx, lo);
  // the chain reads V as fp32 through lo.v with V's own strides (its bf16 operand is unused)
  LUCID_LAUNCH("lucid_precond_fwd_f32_kernel", (lucid::lucid_precond_fwd_kernel<D, true, true>),
               dim3((T / 128) * BH), st, w.kh, ck, (const bf16*)v, S(vs), Hkv, T, BH, w.rinv, nullptr, scale, vprime,
               w.vpb, w.vpt, w.vpbl, w.vptl, w.pinv, w.zx, w.mass, w.counters, lo);
  return LUCID_OK;
}

// O = softmax(s Q K^T, causal) V' on the split Q (split here), the centred keys and V' in
// w.  lse is the row normaliser of the scores against the centred keys.
template <int D>
int launch_attn_fwd_f32(const void* q, const int64_t* qs, void* o, const int64_t* os, float* lse, const FwdWs& w,
                        int B, int Hq, int Hkv, int T, float scale, float dn, hipStream_t st) {
  const int BHq = B * Hq;
  if (int rc = launch_split<D>(q, qs, B, Hq, T, w.qh, w.ql, st)) return rc;
  lucid::Lo lo{};
  lo.q = w.ql;
  lo.k = w.kcl;
  // head dim 128: one 32-row n-tile per wave (128 rows per workgroup), so that the hi/lo
  // operands stay in registers
  constexpr int NT = D == 128 ? 1 : 2;
  const dim3 grid(((T + 128 * NT - 1) / (128 * NT)) * BHq);
  if constexpr (D == 128) {
    const int da = active_dims<D>(dn);
#define LUCID_ATTN_FWD_NARROW(DA)                                                                                    \
  LUCID_LAUNCH("lucid_attn_fwd_f32_kernel", (lucid::lucid_attn_fwd_kernel<D, true, NT, DA>), grid, st, w.qh,        \
               rows_strides(Hq, T, D), w.kch, rows_strides(Hkv, T, D), w.vpt, (float*)o, S(os), lse, w.mass, w.olo, \
               Hq, Hkv, T, BHq, scale, lo, w.vptl, 0)
    if (da == 80) {
      LUCID_ATTN_FWD_NARROW(80);
      return LUCID_OK;
    }
    if (da == 96) {
      LUCID_ATTN_FWD_NARROW(96);
      return LUCID_OK;
    }
#undef LUCID_ATTN_FWD_NARROW
  }
  LUCID_LAUNCH("lucid_attn_fwd_f32_kernel", (lucid::lucid_attn_fwd_kernel<D, true, NT>), grid, st, w.qh,
               rows_strides(Hq, T, D), w.kch, rows_strides(Hkv, T, D), w.vpt, (float*)o, S(os), lse, w.mass, w.olo,
               Hq, Hkv, T, BHq, scale, lo, w.vptl, 0);
  return LUCID_OK;
}

template <int D>
int launch_fwd_f32(const void* q, const int64_t* qs, const void* k, const int64_t* ks, const void* v,
                   const int64_t* vs, void* o, const int64_t* os, float* vprime, float* lse, const FwdWs& w, int B,
                   int Hq, int Hkv, int T, float scale, float eps, float dn, hipStream_t st) {
  if (int rc = launch_precond_fwd_f32<D>(k, ks, v, vs, vprime, w, B, Hkv, T, scale, eps, dn, st)) return rc;
  if (int rc = launch_centered_keys<D>(k, ks, w, B, Hkv, T, st)) return rc;
  return launch_attn_fwd_f32<D>(q, qs, o, os, lse, w, B, Hq, Hkv, T, scale, dn, st);
}

// The attention part of the backward: delta (from fp32 dO and O), dV' and the softmax dK
// (into w.dvp, w.dka) and dQ (fp32).  Reads the split Q, centred K and V' of the forward.
// dQ: four waves of 64 rows at head dim 64, eight waves of 32 rows at 128.
template <int D>
int launch_attn_bwd_f32(const void* dout, const int64_t* dos, const void* o, const int64_t* os, const float* lse,
                        const FwdWs& f, void* dq, const int64_t* dqs, const BwdWs& w, int B, int Hq, int Hkv, int T,
                        float scale, float dn, hipStream_t st) {
  const int BH = B * Hkv, BHq = B * Hq;
  const lucid::Strides cq = rows_strides(Hq, T, D), ck = rows_strides(Hkv, T, D);
  if (int rc = launch_split<D>(dout, dos, B, Hq, T, w.doh, w.dol, st)) return rc;
  lucid::Lo lo{};
  lo.q = f.ql;
  lo.k = f.kcl;
  lo.dout = w.dol;
  lo.o = static_cast<const float*>(o);
  lo.dof = static_cast<const float*>(dout);
  // delta reads fp32 dO and O with their own strides (the bf16 operands are unused)
  LUCID_LAUNCH("lucid_bwd_prep_f32_kernel", (lucid::lucid_bwd_prep_kernel<D, true>), dim3(T / 64, BHq), st,
               (const bf16*)dout, S(dos), (const bf16*)o, S(os), f.olo, f.mass, Hq, Hkv, T, w.delta, w.counters, BH,
               lo, lse, 1.f / (scale * LOG2E_F), w.seeds);
  // head dim 128: four waves of 32 rows for dQ (128 rows per workgroup, one wave per SIMD),
  // so that the hi/lo operands of a wave stay in registers
  constexpr int RW = D == 128 ? 32 : 64, WGR = D == 128 ? 128 : 256;
  const dim3 gkv((T / 128) * BH), gq(((T + WGR - 1) / WGR) * BHq), bq(64 * (WGR / RW));
  if constexpr (D == 128) {
    const int da = active_dims<D>(dn);
#define LUCID_ATTN_BWD_NARROW(DA)                                                                                   \
  LUCID_LAUNCH("lucid_attn_bwd_dkdv_f32_kernel", (lucid::lucid_attn_bwd_dkdv_kernel<D, true, DA>), gkv, st, f.qh,  \
               cq, f.kch, ck, f.vpb, w.doh, cq, w.seeds, w.dvp, w.dka, Hq, Hkv, T, BH, scale, lo, f.vpbl);          \
  LUCID_LAUNCH_B("lucid_attn_bwd_dq_f32_kernel", (lucid::lucid_attn_bwd_dq_kernel<D, true, true, RW, WGR, DA>), gq, \
                 bq, st, f.qh, cq, f.kch, ck, f.vpb, w.doh, cq, lse, w.delta, f.mass, (float*)dq, S(dqs), Hq, Hkv, T,  \
                 BHq, scale, lo, f.vpbl)
    if (da == 80) {
      LUCID_ATTN_BWD_NARROW(80);
      return LUCID_OK;
    }
    if (da == 96) {
      LUCID_ATTN_BWD_NARROW(96);
      return LUCID_OK;
    }
#undef LUCID_ATTN_BWD_NARROW
  }
  LUCID_LAUNCH("lucid_attn_bwd_dkdv_f32_kernel", (lucid::lucid_attn_bwd_dkdv_kernel<D, true>), gkv, st, f.qh, cq,
               f.kch, ck, f.vpb, w.doh, cq, w.seeds, w.dvp, w.dka, Hq, Hkv, T, BH, scale, lo, f.vpbl);
  LUCID_LAUNCH_B("lucid_attn_bwd_dq_f32_kernel", (lucid::lucid_attn_bwd_dq_kernel<D, true, true, RW, WGR>), gq, bq,
                 st, f.qh, cq, f.kch, ck, f.vpb, w.doh, cq, lse, w.delta, f.mass, (float*)dq, S(dqs), Hq, Hkv, T,
                 BHq, scale, lo, f.vpbl);
  return LUCID_OK;
}

// The preconditioner part: dV = P^-T dV' (w.dvp, counters zeroed), then dK (fp32) with the
// softmax part dka added (null: none).
template <int D>
int launch_precond_bwd_f32(const FwdWs& f, void* dk, const int64_t* dks, void* dv, const int64_t* dvs,
                           const BwdWs& w, const float* dka, int B, int Hkv, int T, float scale, float dn,
                           hipStream_t st) {
  const int BH = B * Hkv;
  const lucid::Strides ck = rows_strides(Hkv, T, D);
  lucid::Lo lo{};
  lo.k = f.kl;
  lo.kt = f.ktl;
  auto col_chain = [&](auto dac) -> int {  // over the active head-dim columns
    LUCID_LAUNCH("lucid_precond_bwd_col_f32_kernel",
                 (lucid::lucid_precond_bwd_col_kernel<D, true, true, decltype(dac)::value>), dim3((T / 128) * BH), st,
                 f.kh, ck, Hkv, T, BH, f.rinv, nullptr, scale, f.kt, f.vpb, f.vpbl, f.pinv, f.mass, w.dvp, w.dvb,
                 w.dvbl, (float*)dv, S(dvs), w.colsum, w.counters, lo);
    return LUCID_OK;
  };
  int rc_col;
  if constexpr (D == 128) {
    const int da = active_dims<D>(dn);
    rc_col = da == 80   ? col_chain(std::integral_constant<int, 80>{})
             : da == 96 ? col_chain(std::integral_constant<int, 96>{})
                        : col_chain(std::integral_constant<int, D>{});
  } else {
    rc_col = col_chain(std::integral_constant<int, D>{});
  }
  if (rc_col) return rc_col;
  constexpr int NT = D == 128 ? 1 : 2;  // head dim 128: one n-tile per wave (registers)
  LUCID_LAUNCH("lucid_precond_bwd_row_f32_kernel", (lucid::lucid_precond_bwd_row_kernel<D, true, true, NT>),
               dim3(((T + 128 * NT - 1) / (128 * NT)) * BH), st, f.kh, ck, Hkv, T, BH, f.rinv, nullptr, scale, dn,
               f.vpb, f.vpbl, w.dvb, w.dvbl, f.mass, w.colsum, dka, (float*)dk, S(dks), lo);
  return LUCID_OK;
}

template <int D>
int launch_bwd_f32(const void* dout, const int64_t* dos, const void* o, const int64_t* os, const float* lse,
                   const FwdWs& f, void* dq, const int64_t* dqs, void* dk, const int64_t* dks, void* dv,
                   const int64_t* dvs, const BwdWs& w, int B, int Hq, int Hkv, int T, float scale, float dn,
                   hipStream_t st) {
  if (int rc = launch_attn_bwd_f32<D>(dout, dos, o, os, lse, f, dq, dqs, w, B, Hq, Hkv, T, scale, dn, st)) return rc;
  return launch_precond_bwd_f32<D>(f, dk, dks, dv, dvs, w, w.dka, B, Hkv, T, scale, dn, st);
}

// eager_lucid_attention_forward on fp32 Q, K and V': the centred keys, the V' pair and
// layouts, then the attention (the layout pass's 1/rms, read only by the row-mass pass,
// which the forced precision skips, comes from the centred keys).
template <int D>
int launch_attn_vp_fwd_f32(const void* q, const int64_t* qs, const void* k, const int64_t* ks, const void* vp,
                           const int64_t* vs, void* o, const int64_t* os, float* lse, const FwdWs& w, int B, int Hq,
                           int Hkv, int T, float eps, float scale, float dn, hipStream_t st) {
  const int BH = B * Hkv;
  if (int rc = launch_centered_keys<D>(k, ks, w, B, Hkv, T, st)) return rc;
  LUCID_LAUNCH("lucid_vp_layout_f32_kernel", (lucid::lucid_vp_layout_kernel<D, float, true>), dim3(T / 64, BH), st,
               w.kch, rows_strides(Hkv, T, D), (const float*)vp, S(vs), Hkv, T, eps, dn, w.rinv, w.vpb, w.vpt, w.mass,
               kForceExact, w.vpbl, w.vptl);
  return launch_attn_fwd_f32<D>(q, qs, o, os, lse, w, B, Hq, Hkv, T, scale, dn, st);
}

template <int D>
int launch_attn_vp_bwd_f32(const void* dout, const int64_t* dos, const void* o, const int64_t* os, const float* lse,
                           const FwdWs& f, void* dq, const int64_t* dqs, void* dk, const int64_t* dks, void* dvp,
                           const int64_t* dvps, const BwdWs& w, int B, int Hq, int Hkv, int T, float scale,
                           float dn, hipStream_t st) {
  const int BH = B * Hkv;
  if (int rc = launch_attn_bwd_f32<D>(dout, dos, o, os, lse, f, dq, dqs, w, B, Hq, Hkv, T, scale, dn, st)) return rc;
  LUCID_LAUNCH("lucid_rows_out_kernel", (lucid::lucid_rows_out_kernel<D, float>), dim3(T / 64, BH), st, w.dka,
               (float*)dk, S(dks), Hkv, T, 1.f);
  LUCID_LAUNCH("lucid_rows_out_kernel", (lucid::lucid_rows_out_kernel<D, float>), dim3(T / 64, BH), st, w.dvp,
               (float*)dvp, S(dvps), Hkv, T, 1.f);
  return LUCID_OK;
}

// Gradient of get_v_prime on fp32 inputs: dV' (fp32, strided) in, fp32 dK and dV out.
template <int D>
int launch_precond_only_bwd_f32(const void* dvp, const int64_t* dvps, const FwdWs& f, void* dk, const int64_t* dks,
                                void* dv, const int64_t* dvs, const BwdWs& w, int B, int Hkv, int T, float scale,
                                float dn, hipStream_t st) {
  LUCID_LAUNCH("lucid_rows_in_kernel", (lucid::lucid_rows_in_kernel<D, float>), dim3(T / 64, B * Hkv), st,
               (const float*)dvp, S(dvps), w.dvp, Hkv, T, w.counters);
  return launch_precond_bwd_f32<D>(f, dk, dks, dv, dvs, w, nullptr, B, Hkv, T, scale, dn, st);
}

// Decoding: split the cached sequence so that one resident round of split workgroups
// runs (at least 64 keys per split): the split kernel holds two workgroups per CU at
// head dim 128 (66 KB of LDS each) and four at 64, on 256 CUs.  Monotone in Tp, so the
// workspace sized for the capacity covers every call.
int decode_splits(int BH, int Tp, int D) {
  if (Tp <= 0) return 0;
  const int wgs = padded_dim(D) == 128 ? 512 : 1024;
  const int want = (wgs + BH - 1) / BH, most = (Tp + 63) / 64;
  return want < most ? want : most;
}

// Tokens per split/combine pass: the L (G + 1) columns of one 32-column score tile.
int decode_pass_tokens(int G) { return 32 / (G + 1); }

// Query heads per kv head are decoded in chunks of at most 31 (a chunk's query columns and
// the preconditioner row of each token share one 32-column score tile): G <= 31 is one
// chunk, larger groups split into equal chunks (the last may be smaller), all run with the
// token passes of the largest so that every chunk computes the same V' rows.
struct DecodeGroups {
  int chunks, gs;  // number of chunks, query heads per chunk (the largest)
};
DecodeGroups decode_groups(int G) {
  const int n = (G + 30) / 31;
  return DecodeGroups{n, (G + n - 1) / n};
}

lucid::DecodePartials carve_decode(void* base, int BH, int G, int L, int nsplit, int D, size_t* bytes) {
  D = padded_dim(D);
  lucid::DecodePartials w{};
  size_t off = 0;
  char* p = static_cast<char*>(base);
  auto take = [&](size_t n) {
    char* r = p ? p + off : nullptr;
    off += align256(n);
    return r;
  };
  const size_t ns = nsplit > 0 ? nsplit : 1;
  w.a = reinterpret_cast<float*>(take(ns * BH * L * D * 4));
  w.m = reinterpret_cast<float*>(take(ns * BH * L * G * 4));
  w.l = reinterpret_cast<float*>(take(ns * BH * L * G * 4));
  w.o = reinterpret_cast<float*>(take(ns * BH * L * G * D * 4));
  if (bytes) *bytes = off;
  return w;
}

// Partials of one pass of at most `L` tokens with a cache that grows to `T_end` rows (one
// chunk of query heads at a time: the chunks run in turn on the same partials).
size_t decode_ws_bytes(int BH, int G, int L, int T_end, int D) {
  const int Gs = decode_groups(G).gs;
  const int Lp = L < decode_pass_tokens(Gs) ? L : decode_pass_tokens(Gs);
  size_t n = 0;
  carve_decode(nullptr, BH, Gs, Lp, decode_splits(BH, T_end, D), D, &n);
  return n;
}

// L new tokens in passes of LM tokens: each pass reads the cache once (split kernel) and
// appends its tokens (combine kernel), so the next pass sees them.  The Gs query heads
// g0 .. g0+Gs-1 of each kv head's Gt; G > 0: the instance for Gs = G.
template <int D, int G>
int launch_decode(const void* q, const int64_t* qs, const void* k, const int64_t* ks, const void* v,
                  const int64_t* vs, void* kc, const int64_t* kcs, void* vc, const int64_t* vcs, void* o,
                  const int64_t* os, float* vp_new, void* ws, int B, int Hkv, int L, int Tp, float scale, float eps,
                  float dn, hipStream_t st, int Gs, int Gt, int g0, int LM, int write_cache) {
  const int BH = B * Hkv;
  for (int t0 = 0; t0 < L; t0 += LM) {
    const int Lc = L - t0 < LM ? L - t0 : LM, Tc = Tp + t0;
    const int ns = decode_splits(BH, Tc, D);
    const lucid::DecodePartials part = carve_decode(ws, BH, Gs, Lc, ns, D, nullptr);
    const bf16* qc = (const bf16*)q + t0 * qs[2];
    const bf16* kn = (const bf16*)k + t0 * ks[2];
    const bf16* vn = (const bf16*)v + t0 * vs[2];
    if (ns > 0) {
      const int KS = (Tc + ns - 1) / ns;
      LUCID_LAUNCH("lucid_decode_split_kernel", (lucid::lucid_decode_split_kernel<D, G>), dim3(ns, BH), st, qc,
                   S(qs), kn, S(ks), (const bf16*)kc, S(kcs), (const bf16*)vc, S(vcs), Hkv, Tc, KS, Lc, scale, eps,
                   dn, part, Gs, Gt, g0);
    }
    LUCID_LAUNCH("lucid_decode_combine_kernel", (lucid::lucid_decode_combine_kernel<D, G>), dim3(BH, Gs), st, ns,
                 Lc, qc, S(qs), kn, S(ks), vn, S(vs), (bf16*)kc, S(kcs), (bf16*)vc, S(vcs),
                 (bf16*)o + t0 * os[2], S(os), vp_new + (size_t)t0 * D, L, Hkv, Tc, scale, eps, dn, part, Gs, Gt, g0,
                 write_cache);
  }
  return LUCID_OK;
}

template <int D>
int decode_dispatch_g(int G, const void* q, const int64_t* qs, const void* k, const int64_t* ks, const void* v,
                      const int64_t* vs, void* kc, const int64_t* kcs, void* vc, const int64_t* vcs, void* o,
                      const int64_t* os, float* vp_new, void* ws, int B, int Hkv, int L, int Tp, float scale,
                      float eps, float dn, hipStream_t st) {
#define LUCID_DECODE_G(GI) \
  launch_decode<D, GI>(q, qs, k, ks, v, vs, kc, kcs, vc, vcs, o, os, vp_new, ws, B, Hkv, L, Tp, scale, eps, dn, st, G, G, 0, \
                       decode_pass_tokens(G), 1)
  switch (G) {  // the common groupings as their own instances
    case 1: return LUCID_DECODE_G(1);
    case 2: return LUCID_DECODE_G(2);
    case 4: return LUCID_DECODE_G(4);
    case 8: return LUCID_DECODE_G(8);
    default: break;
  }
#undef LUCID_DECODE_G
  // any other group: the generic instance, in chunks of query heads above 31
  const DecodeGroups dg = decode_groups(G);
  const int LM = decode_pass_tokens(dg.gs);
  for (int c = 0; c < dg.chunks; ++c) {
    const int g0 = c * dg.gs, gs = G - g0 < dg.gs ? G - g0 : dg.gs;
    if (int rc = launch_decode<D, 0>(q, qs, k, ks, v, vs, kc, kcs, vc, vcs, o, os, vp_new, ws, B, Hkv, L, Tp, scale,
                                     eps, dn, st, gs, G, g0, LM, c == 0))
      return rc;
  }
  return LUCID_OK;
}

int check_decode_args(const void* q, const int64_t* qs, const void* k, const int64_t* ks, const void* v,
                      const int64_t* vs, const void* kc, const int64_t* kcs, const void* vc, const int64_t* vcs,
                      const void* o, const int64_t* os, const float* vp_new, int B, int Hq, int Hkv, int L,
                      int T_past, int T_cap, int D) {
  if (B <= 0 || Hq <= 0 || Hkv <= 0) return fail("B, Hq and Hkv must be positive");
  if (L <= 0) return fail("the number of new tokens must be positive");
  if (D < 1 || D > 128) return fail("head_dim must be in [1, 128], got " + std::to_string(D));
  if (Hq % Hkv != 0) return fail("Hq must be a multiple of Hkv");
  if (T_past < 0 || (int64_t)T_past + L > T_cap)
    return fail("the cache is too small: T_past + L must be within T_cap (T_past >= 0)");
  if (int rc = check_tensor("q", q, qs)) return rc;
  if (int rc = check_tensor("k", k, ks)) return rc;
  if (int rc = check_tensor("v", v, vs)) return rc;
  if (int rc = check_tensor("k_cache", kc, kcs)) return rc;
  if (int rc = check_tensor("vp_cache", vc, vcs)) return rc;
  if (int rc = check_tensor("o", o, os)) return rc;
  if (!vp_new) return fail("vp_new must be non-null");
  return LUCID_OK;
}

// ---- allocation-free decoding (lucid_decode_noalloc) ----
// The split partials live in this file-scope device array instead of a caller workspace.
// Each GPU the library runs on holds its own copy until the process ends; host code must
// use the address hipGetSymbolAddress returns for the current device, never the array's
// name (a host-side stand-in).  Every call on a GPU shares that GPU's array: calls that
// overlap on one GPU race.  The split pass writes every partial it combines, so nothing
// has to start at zero.
constexpr size_t kDecodeScratchBytes = size_t(4) << 20;
static __device__ __align__(256) unsigned char scratch[kDecodeScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the current device, looked up once per device.
int decode_scratch(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    g_last_error = std::string("hipGetDevice: ") + hipGetErrorString(e);
    return LUCID_EHIP + (int)e;
  }
  if (dev < 0 || dev >= kMaxDevices) return fail("device index " + std::to_string(dev) + " out of range");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      g_last_error = std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e);
      return LUCID_EHIP + (int)e;
    }
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return LUCID_OK;
}

int decode_impl(const void* q, const int64_t* q_strides, const void* k, const int64_t* k_strides, const void* v,
                const int64_t* v_strides, void* k_cache, const int64_t* k_cache_strides, void* vp_cache,
                const int64_t* vp_cache_strides, void* o, const int64_t* o_strides, float* vp_new, void* ws, int B,
                int Hq, int Hkv, int L, int T_past, int D, float scale, float eps, void* stream) {
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (padded_dim(D) == 64)
    return decode_dispatch_g<64>(Hq / Hkv, q, q_strides, k, k_strides, v, v_strides, k_cache, k_cache_strides,
                                 vp_cache, vp_cache_strides, o, o_strides, vp_new, ws, B, Hkv, L, T_past, scale, eps,
                                 (float)D, st);
  return decode_dispatch_g<128>(Hq / Hkv, q, q_strides, k, k_strides, v, v_strides, k_cache, k_cache_strides,
                                vp_cache, vp_cache_strides, o, o_strides, vp_new, ws, B, Hkv, L, T_past, scale, eps,
                                (float)D, st);
}

// get_v_prime with k_norm (dn = the head dim) or on keys already normalised (dn = 0, the
// Lucid_Tril_Solver seam: 1/rms is 1 and the backward returns dK^ itself).
int get_v_prime_impl(const void* k, const int64_t* k_strides, const void* v, const int64_t* v_strides, float* vprime,
                     void* fwd_ws, int B, int Hkv, int T, int D, float scale, float eps, float dn, void* stream) {
  g_last_error.clear();
  if (int rc = check_dims(B, Hkv, Hkv, T, D)) return rc;
  if (int rc = check_tensor("k", k, k_strides)) return rc;
  if (int rc = check_tensor("v", v, v_strides)) return rc;
  if (!vprime || !fwd_ws) return fail("vprime and fwd_ws must be non-null");
  if (int rc = check_ws("fwd_ws", fwd_ws)) return rc;
  if (int rc = chain_check()) return rc;
  const FwdWs w = carve_fwd(fwd_ws, B, Hkv, Hkv, T, D);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (padded_dim(D) == 64) return launch_precond_fwd<64>(k, k_strides, v, v_strides, vprime, w, B, Hkv, T, scale, eps, dn, st);
  return launch_precond_fwd<128>(k, k_strides, v, v_strides, vprime, w, B, Hkv, T, scale, eps, dn, st);
}

int precond_bwd_impl(const void* k, const int64_t* k_strides, const void* dvprime, const int64_t* dvprime_strides,
                     int dvprime_f32, const void* fwd_ws, void* dk, const int64_t* dk_strides, void* dv,
                     const int64_t* dv_strides, void* bwd_ws, int B, int Hkv, int T, int D, float scale, float dn,
                     void* stream) {
  g_last_error.clear();
  if (int rc = check_dims(B, Hkv, Hkv, T, D)) return rc;
  if (int rc = check_tensor("k", k, k_strides)) return rc;
  if (int rc = check_tensor("dvprime", dvprime, dvprime_strides)) return rc;
  if (int rc = check_tensor("dk", dk, dk_strides)) return rc;
  if (int rc = check_tensor("dv", dv, dv_strides)) return rc;
  if (!fwd_ws || !bwd_ws) return fail("fwd_ws and bwd_ws must be non-null");
  if (int rc = check_ws("fwd_ws", fwd_ws)) return rc;
  if (int rc = check_ws("bwd_ws", bwd_ws)) return rc;
  if (int rc = chain_check()) return rc;
  const FwdWs f = carve_fwd(const_cast<void*>(fwd_ws), B, Hkv, Hkv, T, D);
  const BwdWs w = carve_seam_bwd(bwd_ws, B, Hkv, Hkv, T, D, false);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (padded_dim(D) == 64)
    return launch_precond_only_bwd<64>(k, k_strides, dvprime, dvprime_strides, dvprime_f32, f, dk, dk_strides, dv,
                                       dv_strides, w, B, Hkv, T, scale, dn, st);
  return launch_precond_only_bwd<128>(k, k_strides, dvprime, dvprime_strides, dvprime_f32, f, dk, dk_strides, dv,
                                      dv_strides, w, B, Hkv, T, scale, dn, st);
}

int get_v_prime_f32_impl(const float* k, const int64_t* k_strides, const float* v, const int64_t* v_strides,
                         float* vprime, void* fwd_ws, int B, int Hkv, int T, int D, float scale, float eps, float dn,
                         void* stream) {
  g_last_error.clear();
  if (int rc = check_dims(B, Hkv, Hkv, T, D)) return rc;
  if (int rc = check_tensor("k", k, k_strides)) return rc;
  if (int rc = check_tensor("v", v, v_strides)) return rc;
  if (!vprime || !fwd_ws) return fail("vprime and fwd_ws must be non-null");
  if (int rc = check_ws("fwd_ws", fwd_ws)) return rc;
  if (int rc = chain_check()) return rc;
  const FwdWs w = carve_fwd(fwd_ws, B, Hkv, Hkv, T, D, true, false);
  return (padded_dim(D) == 64 ? launch_precond_fwd_f32<64> : launch_precond_fwd_f32<128>)(k, k_strides, v, v_strides, vprime, w, B, Hkv, T, scale, eps, dn,
                                static_cast<hipStream_t>(stream));
}

int precond_bwd_f32_impl(const float* dvprime, const int64_t* dvprime_strides, const void* fwd_ws, float* dk,
                         const int64_t* dk_strides, float* dv, const int64_t* dv_strides, void* bwd_ws, int B, int Hkv,
                         int T, int D, float scale, float dn, void* stream) {
  g_last_error.clear();
  if (int rc = check_dims(B, Hkv, Hkv, T, D)) return rc;
  if (int rc = check_tensor("dvprime", dvprime, dvprime_strides)) return rc;
  if (int rc = check_tensor("dk", dk, dk_strides)) return rc;
  if (int rc = check_tensor("dv", dv, dv_strides)) return rc;
  if (!fwd_ws || !bwd_ws) return fail("fwd_ws and bwd_ws must be non-null");
  if (int rc = check_ws("fwd_ws", fwd_ws)) return rc;
  if (int rc = check_ws("bwd_ws", bwd_ws)) return rc;
  if (int rc = chain_check()) return rc;
  const FwdWs f = carve_fwd(const_cast<void*>(fwd_ws), B, Hkv, Hkv, T, D, true, false);
  const BwdWs w = carve_seam_bwd(bwd_ws, B, Hkv, Hkv, T, D, false);
  return (padded_dim(D) == 64 ? launch_precond_only_bwd_f32<64> : launch_precond_only_bwd_f32<128>)(dvprime, dvprime_strides, f, dk, dk_strides, dv, dv_strides, w, B, Hkv, T,
                                     scale, dn, static_cast<hipStream_t>(stream));
}

}  // namespace

extern "C" {

size_t lucid_decode_workspace_bytes(int B, int Hq, int Hkv, int T_cap, int D) {
  if (B <= 0 || Hkv <= 0 || Hq <= 0 || Hq % Hkv || T_cap < 0) return 0;
  return decode_ws_bytes(B * Hkv, Hq / Hkv, 1, T_cap, D);
}

size_t lucid_decode_tokens_workspace_bytes(int B, int Hq, int Hkv, int L, int T_cap, int D) {
  if (B <= 0 || Hkv <= 0 || Hq <= 0 || Hq % Hkv || T_cap < 0 || L <= 0) return 0;
  return decode_ws_bytes(B * Hkv, Hq / Hkv, L, T_cap, D);
}

int lucid_decode(const void* q, const int64_t* q_strides, const void* k, const int64_t* k_strides, const void* v,
                 const int64_t* v_strides, void* k_cache, const int64_t* k_cache_strides, void* vp_cache,
                 const int64_t* vp_cache_strides, void* o, const int64_t* o_strides, float* vp_new, void* ws, int B,
                 int Hq, int Hkv, int T_past, int T_cap, int D, float scale, float eps, void* stream) {
  return lucid_decode_tokens(q, q_strides, k, k_strides, v, v_strides, k_cache, k_cache_strides, vp_cache,
                             vp_cache_strides, o, o_strides, vp_new, ws, B, Hq, Hkv, 1, T_past, T_cap, D, scale, eps,
                             stream);
}

int lucid_decode_tokens(const void* q, const int64_t* q_strides, const void* k, const int64_t* k_strides,
                        const void* v, const int64_t* v_strides, void* k_cache, const int64_t* k_cache_strides,
                        void* vp_cache, const int64_t* vp_cache_strides, void* o, const int64_t* o_strides,
                        float* vp_new, void* ws, int B, int Hq, int Hkv, int L, int T_past, int T_cap, int D,
                        float scale, float eps, void* stream) {
  g_last_error.clear();
  if (int rc = check_decode_args(q, q_strides, k, k_strides, v, v_strides, k_cache, k_cache_strides, vp_cache,
                                 vp_cache_strides, o, o_strides, vp_new, B, Hq, Hkv, L, T_past, T_cap, D))
    return rc;
  if (!ws) return fail("ws must be non-null");
  if (int rc = check_ws("ws", ws)) return rc;
  return decode_impl(q, q_strides, k, k_strides, v, v_strides, k_cache, k_cache_strides, vp_cache, vp_cache_strides,
                     o, o_strides, vp_new, ws, B, Hq, Hkv, L, T_past, D, scale, eps, stream);
}

int lucid_decode_noalloc(const void* q, const int64_t* q_strides, const void* k, const int64_t* k_strides,
                         const void* v, const int64_t* v_strides, void* k_cache, const int64_t* k_cache_strides,
                         void* vp_cache, const int64_t* vp_cache_strides, void* o, const int64_t* o_strides,
                         float* vp_new, int B, int Hq, int Hkv, int T_past, int T_cap, int D, float scale, float eps,
                         void* stream) {
  g_last_error.clear();
  if (int rc = check_decode_args(q, q_strides, k, k_strides, v, v_strides, k_cache, k_cache_strides, vp_cache,
                                 vp_cache_strides, o, o_strides, vp_new, B, Hq, Hkv, 1, T_past, T_cap, D))
    return rc;
  const size_t need = decode_ws_bytes(B * Hkv, Hq / Hkv, 1, T_past, D);
  if (need > kDecodeScratchBytes)
    return fail("lucid_decode_noalloc needs " + std::to_string(need) + " bytes of scratch for these sizes, above its " +
                std::to_string(kDecodeScratchBytes) + "-byte static scratch; call lucid_decode with a workspace");
  void* ws = nullptr;
  if (int rc = decode_scratch(&ws)) return rc;
  return decode_impl(q, q_strides, k, k_strides, v, v_strides, k_cache, k_cache_strides, vp_cache, vp_cache_strides,
                     o, o_strides, vp_new, ws, B, Hq, Hkv, 1, T_past, D, scale, eps, stream);
}


int lucid_abi_version(void) { return 6; }

int lucid_set_precision(int mode) {
  g_last_error.clear();
  if (mode != LUCID_PRECISION_AUTO && mode != LUCID_PRECISION_FAST && mode != LUCID_PRECISION_EXACT)
    return fail("precision mode must be LUCID_PRECISION_AUTO, _FAST or _EXACT, got " + std::to_string(mode));
  g_precision = mode;
  return LUCID_OK;
}

int lucid_get_precision(void) { return g_precision; }

int lucid_set_fused_forward(int on) {
  g_last_error.clear();
  g_fused_fwd = on != 0;
  return LUCID_OK;
}

int lucid_get_fused_forward(void) { return g_fused_fwd ? 1 : 0; }

int lucid_chain_status(void) {
  g_last_error.clear();
  return chain_check();
}

int lucid_set_chain_wait_limit(double seconds) {
  g_last_error.clear();
  if (!(seconds > 0.0)) return fail("the chain wait limit must be positive");
  chain_guard::set_limit(seconds);
  return LUCID_OK;
}

size_t lucid_fwd_workspace_mass_offset(int B, int Hq, int Hkv, int T, int D) {
  char* base = reinterpret_cast<char*>(size_t(256));  // any non-null 256-aligned base
  return static_cast<size_t>(reinterpret_cast<char*>(carve_fwd(base, B, Hq, Hkv, T, D).mass) - base);
}

const char* lucid_last_error(void) { return g_last_error.c_str(); }

size_t lucid_fwd_workspace_bytes(int B, int Hq, int Hkv, int T, int D) {
  return carve_fwd(nullptr, B, Hq, Hkv, T, D).bytes;
}

size_t lucid_bwd_workspace_bytes(int B, int Hq, int Hkv, int T, int D) {
  return carve_bwd(nullptr, B, Hq, Hkv, T, D).bytes;
}

int lucid_get_v_prime(const void* k, const int64_t* k_strides, const void* v, const int64_t* v_strides,
                      float* vprime, void* fwd_ws, int B, int Hkv, int T, int D, float scale, float eps,
                      void* stream) {
  return get_v_prime_impl(k, k_strides, v, v_strides, vprime, fwd_ws, B, Hkv, T, D, scale, eps, (float)D, stream);
}

int lucid_tril_solve(const void* key_hat, const int64_t* k_strides, const void* v, const int64_t* v_strides,
                     float* vprime, void* fwd_ws, int B, int Hkv, int T, int D, float scale, void* stream) {
  return get_v_prime_impl(key_hat, k_strides, v, v_strides, vprime, fwd_ws, B, Hkv, T, D, scale, 0.f, 0.f, stream);
}

int lucid_tril_solve_bwd(const void* key_hat, const int64_t* k_strides, const void* dvprime,
                         const int64_t* dvprime_strides, int dvprime_f32, const void* fwd_ws, void* dk,
                         const int64_t* dk_strides, void* dv, const int64_t* dv_strides, void* bwd_ws, int B, int Hkv,
                         int T, int D, float scale, void* stream) {
  return precond_bwd_impl(key_hat, k_strides, dvprime, dvprime_strides, dvprime_f32, fwd_ws, dk, dk_strides, dv,
                          dv_strides, bwd_ws, B, Hkv, T, D, scale, 0.f, stream);
}

int lucid_tril_solve_f32(const float* key_hat, const int64_t* k_strides, const float* v, const int64_t* v_strides,
                         float* vprime, void* fwd_ws, int B, int Hkv, int T, int D, float scale, void* stream) {
  return get_v_prime_f32_impl(key_hat, k_strides, v, v_strides, vprime, fwd_ws, B, Hkv, T, D, scale, 0.f, 0.f,
                              stream);
}

int lucid_tril_solve_bwd_f32(const float* dvprime, const int64_t* dvprime_strides, const void* fwd_ws, float* dk,
                             const int64_t* dk_strides, float* dv, const int64_t* dv_strides, void* bwd_ws, int B,
                             int Hkv, int T, int D, float scale, void* stream) {
  return precond_bwd_f32_impl(dvprime, dvprime_strides, fwd_ws, dk, dk_strides, dv, dv_strides, bwd_ws, B, Hkv, T, D,
                              scale, 0.f, stream);
}

int lucid_attn_fwd(const void* q, const int64_t* q_strides, const void* k, const int64_t* k_strides,
                   const void* v, const int64_t* v_strides, void* o, const int64_t* o_strides, float* vprime,
                   float* lse, void* fwd_ws, int B, int Hq, int Hkv, int T, int D, float scale, float eps,
                   void* stream) {
  g_last_error.clear();
  if (int rc = check_dims(B, Hq, Hkv, T, D)) return rc;
  if (int rc = check_tensor("q", q, q_strides)) return rc;
  if (int rc = check_tensor("k", k, k_strides)) return rc;
  if (int rc = check_tensor("v", v, v_strides)) return rc;
  if (int rc = check_tensor("o", o, o_strides)) return rc;
  if (!vprime || !lse || !fwd_ws) return fail("vprime, lse and fwd_ws must be non-null");
  if (int rc = check_ws("fwd_ws", fwd_ws)) return rc;
  if (int rc = chain_check()) return rc;
  const FwdWs w = carve_fwd(fwd_ws, B, Hq, Hkv, T, D);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (padded_dim(D) == 64)
    return launch_fwd<64>(q, q_strides, k, k_strides, v, v_strides, o, o_strides, vprime, lse, w, B, Hq, Hkv, T,
                          scale, eps, (float)D, st);
  return launch_fwd<128>(q, q_strides, k, k_strides, v, v_strides, o, o_strides, vprime, lse, w, B, Hq, Hkv, T,
                         scale, eps, (float)D, st);
}

int lucid_attn_bwd(const void* dout, const int64_t* do_strides, const void* q, const int64_t* q_strides,
                   const void* k, const int64_t* k_strides, const void* o, const int64_t* o_strides,
                   const float* lse, const void* fwd_ws, void* dq, const int64_t* dq_strides, void* dk,
                   const int64_t* dk_strides, void* dv, const int64_t* dv_strides, void* bwd_ws, int B, int Hq,
                   int Hkv, int T, int D, float scale, float eps, void* stream) {
  (void)eps;
  g_last_error.clear();
  if (int rc = check_dims(B, Hq, Hkv, T, D)) return rc;
  if (int rc = check_tensor("dout", dout, do_strides)) return rc;
  if (int rc = check_tensor("q", q, q_strides)) return rc;
  if (int rc = check_tensor("k", k, k_strides)) return rc;
  if (int rc = check_tensor("o", o, o_strides)) return rc;
  if (int rc = check_tensor("dq", dq, dq_strides)) return rc;
  if (int rc = check_tensor("dk", dk, dk_strides)) return rc;
  if (int rc = check_tensor("dv", dv, dv_strides)) return rc;
  if (!lse || !fwd_ws || !bwd_ws) return fail("lse, fwd_ws and bwd_ws must be non-null");
  if (int rc = check_ws("fwd_ws", fwd_ws)) return rc;
  if (int rc = check_ws("bwd_ws", bwd_ws)) return rc;
  if (int rc = chain_check()) return rc;
  const FwdWs f = carve_fwd(const_cast<void*>(fwd_ws), B, Hq, Hkv, T, D);
  const BwdWs w = carve_bwd(bwd_ws, B, Hq, Hkv, T, D);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (padded_dim(D) == 64)
    return launch_bwd<64>(dout, do_strides, q, q_strides, k, k_strides, o, o_strides, lse, f, dq, dq_strides, dk,
                          dk_strides, dv, dv_strides, w, B, Hq, Hkv, T, scale, (float)D, st);
  return launch_bwd<128>(dout, do_strides, q, q_strides, k, k_strides, o, o_strides, lse, f, dq, dq_strides, dk,
                         dk_strides, dv, dv_strides, w, B, Hq, Hkv, T, scale, (float)D, st);
}

size_t lucid_fwd_f32_workspace_bytes(int B, int Hq, int Hkv, int T, int D) {
  return carve_fwd(nullptr, B, Hq, Hkv, T, D, true).bytes;
}

size_t lucid_bwd_f32_workspace_bytes(int B, int Hq, int Hkv, int T, int D) {
  return carve_bwd(nullptr, B, Hq, Hkv, T, D, true).bytes;
}

int lucid_attn_fwd_f32(const float* q, const int64_t* q_strides, const float* k, const int64_t* k_strides,
                       const float* v, const int64_t* v_strides, float* o, const int64_t* o_strides, float* vprime,
                       float* lse, void* fwd_ws, int B, int Hq, int Hkv, int T, int D, float scale, float eps,
                       void* stream) {
  g_last_error.clear();
  if (int rc = check_dims(B, Hq, Hkv, T, D)) return rc;
  if (int rc = check_tensor("q", q, q_strides)) return rc;
  if (int rc = check_tensor("k", k, k_strides)) return rc;
  if (int rc = check_tensor("v", v, v_strides)) return rc;
  if (int rc = check_tensor("o", o, o_strides)) return rc;
  if (!vprime || !lse || !fwd_ws) return fail("vprime, lse and fwd_ws must be non-null");
  if (int rc = check_ws("fwd_ws", fwd_ws)) return rc;
  if (int rc = chain_check()) return rc;
  const FwdWs w = carve_fwd(fwd_ws, B, Hq, Hkv, T, D, true);
  return (padded_dim(D) == 64 ? launch_fwd_f32<64> : launch_fwd_f32<128>)(q, q_strides, k, k_strides, v, v_strides, o, o_strides, vprime, lse, w, B, Hq, Hkv, T,
                        scale, eps, (float)D, static_cast<hipStream_t>(stream));
}

int lucid_attn_bwd_f32(const float* dout, const int64_t* do_strides, const float* o, const int64_t* o_strides,
                       const float* lse, const void* fwd_ws, float* dq, const int64_t* dq_strides, float* dk,
                       const int64_t* dk_strides, float* dv, const int64_t* dv_strides, void* bwd_ws, int B, int Hq,
                       int Hkv, int T, int D, float scale, void* stream) {
  g_last_error.clear();
  if (int rc = check_dims(B, Hq, Hkv, T, D)) return rc;
  if (int rc = check_tensor("dout", dout, do_strides)) return rc;
  if (int rc = check_tensor("o", o, o_strides)) return rc;
  if (int rc = check_tensor("dq", dq, dq_strides)) return rc;
  if (int rc = check_tensor("dk", dk, dk_strides)) return rc;
  if (int rc = check_tensor("dv", dv, dv_strides)) return rc;
  if (!lse || !fwd_ws || !bwd_ws) return fail("lse, fwd_ws and bwd_ws must be non-null");
  if (int rc = check_ws("fwd_ws", fwd_ws)) return rc;
  if (int rc = check_ws("bwd_ws", bwd_ws)) return rc;
  if (int rc = chain_check()) return rc;
  const FwdWs f = carve_fwd(const_cast<void*>(fwd_ws), B, Hq, Hkv, T, D, true);
  const BwdWs w = carve_bwd(bwd_ws, B, Hq, Hkv, T, D, true);
  return (padded_dim(D) == 64 ? launch_bwd_f32<64> : launch_bwd_f32<128>)(dout, do_strides, o, o_strides, lse, f, dq, dq_strides, dk, dk_strides, dv, dv_strides, w,
                        B, Hq, Hkv, T, scale, (float)D, static_cast<hipStream_t>(stream));
}

size_t lucid_v_prime_f32_workspace_bytes(int B, int Hkv, int T, int D) {
  return carve_fwd(nullptr, B, Hkv, Hkv, T, D, true, false).bytes;
}

int lucid_get_v_prime_f32(const float* k, const int64_t* k_strides, const float* v, const int64_t* v_strides,
                          float* vprime, void* fwd_ws, int B, int Hkv, int T, int D, float scale, float eps,
                          void* stream) {
  return get_v_prime_f32_impl(k, k_strides, v, v_strides, vprime, fwd_ws, B, Hkv, T, D, scale, eps, (float)D, stream);
}

int lucid_precond_bwd_f32(const float* dvprime, const int64_t* dvprime_strides, const void* fwd_ws, float* dk,
                          const int64_t* dk_strides, float* dv, const int64_t* dv_strides, void* bwd_ws, int B,
                          int Hkv, int T, int D, float scale, void* stream) {
  return precond_bwd_f32_impl(dvprime, dvprime_strides, fwd_ws, dk, dk_strides, dv, dv_strides, bwd_ws, B, Hkv, T, D,
                              scale, (float)D, stream);
}

size_t lucid_attn_vp_fwd_f32_workspace_bytes(int B, int Hq, int Hkv, int T, int D) {
  return carve_attn_vp(nullptr, B, Hq, Hkv, T, D, true).bytes;
}

int lucid_attn_vp_fwd_f32(const float* q, const int64_t* q_strides, const float* k, const int64_t* k_strides,
                          const float* vprime, const int64_t* vprime_strides, float* o, const int64_t* o_strides,
                          float* lse, void* ws, int B, int Hq, int Hkv, int T, int D, float scale, float eps,
                          void* stream) {
  g_last_error.clear();
  if (int rc = check_dims(B, Hq, Hkv, T, D)) return rc;
  if (int rc = check_tensor("q", q, q_strides)) return rc;
  if (int rc = check_tensor("k", k, k_strides)) return rc;
  if (int rc = check_tensor("vprime", vprime, vprime_strides)) return rc;
  if (int rc = check_tensor("o", o, o_strides)) return rc;
  if (!lse || !ws) return fail("lse and ws must be non-null");
  if (int rc = check_ws("ws", ws)) return rc;
  const FwdWs w = carve_attn_vp(ws, B, Hq, Hkv, T, D, true);
  return (padded_dim(D) == 64 ? launch_attn_vp_fwd_f32<64> : launch_attn_vp_fwd_f32<128>)(q, q_strides, k, k_strides, vprime, vprime_strides, o, o_strides, lse, w, B, Hq, Hkv,
                                T, eps, scale, (float)D, static_cast<hipStream_t>(stream));
}

size_t lucid_attn_vp_bwd_f32_workspace_bytes(int B, int Hq, int Hkv, int T, int D) {
  return carve_seam_bwd(nullptr, B, Hq, Hkv, T, D, true, true).bytes;
}

int lucid_attn_vp_bwd_f32(const float* dout, const int64_t* do_strides, const float* o, const int64_t* o_strides,
                          const float* lse, const void* fwd_ws, float* dq, const int64_t* dq_strides, float* dk,
                          const int64_t* dk_strides, float* dvprime, const int64_t* dvprime_strides, void* bwd_ws,
                          int B, int Hq, int Hkv, int T, int D, float scale, void* stream) {
  g_last_error.clear();
  if (int rc = check_dims(B, Hq, Hkv, T, D)) return rc;
  if (int rc = check_tensor("dout", dout, do_strides)) return rc;
  if (int rc = check_tensor("o", o, o_strides)) return rc;
  if (int rc = check_tensor("dq", dq, dq_strides)) return rc;
  if (int rc = check_tensor("dk", dk, dk_strides)) return rc;
  if (int rc = check_tensor("dvprime", dvprime, dvprime_strides)) return rc;
  if (!lse || !fwd_ws || !bwd_ws) return fail("lse, fwd_ws and bwd_ws must be non-null");
  if (int rc = check_ws("fwd_ws", fwd_ws)) return rc;
  if (int rc = check_ws("bwd_ws", bwd_ws)) return rc;
  const FwdWs f = carve_attn_vp(const_cast<void*>(fwd_ws), B, Hq, Hkv, T, D, true);
  const BwdWs w = carve_seam_bwd(bwd_ws, B, Hq, Hkv, T, D, true, true);
  return (padded_dim(D) == 64 ? launch_attn_vp_bwd_f32<64> : launch_attn_vp_bwd_f32<128>)(dout, do_strides, o, o_strides, lse, f, dq, dq_strides, dk, dk_strides, dvprime,
                                dvprime_strides, w, B, Hq, Hkv, T, scale, (float)D, static_cast<hipStream_t>(stream));
}

size_t lucid_attn_vp_fwd_workspace_bytes(int B, int Hq, int Hkv, int T, int D) {
  return carve_attn_vp(nullptr, B, Hq, Hkv, T, D).bytes;
}

int lucid_attn_vp_fwd(const void* q, const int64_t* q_strides, const void* k, const int64_t* k_strides,
                      const void* vprime, const int64_t* vprime_strides, int vprime_f32, void* o,
                      const int64_t* o_strides, float* lse, void* ws, int B, int Hq, int Hkv, int T, int D,
                      float scale, float eps, void* stream) {
  g_last_error.clear();
  if (int rc = check_dims(B, Hq, Hkv, T, D)) return rc;
  if (int rc = check_tensor("q", q, q_strides)) return rc;
  if (int rc = check_tensor("k", k, k_strides)) return rc;
  if (int rc = check_tensor("vprime", vprime, vprime_strides)) return rc;
  if (int rc = check_tensor("o", o, o_strides)) return rc;
  if (!lse || !ws) return fail("lse and ws must be non-null");
  if (int rc = check_ws("ws", ws)) return rc;
  const FwdWs w = carve_attn_vp(ws, B, Hq, Hkv, T, D);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (padded_dim(D) == 64)
    return launch_attn_vp_fwd<64>(q, q_strides, k, k_strides, vprime, vprime_strides, vprime_f32, o, o_strides, lse,
                                  w, B, Hq, Hkv, T, scale, eps, (float)D, st);
  return launch_attn_vp_fwd<128>(q, q_strides, k, k_strides, vprime, vprime_strides, vprime_f32, o, o_strides, lse,
                                 w, B, Hq, Hkv, T, scale, eps, (float)D, st);
}

size_t lucid_attn_vp_bwd_workspace_bytes(int B, int Hq, int Hkv, int T, int D) {
  return carve_seam_bwd(nullptr, B, Hq, Hkv, T, D, true).bytes;
}

int lucid_attn_vp_bwd(const void* dout, const int64_t* do_strides, const void* q, const int64_t* q_strides,
                      const void* k, const int64_t* k_strides, const void* o, const int64_t* o_strides,
                      const float* lse, const void* fwd_ws, void* dq, const int64_t* dq_strides, void* dk,
                      const int64_t* dk_strides, void* dvprime, const int64_t* dvprime_strides, int dvprime_f32,
                      void* bwd_ws, int B, int Hq, int Hkv, int T, int D, float scale, void* stream) {
  g_last_error.clear();
  if (int rc = check_dims(B, Hq, Hkv, T, D)) return rc;
  if (int rc = check_tensor("dout", dout, do_strides)) return rc;
  if (int rc = check_tensor("q", q, q_strides)) return rc;
  if (int rc = check_tensor("k", k, k_strides)) return rc;
  if (int rc = check_tensor("o", o, o_strides)) return rc;
  if (int rc = check_tensor("dq", dq, dq_strides)) return rc;
  if (int rc = check_tensor("dk", dk, dk_strides)) return rc;
  if (int rc = check_tensor("dvprime", dvprime, dvprime_strides)) return rc;
  if (!lse || !fwd_ws || !bwd_ws) return fail("lse, fwd_ws and bwd_ws must be non-null");
  if (int rc = check_ws("fwd_ws", fwd_ws)) return rc;
  if (int rc = check_ws("bwd_ws", bwd_ws)) return rc;
  const FwdWs f = carve_attn_vp(const_cast<void*>(fwd_ws), B, Hq, Hkv, T, D);
  const BwdWs w = carve_seam_bwd(bwd_ws, B, Hq, Hkv, T, D, true);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (padded_dim(D) == 64)
    return launch_attn_vp_bwd<64>(dout, do_strides, q, q_strides, k, k_strides, o, o_strides, lse, f, dq,
                                  dq_strides, dk, dk_strides, dvprime, dvprime_strides, dvprime_f32, w, B, Hq, Hkv,
                                  T, scale, (float)D, st);
  return launch_attn_vp_bwd<128>(dout, do_strides, q, q_strides, k, k_strides, o, o_strides, lse, f, dq, dq_strides,
                                 dk, dk_strides, dvprime, dvprime_strides, dvprime_f32, w, B, Hq, Hkv, T, scale,
                                 (float)D, st);
}

size_t lucid_precond_bwd_workspace_bytes(int B, int Hkv, int T, int D) {
  return carve_seam_bwd(nullptr, B, Hkv, Hkv, T, D, false).bytes;
}

int lucid_precond_bwd(const void* k, const int64_t* k_strides, const void* dvprime, const int64_t* dvprime_strides,
                      int dvprime_f32, const void* fwd_ws, void* dk, const int64_t* dk_strides, void* dv,
                      const int64_t* dv_strides, void* bwd_ws, int B, int Hkv, int T, int D, float scale,
                      void* stream) {
  return precond_bwd_impl(k, k_strides, dvprime, dvprime_strides, dvprime_f32, fwd_ws, dk, dk_strides, dv, dv_strides,
                          bwd_ws, B, Hkv, T, D, scale, (float)D, stream);
}

void lucid_profile_enable(int on) { lucid_prof::enabled() = on != 0; }

void lucid_profile_only(const char* name) { lucid_prof::only() = name ? name : ""; }

int lucid_profile_collect(void) { return lucid_prof::collect(); }

int lucid_profile_entry(int idx, char* name, int name_len, double* total_ms, long* count) {
  return lucid_prof::entry(idx, name, name_len, total_ms, count);
}

void lucid_profile_reset(void) { lucid_prof::reset(); }

// ---- the decoder's elementwise layers (modeling_lucid.py:58-75, 118-145) ----

int lucid_rmsnorm_fwd(const void* x, const void* w, void* y, float* rstd, int N, int H, float eps, void* stream) {
  g_last_error.clear();
  if (N < 0 || (H != 512 && H != 1024 && H != 2048 && H != 4096))
    return fail("lucid_rmsnorm_fwd: H must be 512, 1024, 2048 or 4096 and N >= 0, got H=" + std::to_string(H));
  if (N == 0) return LUCID_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid((N + 3) / 4);
#define LUCID_NORM_FWD(NC)                                                                                      \
  LUCID_LAUNCH("lucid_rmsnorm_fwd_kernel", lucid::lucid_rmsnorm_fwd_kernel<NC>, grid, st, (const bf16*)x,   \
               (const bf16*)w, (bf16*)y, rstd, N, eps)
  switch (H) {
    case 512: LUCID_NORM_FWD(1); break;
    case 1024: LUCID_NORM_FWD(2); break;
    case 2048: LUCID_NORM_FWD(4); break;
    default: LUCID_NORM_FWD(8); break;
  }
#undef LUCID_NORM_FWD
  return LUCID_OK;
}

size_t lucid_rmsnorm_bwd_workspace_bytes(int N, int H) {
  return (size_t)((N + lucid::kNormRowsPerBlock - 1) / lucid::kNormRowsPerBlock) * (size_t)H * sizeof(float);
}

int lucid_rmsnorm_bwd(const void* x, const void* w, const void* dy, const float* rstd, void* dx, void* dw,
                      void* workspace, int N, int H, void* stream) {
  g_last_error.clear();
  if (N < 0 || (H != 512 && H != 1024 && H != 2048 && H != 4096))
    return fail("lucid_rmsnorm_bwd: H must be 512, 1024, 2048 or 4096 and N >= 0, got H=" + std::to_string(H));
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int nb = (N + lucid::kNormRowsPerBlock - 1) / lucid::kNormRowsPerBlock;
  float* part = static_cast<float*>(workspace);
  if (nb > 0) {
#define LUCID_NORM_BWD(NC)                                                                                       \
  LUCID_LAUNCH("lucid_rmsnorm_bwd_kernel", lucid::lucid_rmsnorm_bwd_kernel<NC>, dim3(nb), st, (const bf16*)x,  \
               (const bf16*)w, (const bf16*)dy, rstd, (bf16*)dx, part, N)
    switch (H) {
      case 512: LUCID_NORM_BWD(1); break;
      case 1024: LUCID_NORM_BWD(2); break;
      case 2048: LUCID_NORM_BWD(4); break;
      default: LUCID_NORM_BWD(8); break;
    }
#undef LUCID_NORM_BWD
  }
  LUCID_LAUNCH_B("lucid_rmsnorm_dw_kernel", lucid::lucid_rmsnorm_dw_kernel, dim3(H / 256), dim3(64 * lucid::kDwWaves),
                 st, part, nb, H, (bf16*)dw);
  return LUCID_OK;
}

int lucid_rope(const void* x, const int64_t x_strides[3], int B, int Hn, int T, const void* cos, const void* sin,
               void* out, const int64_t out_strides[3], int D, int transpose, void* stream) {
  g_last_error.clear();
  if (D != 64 || B < 0 || T < 0 || Hn <= 0)
    return fail("lucid_rope: head dim 64, B >= 0, T >= 0 and Hn > 0, got D=" + std::to_string(D));
  if (!x_strides || !out_strides) return fail("lucid_rope: strides are null");
  for (int i = 0; i < 3; ++i)
    if (x_strides[i] % 8 || out_strides[i] % 8)
      return fail("lucid_rope: strides must be multiples of 8 elements and pointers 16-byte aligned");
  if (reinterpret_cast<uintptr_t>(x) % 16 || reinterpret_cast<uintptr_t>(cos) % 16 ||
      reinterpret_cast<uintptr_t>(sin) % 16 || reinterpret_cast<uintptr_t>(out) % 16)
    return fail("lucid_rope: strides must be multiples of 8 elements and pointers 16-byte aligned");
  const int64_t R = (int64_t)B * T * Hn;
  if (R == 0) return LUCID_OK;
  if (R > INT32_MAX / 4) return fail("lucid_rope: too many rows");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)((R * 4 + 255) / 256));
  if (transpose)
    LUCID_LAUNCH("lucid_rope_kernel", lucid::lucid_rope_kernel<-1>, grid, st, (const bf16*)x, x_strides[0],
                 x_strides[1], x_strides[2], (int)R, Hn, T, (const bf16*)cos, (const bf16*)sin, (bf16*)out,
                 out_strides[0], out_strides[1], out_strides[2]);
  else
    LUCID_LAUNCH("lucid_rope_kernel", lucid::lucid_rope_kernel<1>, grid, st, (const bf16*)x, x_strides[0],
                 x_strides[1], x_strides[2], (int)R, Hn, T, (const bf16*)cos, (const bf16*)sin, (bf16*)out,
                 out_strides[0], out_strides[1], out_strides[2]);
  return LUCID_OK;
}

static bool misaligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 != 0; }

int lucid_swiglu_fwd(const void* g, const void* u, void* h, int64_t n, void* stream) {
  g_last_error.clear();
  if (n < 0) return fail("lucid_swiglu_fwd: n must be >= 0");
  if (misaligned16(g) || misaligned16(u) || misaligned16(h))
    return fail("lucid_swiglu_fwd: pointers must be 16-byte aligned");
  if (n == 0) return LUCID_OK;
  const int64_t blocks = (n + 2047) / 2048;
  if (blocks > INT32_MAX) return fail("lucid_swiglu_fwd: too many elements");
  LUCID_LAUNCH("lucid_swiglu_fwd_kernel", lucid::lucid_swiglu_fwd_kernel, dim3((unsigned)blocks),
               static_cast<hipStream_t>(stream), (const bf16*)g, (const bf16*)u, (bf16*)h, n);
  return LUCID_OK;
}

int lucid_swiglu_bwd(const void* g, const void* u, const void* dh, void* dg, void* du, int64_t n, void* stream) {
  g_last_error.clear();
  if (n < 0) return fail("lucid_swiglu_bwd: n must be >= 0");
  if (misaligned16(g) || misaligned16(u) || misaligned16(dh) || misaligned16(dg) || misaligned16(du))
    return fail("lucid_swiglu_bwd: pointers must be 16-byte aligned");
  if (n == 0) return LUCID_OK;
  const int64_t blocks = (n + 2047) / 2048;
  if (blocks > INT32_MAX) return fail("lucid_swiglu_bwd: too many elements");
  LUCID_LAUNCH("lucid_swiglu_bwd_kernel", lucid::lucid_swiglu_bwd_kernel, dim3((unsigned)blocks),
               static_cast<hipStream_t>(stream), (const bf16*)g, (const bf16*)u, (const bf16*)dh, (bf16*)dg,
               (bf16*)du, n);
  return LUCID_OK;
}

static int check_ce(const char* what, const void* logits, int64_t ls, int R, int T, int V) {
  if (R < 0 || T < 1 || R % T || V < 1 || V % 8 || ls < V || ls % 8 || misaligned16(logits))
    return fail(std::string(what) + ": R a multiple of T >= 1, V and the row stride multiples of 8, logits "
                "16-byte aligned; got R=" + std::to_string(R) + " T=" + std::to_string(T) + " V=" +
                std::to_string(V));
  return LUCID_OK;
}

int lucid_causal_lm_loss_fwd(const void* logits, int64_t row_stride, const int64_t* labels, int R, int T, int V,
                             float* lse, float* loss, float* valid, void* stream) {
  g_last_error.clear();
  if (int rc = check_ce("lucid_causal_lm_loss_fwd", logits, row_stride, R, T, V)) return rc;
  if (R == 0) return LUCID_OK;
  LUCID_LAUNCH("lucid_ce_fwd_kernel", lucid::lucid_ce_fwd_kernel, dim3(R), static_cast<hipStream_t>(stream),
               (const bf16*)logits, row_stride, labels, T, V, lse, loss, valid);
  return LUCID_OK;
}

int lucid_causal_lm_loss_bwd(const void* logits, int64_t row_stride, const int64_t* labels, int R, int T, int V,
                             const float* lse, const float* valid, const float* scale, void* dlogits, void* stream) {
  g_last_error.clear();
  if (int rc = check_ce("lucid_causal_lm_loss_bwd", logits, row_stride, R, T, V)) return rc;
  if (misaligned16(dlogits)) return fail("lucid_causal_lm_loss_bwd: dlogits must be 16-byte aligned");
  if (R == 0) return LUCID_OK;
  LUCID_LAUNCH("lucid_ce_bwd_kernel", lucid::lucid_ce_bwd_kernel, dim3(R), static_cast<hipStream_t>(stream),
               (const bf16*)logits, row_stride, labels, T, V, lse, valid, scale, (bf16*)dlogits);
  return LUCID_OK;
}

int lucid_adamw_step(int n, void* const* params, const void* const* grads, void* const* exp_avgs,
                     void* const* exp_avg_sqs, const int64_t* numels, int dtype, float lr, float beta1, float beta2,
                     float eps, float weight_decay, int64_t step, void* stream) {
  g_last_error.clear();
  if (n < 0 || (dtype != LUCID_DTYPE_BF16 && dtype != LUCID_DTYPE_F32) || step < 1)
    return fail("lucid_adamw_step: n >= 0, dtype LUCID_DTYPE_BF16 or LUCID_DTYPE_F32 and step >= 1");
  if (!(lr >= 0.f) || !(beta1 >= 0.f && beta1 < 1.f) || !(beta2 >= 0.f && beta2 < 1.f) || !(eps >= 0.f) ||
      !(weight_decay >= 0.f))
    return fail("lucid_adamw_step: lr, eps and weight_decay >= 0, betas in [0, 1)");
  const size_t es = dtype == LUCID_DTYPE_F32 ? 4 : 2;
  for (int i = 0; i < n; ++i) {
    if (numels[i] < 0 || numels[i] > (int64_t)INT32_MAX * lucid::kAdamChunk / 2)
      return fail("lucid_adamw_step: tensor " + std::to_string(i) + " has a bad element count");
    for (const void* ptr : {(const void*)params[i], grads[i], (const void*)exp_avgs[i], (const void*)exp_avg_sqs[i]})
      if (reinterpret_cast<uintptr_t>(ptr) % (8 * es))
        return fail("lucid_adamw_step: tensor " + std::to_string(i) + " is not aligned to 8 elements");
  }
  lucid::AdamWScalars c;
  c.decay = 1.0f - lr * weight_decay;
  c.b1 = beta1;
  c.b2 = beta2;
  c.eps = eps;
  c.step_size = (float)((double)lr / (1.0 - std::pow((double)beta1, (double)step)));
  c.inv_bc2 = (float)(1.0 / std::sqrt(1.0 - std::pow((double)beta2, (double)step)));
  hipStream_t st = static_cast<hipStream_t>(stream);
  lucid::AdamWBatch batch;
  int i = 0;
  while (i < n) {
    batch.n = 0;
    int64_t chunks = 0;
    for (; i < n && batch.n < lucid::kAdamMaxTensors; ++i) {
      if (numels[i] == 0) continue;
      const int64_t nc = (numels[i] + lucid::kAdamChunk - 1) / lucid::kAdamChunk;
      if (batch.n > 0 && chunks + nc > INT32_MAX) break;
      const int k = batch.n++;
      batch.p[k] = params[i];
      batch.g[k] = grads[i];
      batch.m[k] = exp_avgs[i];
      batch.v[k] = exp_avg_sqs[i];
      batch.numel[k] = numels[i];
      batch.chunk0[k] = (int)chunks;
      chunks += nc;
    }
    if (batch.n == 0) continue;
    batch.chunk0[batch.n] = (int)chunks;
    if (dtype == LUCID_DTYPE_F32)
      LUCID_LAUNCH("lucid_adamw_kernel", lucid::lucid_adamw_kernel<float>, dim3((unsigned)chunks), st, batch, c);
    else
      LUCID_LAUNCH("lucid_adamw_kernel", lucid::lucid_adamw_kernel<bf16>, dim3((unsigned)chunks), st, batch, c);
  }
  return LUCID_OK;
}

}  // extern "C"
