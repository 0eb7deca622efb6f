// Fused elementwise layers of the Llama-LUCID decoder (the model around the attention core,
// modeling_lucid.py:58-75, 118-145, 155-167 and the loss of 847-967) and the AdamW step of its
// training (run_clm_chunk.py:776, the Trainer's default optimizer) on CDNA4 (gfx950).  As
// torch ops each of them is a chain of memory-bound passes (RMSNorm: fp32 copy, square, mean,
// rsqrt, two products and a cast, each reading and writing the whole activation); here each
// is one pass over its data.
//
//   lucid_rmsnorm_fwd_kernel      y = w * bf16(x rstd), rstd = 1/sqrt(mean(x^2) + eps) (fp32
//                                 statistics, the weight applied in bf16 as in the reference)
//   lucid_rmsnorm_bwd_kernel      dx = rstd (g - xn mean(g xn)), g = bf16(dy w), xn = x rstd;
//                                 per-block partial sums of dy * bf16(xn) for dw
//   lucid_rmsnorm_dw_kernel       dw = the sum of the partials over the row blocks (fixed
//                                 order: deterministic)
//   lucid_rope_kernel             out = x cos + rotate_half(x) sin over [B, T, H, d] rows (and
//                                 its transpose for the backward), one rounding to bf16
//   lucid_swiglu_fwd/bwd_kernel   h = silu(g) u (modeling_lucid.py:155-167 between the gate / up
//                                 and down projections) and its gradients, fp32 inside
//   lucid_adamw_kernel            one AdamW update over up to kAdamMaxTensors parameter
//                                 tensors per launch (p, grad, exp_avg, exp_avg_sq; fp32 math)
//   lucid_ce_fwd/bwd_kernel       the shifted causal-LM cross entropy on bf16 logits
//                                 (modeling_lucid.py:847-967: labels shifted by one, -100
//                                 ignored): per-row logsumexp and loss in one read of the row;
//                                 backward (softmax - onehot) scale written as bf16
#include <type_traits>

#include "lucid_common.h"

namespace lucid {

typedef float f32x8_t __attribute__((ext_vector_type(8)));

constexpr int kNormRowsPerBlock = 16;  // rows per workgroup of the backward (one dw partial each)
constexpr int kDwWaves = 16;           // waves of the dw reduction workgroup (256 columns each)

// One wave per row; H = 64 * 8 * NC (a lane holds NC chunks of 8 consecutive values).
template <int NC>
__global__ __launch_bounds__(256) void lucid_rmsnorm_fwd_kernel(const bf16* __restrict__ x, const bf16* __restrict__ w,
                                                                bf16* __restrict__ y, float* __restrict__ rstd, int N,
                                                                float eps) {
  constexpr int H = 64 * 8 * NC;
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= N) return;
  const bf16* xr = x + (int64_t)row * H;
  bf16x8 xv[NC];
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    xv[c] = ld8(xr + (c * 64 + lane) * 8);
#pragma unroll
    for (int e = 0; e < 8; ++e) ss = fmaf((float)xv[c][e], (float)xv[c][e], ss);
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o, 64);
  const float r = 1.0f / sqrtf(ss / (float)H + eps);
  bf16* yr = y + (int64_t)row * H;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const bf16x8 wv = ld8(w + (c * 64 + lane) * 8);
    bf16x8 o;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = (bf16)((float)wv[e] * (float)(bf16)((float)xv[c][e] * r));
    *reinterpret_cast<bf16x8*>(yr + (c * 64 + lane) * 8) = o;
  }
  if (lane == 0) rstd[row] = r;
}

// One wave per row, kNormRowsPerBlock rows per workgroup; the workgroup's dw partial
// (sum over its rows of dy * bf16(xn)) goes to part[blockIdx.x][H] in fp32.
template <int NC>
__global__ __launch_bounds__(256) void lucid_rmsnorm_bwd_kernel(const bf16* __restrict__ x, const bf16* __restrict__ w,
                                                                const bf16* __restrict__ dy,
                                                                const float* __restrict__ rstd, bf16* __restrict__ dx,
                                                                float* __restrict__ part, int N) {
  constexpr int H = 64 * 8 * NC;
  __shared__ float red[4][H];
  const int lane = threadIdx.x & 63, wv_ = threadIdx.x >> 6;
  float pw[NC][8];
#pragma unroll
  for (int c = 0; c < NC; ++c)
#pragma unroll
    for (int e = 0; e < 8; ++e) pw[c][e] = 0.f;
  bf16x8 wv[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) wv[c] = ld8(w + (c * 64 + lane) * 8);
  for (int i = wv_; i < kNormRowsPerBlock; i += 4) {
    const int row = blockIdx.x * kNormRowsPerBlock + i;
    if (row >= N) break;
    const float r = rstd[row];
    float xn[NC][8], g[NC][8];
    float dot = 0.f;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const bf16x8 xv = ld8(x + (int64_t)row * H + (c * 64 + lane) * 8);
      const bf16x8 dv = ld8(dy + (int64_t)row * H + (c * 64 + lane) * 8);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        xn[c][e] = (float)xv[e] * r;
        g[c][e] = (float)(bf16)((float)dv[e] * (float)wv[c][e]);
        dot = fmaf(g[c][e], xn[c][e], dot);
        pw[c][e] = fmaf((float)dv[e], (float)(bf16)xn[c][e], pw[c][e]);
      }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) dot += __shfl_xor(dot, o, 64);
    const float mdot = dot / (float)H;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      bf16x8 o;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = (bf16)(r * (g[c][e] - xn[c][e] * mdot));
      *reinterpret_cast<bf16x8*>(dx + (int64_t)row * H + (c * 64 + lane) * 8) = o;
    }
  }
#pragma unroll
  for (int c = 0; c < NC; ++c)
#pragma unroll
    for (int e = 0; e < 8; ++e) red[wv_][(c * 64 + lane) * 8 + e] = pw[c][e];
  __syncthreads();
  for (int j = threadIdx.x; j < H; j += 256)
    part[(int64_t)blockIdx.x * H + j] = (red[0][j] + red[1][j]) + (red[2][j] + red[3][j]);
}

// dw[j] = sum over the row blocks of part[b][j]: a workgroup of kDwWaves waves per 256 columns
// (4 per lane, one 16-byte load); wave w sums the blocks b = w, w + kDwWaves, ... in order, and
// the waves' sums are added in a fixed tree order (deterministic).  Grid H / 256.
__global__ __launch_bounds__(64 * kDwWaves) void lucid_rmsnorm_dw_kernel(const float* __restrict__ part, int nb,
                                                                         int H, bf16* __restrict__ dw) {
  __shared__ float4 red[kDwWaves][64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int j = blockIdx.x * 256 + lane * 4;
  float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll 8
  for (int b = w; b < nb; b += kDwWaves) {
    const float4 p = *reinterpret_cast<const float4*>(part + (int64_t)b * H + j);
    s.x += p.x;
    s.y += p.y;
    s.z += p.z;
    s.w += p.w;
  }
  red[w][lane] = s;
  __syncthreads();
#pragma unroll
  for (int h = kDwWaves / 2; h >= 1; h >>= 1) {
    if (w < h) {
      const float4 o = red[w + h][lane];
      s.x += o.x;
      s.y += o.y;
      s.z += o.z;
      s.w += o.w;
      red[w][lane] = s;
    }
    __syncthreads();
  }
  if (w == 0) {
    bf16 o[4] = {(bf16)s.x, (bf16)s.y, (bf16)s.z, (bf16)s.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) dw[j + e] = o[e];
  }
}

// Rotary embedding over rows of head dim D = 64 (the model's).  Row (b, t, h) reads
// x + b sb + h sh + t st and writes out + b ob + h oh + t ot (element strides, multiples of 8),
// with the cos / sin row of token b T + t ([B T][64]).  SIGN = +1: the forward
// out = x cos + rotate_half(x) sin, rotate_half(x) = (-x2, x1); SIGN = -1: its transpose (the
// backward), out = x cos + rotate_half^T(x sin), rotate_half^T(y) = (y2, -y1).  Four lanes per
// row, each holding 8 pairs (i, i + 32) in 16-byte loads.
template <int SIGN>
__global__ __launch_bounds__(256) void lucid_rope_kernel(const bf16* __restrict__ x, int64_t sb, int64_t sh,
                                                         int64_t st, int R, int Hn, int T,
                                                         const bf16* __restrict__ cs, const bf16* __restrict__ sn,
                                                         bf16* __restrict__ out, int64_t ob, int64_t oh, int64_t ot) {
  constexpr int D = 64, HD = D / 2;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int row = (int)(idx >> 2), i0 = (int)(idx & 3) * 8;
  if (row >= R) return;
  const int h = row % Hn, bt = row / Hn;
  const int t = bt % T, b = bt / T;
  const bf16* xr = x + b * sb + h * sh + t * st;
  const bf16x8 x1 = ld8(xr + i0), x2 = ld8(xr + HD + i0);
  const bf16x8 c1 = ld8(cs + (int64_t)bt * D + i0), c2 = ld8(cs + (int64_t)bt * D + HD + i0);
  const bf16x8 s1 = ld8(sn + (int64_t)bt * D + i0), s2 = ld8(sn + (int64_t)bt * D + HD + i0);
  bf16x8 o1, o2;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float a = (float)x1[e], c = (float)x2[e];
    if constexpr (SIGN > 0) {
      o1[e] = (bf16)(a * (float)c1[e] - c * (float)s1[e]);
      o2[e] = (bf16)(c * (float)c2[e] + a * (float)s2[e]);
    } else {
      o1[e] = (bf16)(a * (float)c1[e] + c * (float)s2[e]);
      o2[e] = (bf16)(c * (float)c2[e] - a * (float)s1[e]);
    }
  }
  bf16* orow = out + b * ob + h * oh + t * ot;
  *reinterpret_cast<bf16x8*>(orow + i0) = o1;
  *reinterpret_cast<bf16x8*>(orow + HD + i0) = o2;
}

__device__ __forceinline__ float sigmoidf_(float x) { return 1.0f / (1.0f + __expf(-x)); }

// h = silu(g) u elementwise over n values; 8 per lane (16-byte accesses) and a scalar tail.
__global__ __launch_bounds__(256) void lucid_swiglu_fwd_kernel(const bf16* __restrict__ g, const bf16* __restrict__ u,
                                                               bf16* __restrict__ h, int64_t n) {
  const int64_t c = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 8;
  if (c + 8 <= n) {
    const bf16x8 gv = ld8(g + c), uv = ld8(u + c);
    bf16x8 o;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float x = (float)gv[e];
      o[e] = (bf16)(x * sigmoidf_(x) * (float)uv[e]);
    }
    *reinterpret_cast<bf16x8*>(h + c) = o;
  } else {
    for (int64_t i = c; i < n; ++i) {
      const float x = (float)g[i];
      h[i] = (bf16)(x * sigmoidf_(x) * (float)u[i]);
    }
  }
}

// dg = dh u silu'(g), du = dh silu(g); silu'(x) = sig(x) (1 + x (1 - sig(x))).
__global__ __launch_bounds__(256) void lucid_swiglu_bwd_kernel(const bf16* __restrict__ g, const bf16* __restrict__ u,
                                                               const bf16* __restrict__ dh, bf16* __restrict__ dg,
                                                               bf16* __restrict__ du, int64_t n) {
  const int64_t c = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 8;
  auto one = [](float x, float uu, float d, float& og, float& ou) {
    const float sg = sigmoidf_(x);
    og = d * uu * sg * (1.0f + x * (1.0f - sg));
    ou = d * x * sg;
  };
  if (c + 8 <= n) {
    const bf16x8 gv = ld8(g + c), uv = ld8(u + c), dv = ld8(dh + c);
    bf16x8 og, ou;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float a, b;
      one((float)gv[e], (float)uv[e], (float)dv[e], a, b);
      og[e] = (bf16)a;
      ou[e] = (bf16)b;
    }
    *reinterpret_cast<bf16x8*>(dg + c) = og;
    *reinterpret_cast<bf16x8*>(du + c) = ou;
  } else {
    for (int64_t i = c; i < n; ++i) {
      float a, b;
      one((float)g[i], (float)u[i], (float)dh[i], a, b);
      dg[i] = (bf16)a;
      du[i] = (bf16)b;
    }
  }
}

constexpr int kIgnoreIndex = -100;  // F.cross_entropy's default ignore_index

// Workgroup-wide (max, sum of exp) merge of the 256 lanes' running pairs; every lane returns
// the row's logsumexp.
__device__ __forceinline__ float block_lse(float m, float s) {
  __shared__ float sm[4], ss[4];
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const float m2 = __shfl_xor(m, o, 64), s2 = __shfl_xor(s, o, 64);
    const float mm = fmaxf(m, m2);
    s = s * __expf(m - mm) + s2 * __expf(m2 - mm);
    m = mm;
  }
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    sm[w] = m;
    ss[w] = s;
  }
  __syncthreads();
  float mm = fmaxf(fmaxf(sm[0], sm[1]), fmaxf(sm[2], sm[3]));
  float st = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) st += ss[i] * __expf(sm[i] - mm);
  return mm + __logf(st);
}

// Row r of logits [R][V] (row stride ls, V and ls multiples of 8) is position t = r % T of its
// sequence; its target is labels[r + 1] for t < T - 1 (the shift of the causal-LM loss), and the
// last position of each sequence has none.  Writes lse[r], loss[r] = lse - logit[target] and
// valid[r] (1 when the row counts, else 0 with loss 0); a target outside [0, V) other than the
// ignore index gives a NaN loss.
__global__ __launch_bounds__(256) void lucid_ce_fwd_kernel(const bf16* __restrict__ logits, int64_t ls,
                                                           const int64_t* __restrict__ labels, int T, int V,
                                                           float* __restrict__ lse, float* __restrict__ loss,
                                                           float* __restrict__ valid) {
  const int r = blockIdx.x;
  const bf16* row = logits + (int64_t)r * ls;
  float m = -3.0e38f, s = 0.f;
  for (int j = threadIdx.x * 8; j < V; j += 256 * 8) {
    const bf16x8 xv = ld8(row + j);
    float cm = (float)xv[0];
#pragma unroll
    for (int e = 1; e < 8; ++e) cm = fmaxf(cm, (float)xv[e]);
    if (cm > m) {
      s *= __expf(m - cm);
      m = cm;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) s += __expf((float)xv[e] - m);
  }
  const float l = block_lse(m, s);
  if (threadIdx.x == 0) {
    lse[r] = l;
    const bool has = (r % T) != T - 1;
    const int64_t tgt = has ? labels[r + 1] : kIgnoreIndex;
    if (tgt == kIgnoreIndex) {
      loss[r] = 0.f;
      valid[r] = 0.f;
    } else if (tgt < 0 || tgt >= V) {
      loss[r] = __int_as_float(0x7fc00000);
      valid[r] = 1.f;
    } else {
      loss[r] = l - (float)row[tgt];
      valid[r] = 1.f;
    }
  }
}

// dlogits[r][j] = (exp(logit - lse[r]) - [j == target]) * scale[0] for counted rows, 0 for the
// others (dlogits [R][V] contiguous).
__global__ __launch_bounds__(256) void lucid_ce_bwd_kernel(const bf16* __restrict__ logits, int64_t ls,
                                                           const int64_t* __restrict__ labels, int T, int V,
                                                           const float* __restrict__ lse,
                                                           const float* __restrict__ valid,
                                                           const float* __restrict__ scale,
                                                           bf16* __restrict__ dlogits) {
  const int r = blockIdx.x;
  const bf16* row = logits + (int64_t)r * ls;
  bf16* drow = dlogits + (int64_t)r * V;
  const bool on = valid[r] != 0.f;
  const float sc = on ? scale[0] : 0.f, l = lse[r];
  const int64_t tgt = on ? labels[r + 1] : -1;
  for (int j = threadIdx.x * 8; j < V; j += 256 * 8) {
    bf16x8 o;
    if (on) {
      const bf16x8 xv = ld8(row + j);
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = (bf16)((__expf((float)xv[e] - l) - (j + e == tgt ? 1.f : 0.f)) * sc);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = (bf16)0.f;
    }
    *reinterpret_cast<bf16x8*>(drow + j) = o;
  }
}

// AdamW (decoupled weight decay, Loshchilov & Hutter), the update of torch.optim.AdamW:
//   p <- p (1 - lr wd);  m <- m + (1 - b1) (g - m);  v <- b2 v + (1 - b2) g^2
//   p <- p - step_size m / (sqrt(v) / sqrt(1 - b2^t) + eps),  step_size = lr / (1 - b1^t)
// in fp32 with one rounding per stored value.  A launch covers up to kAdamMaxTensors tensors
// (pointers in the kernel argument), cut into chunks of kAdamChunk elements: workgroup c
// finds its tensor in the chunk prefix sums.  8 elements per lane (16- or 32-byte accesses
// when the tensor's base is aligned, which the host checks), a scalar tail.
constexpr int kAdamMaxTensors = 48;
constexpr int kAdamChunk = 256 * 8;

struct AdamWBatch {
  void* p[kAdamMaxTensors];
  const void* g[kAdamMaxTensors];
  void* m[kAdamMaxTensors];
  void* v[kAdamMaxTensors];
  int64_t numel[kAdamMaxTensors];
  int chunk0[kAdamMaxTensors + 1];  // first chunk of each tensor; chunk0[n] = the grid size
  int n;
};

struct AdamWScalars {
  float decay;       // 1 - lr wd
  float b1, b2, eps;
  float step_size;   // lr / (1 - b1^t)
  float inv_bc2;     // 1 / sqrt(1 - b2^t)
};

template <typename T>
__device__ __forceinline__ void adamw_one(T& p, float g, T& m, T& v, const AdamWScalars& c) {
  float pf = (float)p * c.decay;
  const float mf = (float)m + (1.0f - c.b1) * (g - (float)m);
  const float vf = c.b2 * (float)v + (1.0f - c.b2) * g * g;
  pf -= c.step_size * mf / (sqrtf(vf) * c.inv_bc2 + c.eps);
  p = (T)pf;
  m = (T)mf;
  v = (T)vf;
}

template <typename T>
__global__ __launch_bounds__(256) void lucid_adamw_kernel(const AdamWBatch batch, const AdamWScalars c) {
  const int chunk = blockIdx.x;
  int lo = 0, hi = batch.n - 1;  // the tensor i with chunk0[i] <= chunk < chunk0[i + 1]
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (batch.chunk0[mid] <= chunk) lo = mid;
    else hi = mid - 1;
  }
  const int i = lo;
  T* p = static_cast<T*>(batch.p[i]);
  const T* g = static_cast<const T*>(batch.g[i]);
  T* m = static_cast<T*>(batch.m[i]);
  T* v = static_cast<T*>(batch.v[i]);
  const int64_t n = batch.numel[i];
  const int64_t e0 = (int64_t)(chunk - batch.chunk0[i]) * kAdamChunk + threadIdx.x * 8;
  if (e0 + 8 <= n) {
    using V8 = std::conditional_t<std::is_same_v<T, float>, f32x8_t, bf16x8>;
    V8 pv = *reinterpret_cast<const V8*>(p + e0), mv = *reinterpret_cast<const V8*>(m + e0);
    V8 vv = *reinterpret_cast<const V8*>(v + e0);
    const V8 gv = *reinterpret_cast<const V8*>(g + e0);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      T pe = pv[e], me = mv[e], ve = vv[e];
      adamw_one<T>(pe, (float)gv[e], me, ve, c);
      pv[e] = pe;
      mv[e] = me;
      vv[e] = ve;
    }
    *reinterpret_cast<V8*>(p + e0) = pv;
    *reinterpret_cast<V8*>(m + e0) = mv;
    *reinterpret_cast<V8*>(v + e0) = vv;
  } else {
    for (int64_t e = e0; e < n; ++e) adamw_one<T>(p[e], (float)g[e], m[e], v[e], c);
  }
}

}  // namespace lucid
