// Fused elementwise layers of the Llama-LUCID decoder (the model around the attention core,
// modeling_lucid.py:58-75 and 118-145) on CDNA4 (gfx950).  As torch ops each of them is a
// chain of memory-bound passes (RMSNorm: fp32 copy, square, mean, rsqrt, two products and a
// cast, each reading and writing the whole activation); here each is one pass over its rows.
//
//   lucid_rmsnorm_fwd_kernel      y = w * bf16(x rstd), rstd = 1/sqrt(mean(x^2) + eps) (fp32
//                                 statistics, the weight applied in bf16 as in the reference)
//   lucid_rmsnorm_bwd_kernel      dx = rstd (g - xn mean(g xn)), g = bf16(dy w), xn = x rstd;
//                                 per-block partial sums of dy * bf16(xn) for dw
//   lucid_rmsnorm_dw_kernel       dw = the sum of the partials over the row blocks (fixed
//                                 order: deterministic)
//   lucid_rope_kernel             out = x cos + rotate_half(x) sin over [B, T, H, d] rows (and
//                                 its transpose for the backward), one rounding to bf16
#include "lucid_common.h"

namespace lucid {

constexpr int kNormRowsPerBlock = 64;  // rows per workgroup of the backward (one dw partial each)

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

// dw[j] = sum over the row blocks of part[b][j], in block order; grid H / 256.
__global__ __launch_bounds__(256) void lucid_rmsnorm_dw_kernel(const float* __restrict__ part, int nb, int H,
                                                               bf16* __restrict__ dw) {
  const int j = blockIdx.x * 256 + threadIdx.x;
  if (j >= H) return;
  float s = 0.f;
  for (int b = 0; b < nb; ++b) s += part[(int64_t)b * H + j];
  dw[j] = (bf16)s;
}

// Rotary embedding over rows of head dim D = 64 (the model's): x [R][D] with row stride
// xs (elements) and head index h = row % Hn, token t = row / Hn (the [B, T, H, D] layout of
// the projections, B folded into t); cos / sin [Tt][D] rows of the token.  SIGN = +1: the
// forward out = x cos + rotate_half(x) sin; SIGN = -1: its transpose (the backward),
// out = x cos + rotate_half^T(x sin).  One lane per pair (i, i + D/2).
template <int SIGN>
__global__ __launch_bounds__(256) void lucid_rope_kernel(const bf16* __restrict__ x, int64_t xs, int R, int Hn,
                                                         const bf16* __restrict__ cs, const bf16* __restrict__ sn,
                                                         bf16* __restrict__ out) {
  constexpr int D = 64, HD = D / 2;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;  // (row, pair)
  const int row = (int)(idx / HD), i = (int)(idx % HD);
  if (row >= R) return;
  const int t = row / Hn;
  const bf16* xr = x + (int64_t)row * xs;
  const float x1 = (float)xr[i], x2 = (float)xr[i + HD];
  const float c1 = (float)cs[(int64_t)t * D + i], c2 = (float)cs[(int64_t)t * D + i + HD];
  const float s1 = (float)sn[(int64_t)t * D + i], s2 = (float)sn[(int64_t)t * D + i + HD];
  float o1, o2;
  if constexpr (SIGN > 0) {  // rotate_half(x) = (-x2, x1)
    o1 = x1 * c1 - x2 * s1;
    o2 = x2 * c2 + x1 * s2;
  } else {  // rotate_half^T(y) = (y2, -y1) with y = x sin
    o1 = x1 * c1 + x2 * s2;
    o2 = x2 * c2 - x1 * s1;
  }
  bf16* orow = out + (int64_t)row * D;
  orow[i] = (bf16)o1;
  orow[i + HD] = (bf16)o2;
}

}  // namespace lucid
