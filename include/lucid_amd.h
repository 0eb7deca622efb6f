/*
 * lucid_amd -- C ABI of the MI355X (gfx950) LUCID attention kernels.
 *
 * Plain pointers and sizes only; every buffer is caller-owned device memory (the
 * library allocates no device memory; its only allocation is the 4-byte pinned flag of the
 * bounded chain waits, made with a per-device set-up -- hipHostMalloc once per process,
 * hipMemcpyToSymbol once per device -- by the first chain call on a device and again after
 * lucid_set_chain_wait_limit; code that captures HIP graphs calls lucid_chain_status() once per
 * device before capture, which does that set-up).  Tensors are bf16 (fp32 for the _f32 entry
 * points) with the last (head_dim) axis contiguous; the other axes are described by element strides
 * {batch, head, time}.  All launches go on `stream` (a hipStream_t, NULL =
 * default stream); calls are asynchronous.  Return value: 0 on success,
 * LUCID_EINVAL for a rejected argument (text in lucid_last_error()), or
 * LUCID_EHIP + hipError_t for a HIP launch failure.
 *
 * Supported: head_dim D in [1, 128] (bf16 and fp32 entry points); T a multiple of
 * 128 (the Python layer zero-pads the sequence end, which leaves every real row
 * unchanged because both P and the attention mask are causal); Hq a multiple of
 * Hkv (GQA).  Head dims other than 64 and 128 (the reference model's is 68,
 * lucid/config/config.json:9) run on zero-padded rows: every [.., D] operand then
 * has Dp = 64 (D <= 64) or 128 (D > 64) elements per row, columns D .. Dp-1 zero in
 * the inputs (dout included) and written zero in the outputs; the dot products are
 * unchanged and the RMS of k_norm divides by D itself (the attention sweeps of D in
 * 65 .. 96 leave out the columns beyond 80 or 96, whose products are zero).  Workspace
 * sizes take D and are those of Dp.
 */
#ifndef LUCID_AMD_H
#define LUCID_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* The libraries are built with hidden symbol visibility; only these entry points are exported. */
#pragma GCC visibility push(default)

#define LUCID_OK 0
#define LUCID_EINVAL 1

/* element types of lucid_adamw_step */
#define LUCID_DTYPE_BF16 0
#define LUCID_DTYPE_F32 1
#define LUCID_ECHAIN 2 /* a chain wait gave up in an earlier launch (lucid_chain_status) */
#define LUCID_EHIP 1000

/* Precision of the preconditioner chains (lucid_set_precision). */
#define LUCID_PRECISION_AUTO 0  /* per head, from the head's row mass (default) */
#define LUCID_PRECISION_FAST 1  /* bf16 products everywhere */
#define LUCID_PRECISION_EXACT 2 /* hi/lo split products for every head */

/* ABI version of this header (bumped on any signature change or new entry point): 6. */
int lucid_abi_version(void);

/* Text of the last error on the calling thread ("" if none). */
const char* lucid_last_error(void);

/* Chain precision for the forward calls that follow on the calling thread (thread-local:
 * another thread's calls keep their own mode; the backward uses the choice recorded in the
 * forward workspace, so it may run on any thread).  The off-diagonal products of the chained
 * solves (P V', P^T dV, (dV V'^T) * P and its sums with K) accumulate over every earlier
 * key of a row; with bf16 operands their error grows like 2^-8 |V'| sqrt(m), m = the
 * row mass sum_{j<i} P_ij^2, which is ~1e-2 for keys with no common direction but ~T for
 * keys along a shared direction (the reference's fp32 TRSM carries those at fp32
 * accuracy).  AUTO measures m per head (sampled) and runs heads with m > 4 through
 * kernels that split every such product into bf16 hi*hi + hi*lo + lo*hi terms (~fp32
 * accuracy); FAST and EXACT force one kind for every head (testing, benchmarking).
 * Returns LUCID_EINVAL for an unknown mode.  No counterpart in the reference, whose
 * torch solve_triangular works in the input dtype (modeling_lucid.py:570). */
int lucid_set_precision(int mode);
int lucid_get_precision(void);

/* Forward kernel schedule for the calls that follow on the calling thread (thread-local;
 * no counterpart in the reference).  On (default): at head dim <= 64 with one query head per kv head, the
 * preconditioner chain and the causal attention of each 128-row block run in one fused
 * kernel (lucid_fused_fwd_kernel) that feeds every staged key tile to both; off: the chain
 * kernel, then the attention kernel.  Both give the same O, V' and lse up to the rounding
 * order of the attention's online softmax.  Any nonzero value means on. */
int lucid_set_fused_forward(int on);
int lucid_get_fused_forward(void);

/* Bounded chain waits (no counterpart in the reference, which has no cross-workgroup
 * waits).  The chained solves hand blocks between workgroups through per-head progress
 * counters; a wait that sees no progress for the wait limit (default 2 s, against waits of
 * microseconds) gives up so that the kernel still finishes, and records it in a word of
 * pinned host memory (4 bytes, allocated once on the first chain call).  Every entry point
 * that launches a chain kernel first reports such an earlier give-up as LUCID_ECHAIN (the
 * results of the launch that gave up are invalid).  lucid_chain_status() makes the same
 * check on its own (synchronize the stream first to cover the launches in flight).
 * lucid_set_chain_wait_limit(seconds) changes the limit for the calls that follow
 * (testing aid: a tiny limit forces the give-up path with every kernel still exiting). */
int lucid_chain_status(void);
int lucid_set_chain_wait_limit(double seconds);

/* Byte offset, inside the forward workspace, of the per-head row masses (float [B*Hkv]);
 * a head ran the exact chain kernels when its mass exceeds 4 (testing aid). */
size_t lucid_fwd_workspace_mass_offset(int B, int Hq, int Hkv, int T, int D);

/* Bytes of the forward workspace.  It holds the state the backward reuses
 * (1/rms of K, K^T and V' in MFMA operand layouts, the inverted 64x64
 * diagonal blocks of P, the in-block coupling of each 128-row chain block,
 * chain counters), so keep it alive until
 * lucid_attn_bwd has been enqueued.  Workspaces must be 256-byte aligned
 * (hipMalloc and the torch allocator return such pointers). */
size_t lucid_fwd_workspace_bytes(int B, int Hq, int Hkv, int T, int D);

/* Preconditioned values only: vprime = P^-1 V, fp32 [B, Hkv, T, D] contiguous.
 * Replaces LucidAttention.get_v_prime (modeling_lucid.py:551-574), both its
 * dense branch (:561-570) and Lucid_Tril_Solver.forward (:284-312). */
int lucid_get_v_prime(const void* k, const int64_t* k_strides, const void* v, const int64_t* v_strides,
                      float* vprime, void* fwd_ws, int B, int Hkv, int T, int D, float scale, float eps,
                      void* stream);

/* Full forward O = softmax(s Q K^T, causal) P^-1 V.
 * q [B,Hq,T,D], k/v [B,Hkv,T,D] (strided), o [B,T,Hq,D] or any strided layout,
 * vprime fp32 [B,Hkv,T,D] contiguous (output), lse fp32 [B,Hq,T] (output,
 * log2-domain row normaliser, needed by the backward).
 * Replaces get_v_prime + eager_lucid_attention_forward
 * (modeling_lucid.py:461-496 -> :551-574 and :505-549). */
int lucid_attn_fwd(const void* q, const int64_t* q_strides, const void* k, const int64_t* k_strides,
                   const void* v, const int64_t* v_strides, void* o, const int64_t* o_strides, float* vprime,
                   float* lse, void* fwd_ws, int B, int Hq, int Hkv, int T, int D, float scale, float eps,
                   void* stream);

/* Bytes of the backward scratch workspace. */
size_t lucid_bwd_workspace_bytes(int B, int Hq, int Hkv, int T, int D);

/* Gradients of sum(O * dO) w.r.t. q, k, v (bf16, strided outputs).
 * Replaces the autograd of the dense path and Lucid_Tril_Solver.backward
 * (modeling_lucid.py:314-382) together with the SDPA backward. */
int lucid_attn_bwd(const void* dout, const int64_t* do_strides, const void* q, const int64_t* q_strides,
                   const void* k, const int64_t* k_strides, const void* o, const int64_t* o_strides,
                   const float* lse, const void* fwd_ws, void* dq, const int64_t* dq_strides, void* dk,
                   const int64_t* dk_strides, void* dv, const int64_t* dv_strides, void* bwd_ws, int B, int Hq,
                   int Hkv, int T, int D, float scale, float eps, void* stream);

/* ---- fp32 inputs (head dims up to 128) ----
 * The reference computes in the dtype of its inputs (modeling_lucid.py:461-496, :284-382 run
 * on whatever q/k/v hold); these are lucid_attn_fwd / lucid_attn_bwd for fp32 tensors, with
 * fp32 outputs (o, dq, dk, dv) and the same layouts and strides.  Q, K and dO are carried as
 * bf16 pairs (hi + lo) through split MFMA products and every head runs the exact chain
 * instances, so the results are within ~1e-4 relative of an fp64 evaluation.  The forward
 * workspace (lucid_fwd_f32_workspace_bytes) holds the split copies of Q and K and must stay
 * alive until lucid_attn_bwd_f32; the backward reads o as written by the forward. */
size_t lucid_fwd_f32_workspace_bytes(int B, int Hq, int Hkv, int T, int D);
size_t lucid_bwd_f32_workspace_bytes(int B, int Hq, int Hkv, int T, int D);
int lucid_attn_fwd_f32(const float* q, const int64_t* q_strides, const float* k, const int64_t* k_strides,
                       const float* v, const int64_t* v_strides, float* o, const int64_t* o_strides, float* vprime,
                       float* lse, void* fwd_ws, int B, int Hq, int Hkv, int T, int D, float scale, float eps,
                       void* stream);
int lucid_attn_bwd_f32(const float* dout, const int64_t* do_strides, const float* o, const int64_t* o_strides,
                       const float* lse, const void* fwd_ws, float* dq, const int64_t* dq_strides, float* dk,
                       const int64_t* dk_strides, float* dv, const int64_t* dv_strides, void* bwd_ws, int B, int Hq,
                       int Hkv, int T, int D, float scale, void* stream);

/* The two seams below (get_v_prime and eager_lucid_attention_forward) on fp32 tensors, head
 * dims up to 128: the same contracts as lucid_get_v_prime / lucid_precond_bwd and lucid_attn_vp_fwd /
 * lucid_attn_vp_bwd, with fp32 inputs (v_prime included) and fp32 outputs.  Workspaces:
 * lucid_v_prime_f32_workspace_bytes for lucid_get_v_prime_f32 (kept until
 * lucid_precond_bwd_f32, whose own workspace is lucid_precond_bwd_workspace_bytes), and the
 * two _f32 sizes of the attention seam. */
size_t lucid_v_prime_f32_workspace_bytes(int B, int Hkv, int T, int D);
int lucid_get_v_prime_f32(const float* k, const int64_t* k_strides, const float* v, const int64_t* v_strides,
                          float* vprime, void* fwd_ws, int B, int Hkv, int T, int D, float scale, float eps,
                          void* stream);
int lucid_precond_bwd_f32(const float* dvprime, const int64_t* dvprime_strides, const void* fwd_ws, float* dk,
                          const int64_t* dk_strides, float* dv, const int64_t* dv_strides, void* bwd_ws, int B,
                          int Hkv, int T, int D, float scale, void* stream);
size_t lucid_attn_vp_fwd_f32_workspace_bytes(int B, int Hq, int Hkv, int T, int D);
int lucid_attn_vp_fwd_f32(const float* q, const int64_t* q_strides, const float* k, const int64_t* k_strides,
                          const float* vprime, const int64_t* vprime_strides, float* o, const int64_t* o_strides,
                          float* lse, void* ws, int B, int Hq, int Hkv, int T, int D, float scale, float eps,
                          void* stream);
size_t lucid_attn_vp_bwd_f32_workspace_bytes(int B, int Hq, int Hkv, int T, int D);
int lucid_attn_vp_bwd_f32(const float* dout, const int64_t* do_strides, const float* o, const int64_t* o_strides,
                          const float* lse, const void* fwd_ws, float* dq, const int64_t* dq_strides, float* dk,
                          const int64_t* dk_strides, float* dvprime, const int64_t* dvprime_strides, void* bwd_ws,
                          int B, int Hq, int Hkv, int T, int D, float scale, void* stream);

/* ---- The two operator seams of LucidAttention.forward, separately ----
 * get_v_prime (modeling_lucid.py:551-574) is lucid_get_v_prime above; its gradient is
 * lucid_precond_bwd.  eager_lucid_attention_forward (:505-549: causal SDPA of q and the
 * repeat_kv'd key and v_prime, output [B,T,Hq,D]) is lucid_attn_vp_fwd and its gradient
 * lucid_attn_vp_bwd.  Composed as LucidAttention.forward composes them (:461-496) they give
 * the same result as lucid_attn_fwd / lucid_attn_bwd.  With v_prime = value they are plain
 * causal softmax attention. */

/* Bytes of the workspace of lucid_attn_vp_fwd, kept alive until lucid_attn_vp_bwd. */
size_t lucid_attn_vp_fwd_workspace_bytes(int B, int Hq, int Hkv, int T, int D);

/* O = softmax(s Q K^T, causal) V' for a caller's V' (bf16, or fp32 when vprime_f32 != 0;
 * [B,Hkv,T,D] strided), o [B,T,Hq,D] (strided), lse fp32 [B,Hq,T] (output).  eps is the
 * k_norm epsilon, used to measure each head's row mass (lucid_set_precision). */
int lucid_attn_vp_fwd(const void* q, const int64_t* q_strides, const void* k, const int64_t* k_strides,
                      const void* vprime, const int64_t* vprime_strides, int vprime_f32, void* o,
                      const int64_t* o_strides, float* lse, void* ws, int B, int Hq, int Hkv, int T, int D,
                      float scale, float eps, void* stream);

/* Bytes of the backward scratch of lucid_attn_vp_bwd. */
size_t lucid_attn_vp_bwd_workspace_bytes(int B, int Hq, int Hkv, int T, int D);

/* Gradients of sum(O * dO) w.r.t. q, k (the softmax part only; bf16) and v_prime (bf16 or
 * fp32 when dvprime_f32 != 0), GQA groups summed.  fwd_ws is lucid_attn_vp_fwd's. */
int lucid_attn_vp_bwd(const void* dout, const int64_t* do_strides, const void* q, const int64_t* q_strides,
                      const void* k, const int64_t* k_strides, const void* o, const int64_t* o_strides,
                      const float* lse, const void* fwd_ws, void* dq, const int64_t* dq_strides, void* dk,
                      const int64_t* dk_strides, void* dvprime, const int64_t* dvprime_strides, int dvprime_f32,
                      void* bwd_ws, int B, int Hq, int Hkv, int T, int D, float scale, void* stream);

/* Bytes of the backward scratch of lucid_precond_bwd. */
size_t lucid_precond_bwd_workspace_bytes(int B, int Hkv, int T, int D);

/* Gradient of V' = P(K^)^-1 V alone: given dV' (bf16, or fp32 when dvprime_f32 != 0;
 * strided), dv = P^-T dV' and dk = RMSNorm backward of dK^ = -s (M K^ + M^T K^),
 * M = tril((dV V'^T) * P) (bf16 outputs).  fwd_ws is the workspace of the lucid_get_v_prime
 * call that produced V' (kept alive until this call is enqueued).  Replaces
 * Lucid_Tril_Solver.backward (modeling_lucid.py:314-382) and the autograd of the dense
 * branch of get_v_prime (:561-570), k_norm (:409) included. */
int lucid_precond_bwd(const void* k, const int64_t* k_strides, const void* dvprime, const int64_t* dvprime_strides,
                      int dvprime_f32, const void* fwd_ws, void* dk, const int64_t* dk_strides, void* dv,
                      const int64_t* dv_strides, void* bwd_ws, int B, int Hkv, int T, int D, float scale,
                      void* stream);

/* ---- Lucid_Tril_Solver: the solve on keys that are already normalised ----
 * V' = P(K^)^-1 V with P_ij = exp(s K^_i . K^_j - 1/s) (j <= i) for a caller's K^ (no k_norm
 * inside: 1/rms is taken as 1), and its gradient dV = P^-T dV', dK^ = -s (M K^ + M^T K^),
 * M = tril((dV V'^T) * P), diagonal included -- dK^ itself, with no RMSNorm backward.
 * Replace Lucid_Tril_Solver.forward / .backward (modeling_lucid.py:284-312, :314-382), which
 * take key = K^ and return (grad_k, grad_v).  The result does not depend on the reference's
 * block size BS (a blocking of the same solve), and value is not modified (the reference's
 * forward subtracts from value's rows in place, :296-299).  Same arguments, layouts and
 * workspaces (lucid_fwd_workspace_bytes(B, Hkv, Hkv, T, D), lucid_precond_bwd_workspace_bytes)
 * as lucid_get_v_prime / lucid_precond_bwd; the _f32 variants those of lucid_get_v_prime_f32 /
 * lucid_precond_bwd_f32 (lucid_v_prime_f32_workspace_bytes). */
int lucid_tril_solve(const void* key_hat, const int64_t* k_strides, const void* v, const int64_t* v_strides,
                     float* vprime, void* fwd_ws, int B, int Hkv, int T, int D, float scale, void* stream);
int lucid_tril_solve_bwd(const void* key_hat, const int64_t* k_strides, const void* dvprime,
                         const int64_t* dvprime_strides, int dvprime_f32, const void* fwd_ws, void* dk,
                         const int64_t* dk_strides, void* dv, const int64_t* dv_strides, void* bwd_ws, int B, int Hkv,
                         int T, int D, float scale, void* stream);
int lucid_tril_solve_f32(const float* key_hat, const int64_t* k_strides, const float* v, const int64_t* v_strides,
                         float* vprime, void* fwd_ws, int B, int Hkv, int T, int D, float scale, void* stream);
int lucid_tril_solve_bwd_f32(const float* dvprime, const int64_t* dvprime_strides, const void* fwd_ws, float* dk,
                             const int64_t* dk_strides, float* dv, const int64_t* dv_strides, void* bwd_ws, int B,
                             int Hkv, int T, int D, float scale, void* stream);

/* Bytes of the decoding workspace for caches of capacity T_cap (0 on bad sizes). */
size_t lucid_decode_workspace_bytes(int B, int Hq, int Hkv, int T_cap, int D);

/* One decoding step: a new token per sequence (q [B,Hq,1,D], k and v [B,Hkv,1,D])
 * against the caches k_cache (keys with RoPE applied, as the attention saw them) and
 * vp_cache (V' rows, bf16), both [B,Hkv,T_cap,D] (padded rows of Dp columns for
 * other head dims) with rows [0, T_past) valid.
 * Computes the token's V' row with the exact diagonal,
 *   v'_t = (v_t - sum_{j<t} P_tj v'_j) / P_tt,
 * writes it to vp_new (fp32 [B,Hkv,D]) and appends (k_t, v'_t) at row T_past of the
 * caches, then o (strides {batch, head, -}, [B,1,Hq,D] in the reference layout) =
 * softmax over j <= t of s q.k_j times v'_j.  Any Hq / Hkv (groups above 31 query heads per kv
 * head run in chunks of query heads).
 * Replaces LucidAttention.get_new_v_prime (modeling_lucid.py:576-598, which omits the
 * division by P_tt) and the cached attention call of LucidAttention.forward
 * (:475-496); a decoded row equals the same row of lucid_attn_fwd on the whole
 * sequence. */
int lucid_decode(const void* q, const int64_t* q_strides, const void* k, const int64_t* k_strides, const void* v,
                 const int64_t* v_strides, void* k_cache, const int64_t* k_cache_strides, void* vp_cache,
                 const int64_t* vp_cache_strides, void* o, const int64_t* o_strides, float* vp_new, void* ws, int B,
                 int Hq, int Hkv, int T_past, int T_cap, int D, float scale, float eps, void* stream);

/* Bytes of the workspace of lucid_decode_tokens for L new tokens per call and caches of
 * capacity T_cap (0 on bad sizes). */
size_t lucid_decode_tokens_workspace_bytes(int B, int Hq, int Hkv, int L, int T_cap, int D);

/* L new tokens per sequence in one call (q [B,Hq,L,D], k and v [B,Hkv,L,D], rows in
 * order; o [B,L,Hq,D] by its strides {batch, head, time}; vp_new fp32 [B,Hkv,L,D]
 * contiguous), appended at rows T_past .. T_past+L-1 of the caches (T_past + L <= T_cap).
 * Each token's V' row is the exact prefill row: it is coupled to the cached rows and to
 * the earlier new tokens, v'_t = (v_t - sum_{j<t} P_tj v'_j) / P_tt, and each token
 * attends to the cache and to the new tokens up to itself.  The tokens run in passes of
 * 32 / (Hq/Hkv + 1) (the columns of one score tile), each pass reading the caches once.
 * Replaces LucidAttention.get_new_v_prime for L_k new tokens (modeling_lucid.py:576-598,
 * which couples a new token to the cache only) and the cached attention call
 * (:475-496).  lucid_decode is this entry with L = 1. */
int lucid_decode_tokens(const void* q, const int64_t* q_strides, const void* k, const int64_t* k_strides,
                        const void* v, const int64_t* v_strides, void* k_cache, const int64_t* k_cache_strides,
                        void* vp_cache, const int64_t* vp_cache_strides, void* o, const int64_t* o_strides,
                        float* vp_new, void* ws, int B, int Hq, int Hkv, int L, int T_past, int T_cap, int D,
                        float scale, float eps, void* stream);

/* lucid_decode without a workspace argument: the same decoding step, with its split
 * partials in a static 4 MiB (4194304-byte) device array of the library instead of `ws`,
 * so that it calls no allocator (hipMalloc, hipFree or an allocating library routine).
 * No counterpart in the reference: for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid allocation).  Sizes whose partials
 * exceed 4 MiB (B*Hkv above about 900 at head dim 128 with 8 query heads per kv head) are
 * rejected with LUCID_EINVAL and a message before anything runs; use lucid_decode for them.  Each GPU
 * holds its own array until the process ends, found on a device's first call; every
 * call on one GPU shares it, so calls that overlap on one GPU (other streams, other
 * threads) race. */
int lucid_decode_noalloc(const void* q, const int64_t* q_strides, const void* k, const int64_t* k_strides,
                         const void* v, const int64_t* v_strides, void* k_cache, const int64_t* k_cache_strides,
                         void* vp_cache, const int64_t* vp_cache_strides, void* o, const int64_t* o_strides,
                         float* vp_new, int B, int Hq, int Hkv, int T_past, int T_cap, int D, float scale, float eps,
                         void* stream);

/* The decoder's elementwise layers, one pass each (the Llama-LUCID model around the attention
 * core; the reference computes them as chains of torch ops).  bf16 tensors, rows contiguous.
 * lucid_rmsnorm_fwd: y[N][H] = w * bf16(x * rstd), rstd[n] = 1/sqrt(mean(x[n]^2) + eps) (fp32;
 * saved for the backward), replacing LlamaRMSNorm.forward (modeling_lucid.py:58-75).
 * lucid_rmsnorm_bwd: dx and dw (summed over the rows in a fixed order) from dy, with a
 * caller-owned fp32 workspace of lucid_rmsnorm_bwd_workspace_bytes(N, H).  H must be 512, 1024,
 * 2048 or 4096.  lucid_rope: out = x cos + rotate_half(x) sin (transpose = 1: the adjoint, for
 * the backward) for x and out [B, Hn, T, 64] at element strides x_strides / out_strides =
 * (b, h, t), multiples of 8, with cos / sin bf16 [B*T][64] (one row per token), pointers
 * 16-byte aligned, replacing apply_rotary_pos_emb (modeling_lucid.py:118-145). */
int lucid_rmsnorm_fwd(const void* x, const void* w, void* y, float* rstd, int N, int H, float eps, void* stream);
size_t lucid_rmsnorm_bwd_workspace_bytes(int N, int H);
int lucid_rmsnorm_bwd(const void* x, const void* w, const void* dy, const float* rstd, void* dx, void* dw,
                      void* workspace, int N, int H, void* stream);
int lucid_rope(const void* x, const int64_t x_strides[3], int B, int Hn, int T, const void* cos, const void* sin,
               void* out, const int64_t out_strides[3], int D, int transpose, void* stream);

/* lucid_swiglu_fwd: h = silu(g) * u over n bf16 values, replacing the act_fn(gate) * up of
 * LlamaMLP.forward (modeling_lucid.py:155-167); lucid_swiglu_bwd: dg = dh u silu'(g),
 * du = dh silu(g).  Pointers 16-byte aligned.
 * lucid_causal_lm_loss_fwd / _bwd: the causal-LM cross entropy of LlamaForCausalLM.forward
 * (modeling_lucid.py:847-967; F.cross_entropy on logits[:, :-1] in fp32 against labels[:, 1:],
 * ignore index -100) over bf16 logits [R = B*T][V] at row_stride elements (V and the stride
 * multiples of 8), labels int64 [R].  The forward writes per row lse, loss (lse - logit of the
 * target; 0 where the row does not count, NaN for a target outside [0, V) other than -100) and
 * valid (1 or 0): the loss is sum(loss) / sum(valid).  The backward writes dlogits [R][V]
 * = (softmax - onehot) * scale[0] on counted rows and 0 elsewhere (scale: a device float,
 * dloss / sum(valid)). */
int lucid_swiglu_fwd(const void* g, const void* u, void* h, int64_t n, void* stream);
int lucid_swiglu_bwd(const void* g, const void* u, const void* dh, void* dg, void* du, int64_t n, void* stream);
int lucid_causal_lm_loss_fwd(const void* logits, int64_t row_stride, const int64_t* labels, int R, int T, int V,
                             float* lse, float* loss, float* valid, void* stream);
int lucid_causal_lm_loss_bwd(const void* logits, int64_t row_stride, const int64_t* labels, int R, int T, int V,
                             const float* lse, const float* valid, const float* scale, void* dlogits, void* stream);

/* One AdamW step (decoupled weight decay) over n parameter tensors, the update of
 * torch.optim.AdamW, the default optimizer of the HF Trainer that the reference's training
 * script builds (run_clm_chunk.py:776; no counterpart in modeling_lucid.py):
 *   p <- p (1 - lr wd);  m <- m + (1 - beta1)(g - m);  v <- beta2 v + (1 - beta2) g^2;
 *   p <- p - lr / (1 - beta1^step) * m / (sqrt(v) / sqrt(1 - beta2^step) + eps)
 * in fp32, each stored value rounded once.  params / grads / exp_avgs / exp_avg_sqs are host
 * arrays of n device pointers to contiguous tensors of numels[i] elements, all of one dtype
 * (LUCID_DTYPE_BF16 or LUCID_DTYPE_F32), each aligned to 8 elements; step (>= 1) is the
 * count after this update.  One launch per 48 tensors. */
int lucid_adamw_step(int n, void* const* params, const void* const* grads, void* const* exp_avgs,
                     void* const* exp_avg_sqs, const int64_t* numels, int dtype, float lr, float beta1, float beta2,
                     float eps, float weight_decay, int64_t step, void* stream);

/* Per-kernel timing (no counterpart in the reference; used by bench.py).
 * When enabled, every launch is bracketed by two HIP events on its stream.
 * lucid_profile_collect() waits for the recorded events, folds them into
 * per-kernel totals and returns the number of distinct kernels;
 * lucid_profile_entry(i, ...) reads total milliseconds and launch count of
 * kernel i; lucid_profile_reset() clears the totals.  lucid_profile_only(name) times only
 * the launches of the named kernel (null or "": every kernel), so that a timed region
 * carries one kernel's events instead of two per launch.  Not thread safe. */
void lucid_profile_enable(int on);
void lucid_profile_only(const char* name);
int lucid_profile_collect(void);
int lucid_profile_entry(int idx, char* name, int name_len, double* total_ms, long* count);
void lucid_profile_reset(void);

#pragma GCC visibility pop

#ifdef __cplusplus
}
#endif

#endif /* LUCID_AMD_H */
