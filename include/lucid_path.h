/*
 * lucid_path -- C ABI of the MI355X (gfx950) LUCID-Path kernels.
 *
 * LUCID-Path (lucid_path/triton_code/parallel.py:180-241):
 *   O = (I + L)^-1 V,  L_ij = exp(s A_ij - 1/s) for j < i,
 *   A_ij = q_i^T H_i ... H_{j+1} k_j,  H_t = I - beta_t w_t w_t^T.
 * Layouts as the reference: q [B,T,HQ,K], k/w [B,T,H,K], v [B,T,H,V], beta [B,T,H],
 * o [B,T,HQ,V]; element strides {batch, head, time}, last axis contiguous.
 * bf16 tensors with K = V = 64 or K = V = 128, or fp32 tensors (the _f32 entry points) with
 * K = V = 64; T a multiple of 64 (the Python layer zero-pads the sequence end, exact for every
 * real row since L is strictly lower triangular, and smaller head dims to 64 or 128).
 * Buffers are caller-owned (no device allocation; the bounded chain waits set up a 4-byte
 * pinned flag on the first chain call per device, as in lucid_amd.h -- call
 * lucid_path_chain_status() once before HIP graph capture); launches go on `stream`.
 * Return codes as in lucid_amd.h (0 ok, 1 bad argument, 1000 + hipError_t).
 */
#ifndef LUCID_PATH_H
#define LUCID_PATH_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* The libraries are built with hidden symbol visibility; only these entry points are exported. */
#pragma GCC visibility push(default)

/* ABI version of this header. */
int lucid_path_abi_version(void);

/* Text of the last error on the calling thread. */
const char* lucid_path_last_error(void);

/* Bounded chain waits of this library (the forward solve and the dV chain hand blocks
 * between workgroups through progress counters): as lucid_chain_status /
 * lucid_set_chain_wait_limit in lucid_amd.h; an earlier give-up is reported as 2 by the
 * next lucid_path_fwd / lucid_path_bwd call.  No counterpart in the reference. */
int lucid_path_chain_status(void);
int lucid_path_set_chain_wait_limit(double seconds);

/* Bytes of the forward workspace (kept alive for lucid_path_bwd).  Both
 * workspaces must be 256-byte aligned. */
size_t lucid_path_fwd_workspace_bytes(int B, int T, int H, int HQ, int K);

/* Forward: o = (I + L)^-1 v; if kcache is non-null also the decode key cache
 * [B,T,H,K] (keys carried through every later Householder).
 * Replaces ParallelLUCIDPathAttentionFunction.forward (parallel.py:27-76): the
 * kkt + solve_tril WY step (:39-51), triangular_solve_fwd_fn (:54-65) and
 * prepare_k_cache_fn (:68). */
int lucid_path_fwd(const void* q, const int64_t* q_strides, const void* k, const int64_t* k_strides,
                   const void* v, const int64_t* v_strides, const void* w, const int64_t* w_strides,
                   const void* beta, const int64_t* beta_strides, void* o, const int64_t* o_strides,
                   void* kcache, const int64_t* kcache_strides, void* fwd_ws, int B, int T, int H, int HQ,
                   int K, float scale, void* stream);

/* Bytes of the backward scratch workspace. */
size_t lucid_path_bwd_workspace_bytes(int B, int T, int H, int HQ, int K);

/* Backward of sum(o * dout) w.r.t. q [B,T,HQ,K], k, v, w [B,T,H,*] and beta [B,T,H]
 * (bf16 outputs, GQA sums applied).  `o` and `fwd_ws` are those of the forward call.
 * Replaces ParallelLUCIDPathAttentionFunction.backward (parallel.py:78-177): the dv
 * solve (:103-114), bwd_prepare (:116-127), the Householder products, transform_q and
 * the inter/intra-chunk gradient kernels (:129-163) and the GQA reduction (:165-171). */
int lucid_path_bwd(const void* dout, const int64_t* do_strides, const void* q, const int64_t* q_strides,
                   const void* k, const int64_t* k_strides, const void* w, const int64_t* w_strides,
                   const void* beta, const int64_t* beta_strides, const void* o, const int64_t* o_strides,
                   const void* fwd_ws, void* dq, const int64_t* dq_strides, void* dk, const int64_t* dk_strides,
                   void* dv, const int64_t* dv_strides, void* dw, const int64_t* dw_strides, void* dbeta,
                   const int64_t* dbeta_strides, void* bwd_ws, int B, int T, int H, int HQ, int K, float scale,
                   void* stream);

/*
 * PaTH softmax attention, the softmax half of a LUCID-Path layer, on the same path
 * logits (diagonal included, A_ii = q_i . k_i):
 *   o_i = sum_{j<=i} softmax_j(s A_ij) v_j.
 * The reference ships only its forward kernels (intra_chunk_preprocess_fwd.py:14-168,
 * parallel_path_fwd.py:13-170, not called by parallel.py); their backward lives in the
 * unvendored flash-linear-attention package.  Same layouts, dtypes and constraints as
 * lucid_path_fwd / lucid_path_bwd (the forward workspace layout differs: size it with
 * lucid_path_softmax_fwd_workspace_bytes).
 */
size_t lucid_path_softmax_fwd_workspace_bytes(int B, int T, int H, int HQ, int K);

/* Forward: o = softmax(s A) v; the row log-sum-exp is kept in fwd_ws for the backward;
 * kcache as in lucid_path_fwd.  Replaces intra_chunk_preprocess_fwd_fn followed by
 * parallel_path_fwd_fn (intra_chunk_preprocess_fwd.py:124-168, parallel_path_fwd.py:127-170). */
int lucid_path_softmax_fwd(const void* q, const int64_t* q_strides, const void* k, const int64_t* k_strides,
                           const void* v, const int64_t* v_strides, const void* w, const int64_t* w_strides,
                           const void* beta, const int64_t* beta_strides, void* o, const int64_t* o_strides,
                           void* kcache, const int64_t* kcache_strides, void* fwd_ws, int B, int T, int H, int HQ,
                           int K, float scale, void* stream);

size_t lucid_path_softmax_bwd_workspace_bytes(int B, int T, int H, int HQ, int K);

/* Backward of sum(o * dout) w.r.t. q, k, v, w and beta (bf16, GQA sums applied); `o`
 * and `fwd_ws` are those of lucid_path_softmax_fwd.  No counterpart in the reference
 * (its PaTH softmax backward is in the unvendored fla package); the gradients equal
 * float64 autograd of the definition. */
int lucid_path_softmax_bwd(const void* dout, const int64_t* do_strides, const void* q, const int64_t* q_strides,
                           const void* k, const int64_t* k_strides, const void* v, const int64_t* v_strides,
                           const void* w, const int64_t* w_strides, const void* beta, const int64_t* beta_strides,
                           const void* o, const int64_t* o_strides, const void* fwd_ws, void* dq,
                           const int64_t* dq_strides, void* dk, const int64_t* dk_strides, void* dv,
                           const int64_t* dv_strides, void* dw, const int64_t* dw_strides, void* dbeta,
                           const int64_t* dbeta_strides, void* bwd_ws, int B, int T, int H, int HQ, int K,
                           float scale, void* stream);

/*
 * fp32 tensors (the reference's LUCID-Path model is fp32: lucid_path/config/config.json:5).
 * Same contracts as the bf16 entry points above, K = V = 64 (smaller head dims zero-padded
 * by the caller); every product of the sweeps runs as a 3-term bf16 split (hi.hi + hi.lo +
 * lo.hi) on hi / lo copies of its operands, ~fp32 accuracy.  The workspaces are larger
 * (the lo copies): size them with the _f32 workspace functions.  The reference's Triton
 * kernels take fp32 tensors through the same entry points (parallel.py:180-241).
 */
size_t lucid_path_fwd_f32_workspace_bytes(int B, int T, int H, int HQ, int K);
int lucid_path_fwd_f32(const float* q, const int64_t* q_strides, const float* k, const int64_t* k_strides,
                       const float* v, const int64_t* v_strides, const float* w, const int64_t* w_strides,
                       const float* beta, const int64_t* beta_strides, float* o, const int64_t* o_strides,
                       float* kcache, const int64_t* kcache_strides, void* fwd_ws, int B, int T, int H, int HQ, int K,
                       float scale, void* stream);
size_t lucid_path_bwd_f32_workspace_bytes(int B, int T, int H, int HQ, int K);
int lucid_path_bwd_f32(const float* dout, const int64_t* do_strides, const float* q, const int64_t* q_strides,
                       const float* k, const int64_t* k_strides, const float* w, const int64_t* w_strides,
                       const float* beta, const int64_t* beta_strides, const float* o, const int64_t* o_strides,
                       const void* fwd_ws, float* dq, const int64_t* dq_strides, float* dk, const int64_t* dk_strides,
                       float* dv, const int64_t* dv_strides, float* dw, const int64_t* dw_strides, float* dbeta,
                       const int64_t* dbeta_strides, void* bwd_ws, int B, int T, int H, int HQ, int K, float scale,
                       void* stream);
size_t lucid_path_softmax_fwd_f32_workspace_bytes(int B, int T, int H, int HQ, int K);
int lucid_path_softmax_fwd_f32(const float* q, const int64_t* q_strides, const float* k, const int64_t* k_strides,
                               const float* v, const int64_t* v_strides, const float* w, const int64_t* w_strides,
                               const float* beta, const int64_t* beta_strides, float* o, const int64_t* o_strides,
                               float* kcache, const int64_t* kcache_strides, void* fwd_ws, int B, int T, int H,
                               int HQ, int K, float scale, void* stream);
size_t lucid_path_softmax_bwd_f32_workspace_bytes(int B, int T, int H, int HQ, int K);
int lucid_path_softmax_bwd_f32(const float* dout, const int64_t* do_strides, const float* q,
                               const int64_t* q_strides, const float* k, const int64_t* k_strides, const float* v,
                               const int64_t* v_strides, const float* w, const int64_t* w_strides, const float* beta,
                               const int64_t* beta_strides, const float* o, const int64_t* o_strides,
                               const void* fwd_ws, float* dq, const int64_t* dq_strides, float* dk,
                               const int64_t* dk_strides, float* dv, const int64_t* dv_strides, float* dw,
                               const int64_t* dw_strides, float* dbeta, const int64_t* dbeta_strides, void* bwd_ws,
                               int B, int T, int H, int HQ, int K, float scale, void* stream);

/* Per-kernel timing with HIP events (no counterpart in the reference; used by
 * bench.py), same contract as lucid_profile_* in lucid_amd.h. */
void lucid_path_profile_enable(int on);
void lucid_path_profile_only(const char* name);
int lucid_path_profile_collect(void);
int lucid_path_profile_entry(int idx, char* name, int name_len, double* total_ms, long* count);
void lucid_path_profile_reset(void);

#pragma GCC visibility pop

#ifdef __cplusplus
}
#endif

#endif /* LUCID_PATH_H */
