"""LUCID-Path restated on the CPU -- test infrastructure only (see oracle/__init__.py).

Definition (reference ``lucid_path/triton_code``; parallel.py:180-241):

* ``H_t = I - beta_t w_t w_t^T``
* ``A_ij = q_i^T H_i H_{i-1} ... H_{j+1} k_j`` for ``j < i``  (PaTH path logits)
* ``L_ij = exp(s A_ij - 1/s)`` for ``j < i``, 0 otherwise (the kernels use ``-1/s``,
  triangular_solve_fwd.py:202,218; the docstring's ``-s`` at parallel.py:195 is stale)
* ``O = (I + L)^-1 V`` (unit diagonal), per query head; kv head = query head // G
* defaults: ``q = k`` and ``s = K^-1/2`` (parallel.py:224-228)
* layouts ``q [B,T,HQ,K]``, ``k, w [B,T,H,K]``, ``v [B,T,H,V]``, ``beta [B,T,H]``,
  ``o [B,T,HQ,V]``

Functions work on float64 torch tensors (CPU).  ``path_attention_bruteforce`` follows
the definition with one explicit Householder application per step; the chunked
restatement ``path_attention_chunked`` follows the reference's chunk algebra
(parallel.py:39-51, triangular_solve_fwd.py:118-225) and is differentiable, so
torch autograd gives the gradients the backward must reproduce.

Pinning: tests/test_oracle_path.py checks chunked == brute force (several chunk
sizes), the WY identity ``I - W^T T_inv (beta W) = H_e ... H_s`` against explicit
products, beta = 0 (A = q.k, no transport), the k-cache decode identity, the
unit-diagonal solve residual, and gradcheck of the brute force.
"""
from __future__ import annotations

import torch


def householder_apply(x: torch.Tensor, w: torch.Tensor, beta: torch.Tensor) -> torch.Tensor:
    """``H x`` for ``H = I - beta w w^T`` (x [..., K], w [..., K], beta [...])."""
    return x - beta[..., None] * (x * w).sum(-1, keepdim=True) * w


def path_logits_bruteforce(q, k, w, beta):
    """A[b, hq, i, j] = q_i^T H_i ... H_{j+1} k_j for j < i (0 elsewhere); O(T^2 K) per head."""
    B, T, HQ, K = q.shape
    H = k.shape[2]
    G = HQ // H
    out = torch.zeros(B, HQ, T, T, dtype=q.dtype)
    for b in range(B):
        for hq in range(HQ):
            h = hq // G
            for j in range(T):
                r = k[b, j, h]
                for i in range(j + 1, T):
                    r = householder_apply(r, w[b, i, h], beta[b, i, h])
                    out[b, hq, i, j] = q[b, i, hq] @ r
    return out


def solve_unit_lower(L: torch.Tensor, V: torch.Tensor) -> torch.Tensor:
    """(I + L)^-1 V for strictly lower L [..., T, T]."""
    T = L.shape[-1]
    eye = torch.eye(T, dtype=L.dtype)
    return torch.linalg.solve_triangular(eye + L, V, upper=False, unitriangular=True)


def path_attention_bruteforce(q, k, v, w, beta, scale=None):
    """O [B,T,HQ,V] from the definition (small T only)."""
    K = k.shape[-1]
    scale = K ** -0.5 if scale is None else scale
    G = q.shape[2] // k.shape[2]
    A = path_logits_bruteforce(q, k, w, beta)
    T = A.shape[-1]
    mask = torch.ones(T, T, dtype=torch.bool).tril(-1)
    L = torch.where(mask, torch.exp(A * scale - 1.0 / scale), torch.zeros((), dtype=A.dtype))
    vv = v.permute(0, 2, 1, 3).repeat_interleave(G, dim=1)  # [B, HQ, T, V]
    o = solve_unit_lower(L, vv)
    return o.permute(0, 2, 1, 3).contiguous()


def wy_chunk(wc: torch.Tensor, bc: torch.Tensor):
    """WY form of one chunk (chunk_scaled_dot_kkt_fwd + solve_tril, parallel.py:39-51).

    wc [C, K], bc [C] -> (T_inv [C, C], W2 [C, K]) with
    ``T_inv = (I + stril(diag(beta) W W^T))^-1`` and ``W2 = T_inv (beta W)``, so that
    ``H_e ... H_s = I - W^T W2`` (row vectors are right-multiplied when crossing the chunk).
    """
    C = wc.shape[0]
    wb = wc * bc[:, None]
    a = torch.tril(wb @ wc.T, -1)
    eye = torch.eye(C, dtype=wc.dtype)
    t_inv = torch.linalg.solve_triangular(eye + a, eye, upper=False, unitriangular=True)
    return t_inv, t_inv @ wb


def path_attention_chunked(q, k, v, w, beta, scale=None, C=64, return_intermediates=False):
    """Chunk restatement of ParallelLUCIDPathAttentionFunction.forward (differentiable).

    Per chunk (triangular_solve_fwd.py:118-148):
      q_new = q - tril(q W^T) W2;  k_new^T = k^T - W^T T_inv stril(beta W k^T);
      A_diag = tril(q k^T - tril(q W^T) T_inv stril(beta W k^T)).
    Off-diagonal blocks (:170-196): A_IJ = Q k_new_J^T with Q = q_new_I propagated
    through chunks I-1 .. J+1 by ``Q <- Q - (Q W_J^T) W2_J`` (J descending).
    Solve: R_I = V_I - sum_{J<I} L_IJ O_J, (I + stril L_II) O_I = R_I.
    """
    B, T, HQ, K = q.shape
    H = k.shape[2]
    G = HQ // H
    scale = K ** -0.5 if scale is None else scale
    if T % C:
        raise ValueError("T must be a multiple of the chunk size")
    NT = T // C
    o = torch.zeros(B, T, HQ, v.shape[-1], dtype=q.dtype)
    outs = []
    inter = {}
    for b in range(B):
        for hq in range(HQ):
            h = hq // G
            qn, kn, w2s, ldiag = [], [], [], []
            for c in range(NT):
                sl = slice(c * C, (c + 1) * C)
                wc, bc, qc, kc = w[b, sl, h], beta[b, sl, h], q[b, sl, hq], k[b, sl, h]
                t_inv, w2 = wy_chunk(wc, bc)
                qw = torch.tril(qc @ wc.T)
                wbk = torch.tril((wc * bc[:, None]) @ kc.T, -1)
                qn.append(qc - qw @ w2)
                kn.append(kc - (wc.T @ (t_inv @ wbk)).T)
                a_diag = torch.tril(qc @ kc.T - qw @ t_inv @ wbk)
                ldiag.append(torch.tril(torch.exp(a_diag * scale - 1.0 / scale), -1))
                w2s.append(w2)
            blocks = []
            for i in range(NT):
                r = v[b, i * C:(i + 1) * C, h]
                qq = qn[i]
                for j in range(i - 1, -1, -1):
                    a_ij = qq @ kn[j].T
                    r = r - torch.exp(a_ij * scale - 1.0 / scale) @ blocks[j]
                    qq = qq - (qq @ w[b, j * C:(j + 1) * C, h].T) @ w2s[j]
                eye = torch.eye(C, dtype=q.dtype)
                blocks.append(torch.linalg.solve_triangular(eye + ldiag[i], r, upper=False, unitriangular=True))
            outs.append((b, hq, torch.cat(blocks, 0)))
            if return_intermediates:
                inter[(b, hq)] = {"q_new": torch.cat(qn), "k_new": torch.cat(kn), "w2": torch.cat(w2s)}
    o = torch.stack([x for _, _, x in outs]).reshape(B, HQ, T, -1).permute(0, 2, 1, 3).contiguous()
    return (o, inter) if return_intermediates else o


def path_kcache_bruteforce(k, w, beta):
    """k_cache_j = H_{T-1} ... H_{j+1} k_j (prepare_k_cache.py:40-46): keys carried to the sequence end."""
    B, T, H, K = k.shape
    out = k.clone()
    for b in range(B):
        for h in range(H):
            for j in range(T):
                r = k[b, j, h]
                for i in range(j + 1, T):
                    r = householder_apply(r, w[b, i, h], beta[b, i, h])
                out[b, j, h] = r
    return out


def path_attention_grads(q, k, v, w, beta, do, scale=None, C=64):
    """(dq, dk, dv, dw, dbeta) of sum(O * dO) by float64 autograd of the chunked restatement."""
    leaves = [t.detach().clone().requires_grad_() for t in (q, k, v, w, beta)]
    o = path_attention_chunked(*leaves, scale=scale, C=C)
    (o * do).sum().backward()
    return tuple(t.grad for t in leaves)


# ---------------------------------------------------------------------------
# PaTH softmax attention (the softmax half of a LUCID-Path layer)
#
#   O_i = sum_{j<=i} softmax_j(s A_ij) v_j,  A_ij = q_i^T H_i ... H_{j+1} k_j  (A_ii = q_i . k_i)
#
# Reference: the forward kernels intra_chunk_preprocess_fwd.py:14-121 (in-chunk
# logits including the diagonal, o, row sum L and row max M in the exp2 domain)
# and parallel_path_fwd.py:13-124 (online-softmax continuation over earlier
# chunks with the query carried down by q <- q - (q W^T) W2, output o and
# L_new = log2(l) + m).  Their backward lives in the unvendored fla package, so
# gradients are pinned by float64 autograd of the brute-force definition.
# ---------------------------------------------------------------------------


def path_softmax_logits_bruteforce(q, k, w, beta):
    """A[b, hq, i, j] for j <= i (the diagonal is q_i . k_i, no reflection applies)."""
    A = path_logits_bruteforce(q, k, w, beta)
    G = q.shape[2] // k.shape[2]
    kk = k.repeat_interleave(G, dim=2)
    diag = (q * kk).sum(-1).permute(0, 2, 1)  # [B, HQ, T]
    return A + torch.diag_embed(diag)


def path_softmax_bruteforce(q, k, v, w, beta, scale=None, return_lse=False):
    """O [B,T,HQ,V] = causal softmax(s A) V from the definition (small T only);
    with ``return_lse`` also the natural log-sum-exp [B,HQ,T] of each row."""
    K = k.shape[-1]
    scale = K ** -0.5 if scale is None else scale
    G = q.shape[2] // k.shape[2]
    A = path_softmax_logits_bruteforce(q, k, w, beta) * scale
    T = A.shape[-1]
    mask = torch.ones(T, T, dtype=torch.bool).tril()
    A = A.masked_fill(~mask, float("-inf"))
    vv = v.permute(0, 2, 1, 3).repeat_interleave(G, dim=1)
    o = (torch.softmax(A, dim=-1) @ vv).permute(0, 2, 1, 3).contiguous()
    return (o, torch.logsumexp(A, dim=-1)) if return_lse else o


def path_softmax_chunked(q, k, v, w, beta, scale=None, C=64):
    """Chunk restatement of the two PaTH softmax forward kernels (differentiable).

    In-chunk (intra_chunk_preprocess_fwd.py:71-115): with T_inv the WY matrix of the
    chunk, ``A = tril(q k^T - tril(q W^T) T_inv stril(beta W k^T))`` (diagonal
    included), row max m, l = sum exp2(s' A - m), o = exp2(...) V, s' = s log2(e).
    Inter-chunk (parallel_path_fwd.py:77-117): for earlier chunks J descending,
    S = q_new k_new_J^T, online-softmax update of (m, l, o), then
    ``q_new <- q_new - (q_new W_J^T) W2_J``.  Returns (o, L_new) with
    ``L_new = log2(l) + m`` [B,T,HQ] as the reference's second kernel stores it.
    """
    B, T, HQ, K = q.shape
    H = k.shape[2]
    G = HQ // H
    scale = K ** -0.5 if scale is None else scale
    if T % C:
        raise ValueError("T must be a multiple of the chunk size")
    sm = scale * 1.4426950408889634
    NT = T // C
    outs, lses = [], []
    for b in range(B):
        for hq in range(HQ):
            h = hq // G
            qn, kn, w2s, ad = [], [], [], []
            for c in range(NT):
                sl = slice(c * C, (c + 1) * C)
                wc, bc, qc, kc = w[b, sl, h], beta[b, sl, h], q[b, sl, hq], k[b, sl, h]
                t_inv, w2 = wy_chunk(wc, bc)
                qw = torch.tril(qc @ wc.T)
                wbk = torch.tril((wc * bc[:, None]) @ kc.T, -1)
                qn.append(qc - qw @ w2)
                kn.append(kc - (wc.T @ (t_inv @ wbk)).T)
                ad.append(qc @ kc.T - qw @ t_inv @ wbk)
                w2s.append(w2)
            mask = torch.ones(C, C, dtype=torch.bool).tril()
            rows_o, rows_l = [], []
            for i in range(NT):
                s_ii = (ad[i] * sm).masked_fill(~mask, float("-inf"))
                m = s_ii.max(-1).values
                p = torch.exp2(s_ii - m[:, None])
                l = p.sum(-1)
                o = p @ v[b, i * C:(i + 1) * C, h]
                qq = qn[i]
                for j in range(i - 1, -1, -1):
                    s = (qq @ kn[j].T) * sm
                    m_new = torch.maximum(m, s.max(-1).values)
                    alpha = torch.exp2(m - m_new)
                    p = torch.exp2(s - m_new[:, None])
                    o = o * alpha[:, None] + p @ v[b, j * C:(j + 1) * C, h]
                    l = l * alpha + p.sum(-1)
                    m = m_new
                    qq = qq - (qq @ w[b, j * C:(j + 1) * C, h].T) @ w2s[j]
                rows_o.append(o / l[:, None])
                rows_l.append(torch.log2(l) + m)
            outs.append(torch.cat(rows_o, 0))
            lses.append(torch.cat(rows_l, 0))
    o = torch.stack(outs).reshape(B, HQ, T, -1).permute(0, 2, 1, 3).contiguous()
    lse2 = torch.stack(lses).reshape(B, HQ, T).permute(0, 2, 1).contiguous()
    return o, lse2


def path_softmax_grads(q, k, v, w, beta, do, scale=None):
    """(dq, dk, dv, dw, dbeta) of sum(O * dO) by float64 autograd of the brute force."""
    leaves = [t.detach().clone().requires_grad_() for t in (q, k, v, w, beta)]
    o = path_softmax_bruteforce(*leaves, scale=scale)
    (o * do).sum().backward()
    return tuple(t.grad for t in leaves)
