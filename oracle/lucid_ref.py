"""LUCID attention restated on the CPU -- test infrastructure only (see oracle/__init__.py).

Math (reference ``modeling_lucid.py``):

* ``s = d**-0.5``                                             (:392)
* ``K^ = K / sqrt(mean_d K^2 + eps)`` (nn.RMSNorm, no affine)  (:409, :564)
* ``P_ij = exp(s * K^_i . K^_j - 1/s)`` for ``j <= i``, else 0 (:565-569)
* ``V' = P^-1 V``  (lower triangular, non-unit diagonal)       (:570)
* ``O = softmax(s Q K^T + causal) repeat_kv(V')`` with the RAW K (:520-530)
* gradients as in ``Lucid_Tril_Solver.backward``               (:314-382)

Every function works on numpy float64 arrays in the reference layout
``q [B, Hq, T, d]``, ``k, v [B, Hkv, T, d]``; the attention output is returned
as ``[B, T, Hq, d]`` like ``eager_lucid_attention_forward`` (:546).

Pinning: ``tests/test_oracle_lucid.py`` checks these functions against
closed forms (T=1, identical keys, orthogonal keys), the solve residual,
the blockwise restatement (block-size invariance), an independent
unit-diagonal restatement (experiment1_cumavg.py:188-202) and float64 torch
autograd (gradcheck) of the dense definition.
"""
from __future__ import annotations

import numpy as np
import scipy.linalg as sla


def rms_inv(k: np.ndarray, eps: float) -> np.ndarray:
    """Row factor ``r = 1/sqrt(mean_d k^2 + eps)`` of nn.RMSNorm(elementwise_affine=False).

    modeling_lucid.py:409 (k_norm), :564 (applied in get_v_prime).
    """
    return 1.0 / np.sqrt(np.mean(k * k, axis=-1) + eps)


def k_hat(k: np.ndarray, eps: float) -> np.ndarray:
    return k * rms_inv(k, eps)[..., None]


def precond_matrix(khat: np.ndarray, scale: float) -> np.ndarray:
    """Dense lower-triangular P for one head, ``khat [T, d]`` -> ``[T, T]``.

    modeling_lucid.py:565-569: einsum K^K^T, mul_(scaling), sub_(1/scaling),
    masked_fill_(~causal, -inf), exp_().
    """
    s = khat @ khat.T * scale - 1.0 / scale
    t = s.shape[0]
    s[np.triu_indices(t, 1)] = -np.inf
    return np.exp(s)


def repeat_kv(x: np.ndarray, n_rep: int) -> np.ndarray:
    """modeling_lucid.py:171-180: [B, Hkv, T, d] -> [B, Hkv*n_rep, T, d] (head h -> h//n_rep)."""
    if n_rep == 1:
        return x
    return np.repeat(x, n_rep, axis=1)


def vprime_dense(k: np.ndarray, v: np.ndarray, scale: float, eps: float) -> np.ndarray:
    """``V' = P^-1 V`` per (batch, kv head) -- the dense branch of get_v_prime (modeling_lucid.py:561-570)."""
    kh = k_hat(k, eps)
    out = np.empty_like(v)
    for b in range(k.shape[0]):
        for h in range(k.shape[1]):
            p = precond_matrix(kh[b, h], scale)
            out[b, h] = sla.solve_triangular(p, v[b, h], lower=True)
    return out


def vprime_blockwise(k: np.ndarray, v: np.ndarray, scale: float, eps: float, bs: int) -> np.ndarray:
    """Block forward substitution of ``Lucid_Tril_Solver.forward`` (modeling_lucid.py:285-312).

    For row block i: ``rhs_i = V_i - sum_{j<i} exp(K^_i K^_j^T s - 1/s) V'_j`` then
    ``V'_i = tril(P_ii)^-1 rhs_i``.  Unlike the reference it does not mutate ``v``
    (the reference's ``rhs.sub_`` writes into the caller's value, :297).
    The reference asserts ``T > bs`` and ``T % bs == 0`` (:288-289); here only
    divisibility is required so that small block sizes can be compared.
    """
    t = k.shape[-2]
    if t % bs:
        raise ValueError(f"sequence length {t} must be divisible by block size {bs}")
    kh = k_hat(k, eps)
    vp = np.zeros_like(v)
    for i in range(0, t, bs):
        rhs = v[..., i:i + bs, :].copy()
        ki = kh[..., i:i + bs, :]
        for j in range(0, i, bs):
            e = np.exp(ki @ np.swapaxes(kh[..., j:j + bs, :], -1, -2) * scale - 1.0 / scale)
            rhs -= e @ vp[..., j:j + bs, :]
        e_ii = np.tril(np.exp(ki @ np.swapaxes(ki, -1, -2) * scale - 1.0 / scale))
        for idx in np.ndindex(*k.shape[:-2]):
            vp[idx + (slice(i, i + bs),)] = sla.solve_triangular(e_ii[idx], rhs[idx], lower=True)
    return vp


def causal_attention(q: np.ndarray, k: np.ndarray, vp: np.ndarray, scale: float):
    """``softmax(s Q K^T + causal) V'`` with GQA expansion; returns (O [B,T,Hq,d], probs [B,Hq,T,T]).

    modeling_lucid.py:520-530 (SDPA is_causal=True, enable_gqa=False after repeat_kv), :546 transpose.
    """
    g = q.shape[1] // k.shape[1]
    kr, vr = repeat_kv(k, g), repeat_kv(vp, g)
    s = q @ np.swapaxes(kr, -1, -2) * scale
    t = s.shape[-1]
    s = np.where(np.tril(np.ones((t, t), dtype=bool)), s, -np.inf)
    s = s - s.max(-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(-1, keepdims=True)
    o = p @ vr
    return np.swapaxes(o, 1, 2).copy(), p


def lucid_attention(q, k, v, scale=None, eps=1e-5, block=None):
    """Full LUCID forward: returns (O [B,T,Hq,d], V' [B,Hkv,T,d]).

    ``block=None`` uses the dense solve (get_v_prime for L < 2**16), otherwise
    the blockwise solver restatement with that block size.
    """
    d = q.shape[-1]
    scale = d ** -0.5 if scale is None else scale
    vp = vprime_dense(k, v, scale, eps) if block is None else vprime_blockwise(k, v, scale, eps, block)
    o, _ = causal_attention(q, k, vp, scale)
    return o, vp


def precond_backward(khat: np.ndarray, vp: np.ndarray, dvp: np.ndarray, scale: float):
    """Gradient of ``V' = P(K^)^-1 V`` for one head (modeling_lucid.py:314-382, dense form).

    ``dV = P^-T dV'``; ``M = tril((dV V'^T) * P)``; ``dK^ = -s (M K^ + M^T K^)``.
    Returns (dK^, dV).
    """
    p = precond_matrix(khat, scale)
    dv = sla.solve_triangular(p, dvp, lower=True, trans='T')
    m = np.tril((dv @ vp.T) * p)
    dkh = -scale * (m @ khat + m.T @ khat)
    return dkh, dv


def precond_backward_blockwise(khat, vp, dvp, scale, bs):
    """Blockwise restatement of Lucid_Tril_Solver.backward (modeling_lucid.py:314-382) for one head.

    Upper block solve bottom-up (:328-334), then the two block sums
    ``k1`` (rows, M K^) and ``k2`` (columns, M^T K^) (:340-379).
    """
    t = khat.shape[0]
    if t % bs:
        raise ValueError("T must be divisible by the block size")

    def e(a, b):
        return np.exp(khat[a:a + bs] @ khat[b:b + bs].T * scale - 1.0 / scale)

    dv = np.zeros_like(dvp)
    for i in range(t - bs, -bs, -bs):
        rhs = dvp[i:i + bs].copy()
        for j in range(t - bs, i, -bs):
            rhs -= e(j, i).T @ dv[j:j + bs]
        dv[i:i + bs] = sla.solve_triangular(np.triu(e(i, i).T), rhs, lower=False)
    gk = np.zeros_like(khat)
    for i in range(0, t, bs):
        k1 = ((dv[i:i + bs] @ vp[i:i + bs].T) * np.tril(e(i, i))) @ khat[i:i + bs]
        for j in range(0, i, bs):
            k1 += ((dv[i:i + bs] @ vp[j:j + bs].T) * e(i, j)) @ khat[j:j + bs]
        gk[i:i + bs] += k1
        # column sum for block i: sum over row blocks r >= i of M_ri^T K^_r
        k2 = ((dv[i:i + bs] @ vp[i:i + bs].T) * np.tril(e(i, i))).T @ khat[i:i + bs]
        for r in range(i + bs, t, bs):
            k2 += ((dv[r:r + bs] @ vp[i:i + bs].T) * e(r, i)).T @ khat[r:r + bs]
        gk[i:i + bs] += k2
    return -scale * gk, dv


def rmsnorm_backward(k: np.ndarray, dkh: np.ndarray, eps: float) -> np.ndarray:
    """Backward of ``K^ = K r``, ``r = (mean K^2 + eps)^-1/2``: ``dK = r (dK^ - K^ (K^.dK^)/d)``."""
    r = rms_inv(k, eps)[..., None]
    kh = k * r
    d = k.shape[-1]
    return r * (dkh - kh * np.sum(kh * dkh, axis=-1, keepdims=True) / d)


def lucid_attention_grads(q, k, v, do, scale=None, eps=1e-5):
    """Closed-form gradients of ``sum(O * dO)`` w.r.t. (q, k, v).

    ``do`` is ``[B, T, Hq, d]`` like O.  Returns (dq [B,Hq,T,d], dk, dv [B,Hkv,T,d]).
    Attention part: standard softmax backward; preconditioner part:
    :func:`precond_backward`; K^ -> K through :func:`rmsnorm_backward`.
    """
    d = q.shape[-1]
    scale = d ** -0.5 if scale is None else scale
    g = q.shape[1] // k.shape[1]
    o, vp = lucid_attention(q, k, v, scale, eps)
    _, p = causal_attention(q, k, vp, scale)
    dot = np.swapaxes(do, 1, 2)                       # [B, Hq, T, d]
    vr, kr = repeat_kv(vp, g), repeat_kv(k, g)
    dvp_r = np.swapaxes(p, -1, -2) @ dot
    dp = dot @ np.swapaxes(vr, -1, -2)
    ds = p * (dp - np.sum(dp * p, axis=-1, keepdims=True))
    dq = scale * ds @ kr
    dk_attn_r = scale * np.swapaxes(ds, -1, -2) @ q
    B, Hkv = k.shape[:2]
    dvp = dvp_r.reshape(B, Hkv, g, *dvp_r.shape[2:]).sum(2)
    dk_attn = dk_attn_r.reshape(B, Hkv, g, *dk_attn_r.shape[2:]).sum(2)
    kh = k_hat(k, eps)
    dkh = np.empty_like(k)
    dv = np.empty_like(v)
    for b in range(B):
        for h in range(Hkv):
            dkh[b, h], dv[b, h] = precond_backward(kh[b, h], vp[b, h], dvp[b, h], scale)
    dk = rmsnorm_backward(k, dkh, eps) + dk_attn
    return dq, dk, dv


# ---------------------------------------------------------------------------
# torch restatements: float64 autograd (to pin the closed forms above) and the
# float32 CPU baseline, which follows the reference's own op sequence.
# ---------------------------------------------------------------------------

def lucid_group_torch(q, k, v, do=None, scale=None, eps=1e-5):
    """One kv head and its G query heads in float64 torch, on whatever device the inputs are on.

    ``q [G, T, d]``, ``k, v [T, d]``, ``do [G, T, d]`` (or None).  Returns a dict with
    ``o [G, T, d]`` and ``vp [T, d]`` and, when ``do`` is given, ``dq [G, T, d]``, ``dk`` and
    ``dv [T, d]``.  The same closed forms as :func:`lucid_attention` and
    :func:`lucid_attention_grads` (modeling_lucid.py:551-574, :505-549 forward;
    :314-382 backward) written so that the T x T temporaries of one query head at a time
    are the only large allocations: this is the full-size ground truth of the GPU parity
    tests (T = 32768 needs ~40 GB of device memory in float64).
    """
    import torch

    q, k, v = q.double(), k.double(), v.double()
    G, T, d = q.shape
    scale = d ** -0.5 if scale is None else scale
    r = torch.rsqrt(k.pow(2).mean(-1, keepdim=True) + eps)
    kh = k * r
    causal = torch.ones(T, T, dtype=torch.bool, device=k.device).tril_()
    p = (kh @ kh.T).mul_(scale).sub_(1.0 / scale).masked_fill_(~causal, float("-inf")).exp_()
    vp = torch.linalg.solve_triangular(p, v, upper=False)
    out = {"vp": vp, "o": torch.empty_like(q)}
    if do is not None:
        do = do.double()
        dvp = torch.zeros_like(v)
        dk_attn = torch.zeros_like(k)
        out["dq"] = torch.empty_like(q)
    for gi in range(G):
        a = (q[gi] @ k.T).mul_(scale).masked_fill_(~causal, float("-inf"))
        a = torch.softmax(a, dim=-1)
        out["o"][gi] = a @ vp
        if do is None:
            continue
        dvp += a.T @ do[gi]
        ds = do[gi] @ vp.T
        ds -= (ds * a).sum(-1, keepdim=True)
        ds *= a
        del a
        out["dq"][gi] = scale * (ds @ k)
        dk_attn += scale * (ds.T @ q[gi])
        del ds
    if do is None:
        return out
    dv = torch.linalg.solve_triangular(p.T, dvp, upper=True)
    m = (dv @ vp.T).mul_(p)  # p is zero above the diagonal, so m is lower triangular
    del p
    dkh = -scale * (m @ kh + m.T @ kh)
    del m
    dk = r * (dkh - kh * (kh * dkh).sum(-1, keepdim=True) / d) + dk_attn
    out["dk"], out["dv"] = dk, dv
    return out


def lucid_attention_torch(q, k, v, scale=None, eps=1e-5):
    """Differentiable torch restatement of get_v_prime + eager_lucid_attention_forward.

    Op sequence as in modeling_lucid.py:561-570 (k_norm, einsum, mul, sub, masked_fill,
    exp, solve_triangular) and :520-530 (causal attention on repeat_kv'd K and V').
    Works in the dtype of its inputs (float64 for gradcheck, float32 for the CPU baseline).
    Inputs ``[B,H,T,d]``; output ``[B,T,Hq,d]``.
    """
    import torch

    d = q.shape[-1]
    scale = d ** -0.5 if scale is None else scale
    g = q.shape[1] // k.shape[1]
    t = k.shape[-2]
    kh = k * torch.rsqrt(k.pow(2).mean(-1, keepdim=True) + eps)
    s = torch.einsum("bhld,bhsd->bhls", kh, kh) * scale - 1.0 / scale
    mask = torch.ones(t, t, dtype=torch.bool).tril()
    p = torch.exp(s.masked_fill(~mask, float("-inf")))
    vp = torch.linalg.solve_triangular(p, v, upper=False)
    kr = k.repeat_interleave(g, dim=1) if g > 1 else k
    vr = vp.repeat_interleave(g, dim=1) if g > 1 else vp
    o = torch.nn.functional.scaled_dot_product_attention(q, kr, vr, is_causal=True, scale=scale)
    return o.transpose(1, 2), vp
