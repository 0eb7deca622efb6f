"""LUCID-Path (and PaTH softmax attention) for one query head, vectorised over chunks, float64,
on whatever device the inputs are on -- test infrastructure only (see oracle/__init__.py).

This is the full-size ground truth of the GPU parity tests: the per-chunk Python loops of
``path_ref.path_attention_chunked`` and ``path_twolevel.forward`` visit every pair of 64-row
chunks (131 k pairs per head at T = 32768), while this restatement builds the dense T x T
logits in a few dozen batched products, solves densely, and takes its gradients from torch
autograd.  Memory is O(T^2) per head (~9 GB at T = 32768 in float64 per T x T temporary).

Algebra (reference parallel.py:27-177 and triangular_solve_fwd.py:99-225, in the two-level form
of ``path_twolevel``; row vectors are right-multiplied when carried down through a chunk):
  per small chunk c (C rows):  T_inv = (I + stril(diag(beta) W W^T))^-1,  W2 = T_inv (beta W),
    Hc_c = I - W^T W2,  q~ = Q - tril(Q W^T) W2,  k~ = K - (T_inv stril(beta W K^T))^T W,
    A_cc = tril(Q K^T - tril(Q W^T) T_inv stril(beta W K^T))                 (in-chunk logits)
  same large chunk (S rows), J < I:  A_IJ = q~_I Hc_{I-1} ... Hc_{J+1} k~_J^T
  earlier large chunk s:             A_IJ = q~_I PRE_I HL_{sI-1} ... HL_{s+1} KL_J^T,
    PRE_I = Hc_{I-1} ... Hc_{c0(I)},  HL_s = Hc_{top} ... Hc_{bottom} of s,  KL_J = k~_J SUF_J^T,
    SUF_J = Hc_{top} ... Hc_{J+1} (inside J's large chunk)
  LUCID-Path:  O = (I + tril(exp(s A - 1/s), -1))^-1 V
  PaTH softmax:  O = softmax_{j <= i}(s A_ij) V   (diagonal included)

Pinning: tests/test_oracle_path_dense.py checks it against ``path_ref.path_attention_chunked``
(itself pinned against the brute-force definition) and the float64 autograd gradients of that
restatement, against ``path_ref.path_softmax_bruteforce`` for the softmax mode, at sizes that
span several large chunks with a partial last one.
"""
from __future__ import annotations

import torch


def path_logits_dense(q, k, w, beta, C=64, S=512):
    """Dense path logits A [T, T] (entries j <= i are the logits; entries above the diagonal
    hold finite values that callers mask) for one head: q, k, w [T, K], beta [T]."""
    T, K = k.shape
    if T % C or S % C:
        raise ValueError("T and S must be multiples of C")
    dt, dev = k.dtype, k.device
    NT, R = T // C, S // C
    NS = (NT + R - 1) // R
    eye_c = torch.eye(C, dtype=dt, device=dev)
    eye_k = torch.eye(K, dtype=dt, device=dev)
    W, b = w.reshape(NT, C, K), beta.reshape(NT, C)
    Q, Kc = q.reshape(NT, C, K), k.reshape(NT, C, K)
    Wb = W * b[..., None]
    a = torch.tril(Wb @ W.transpose(1, 2), -1)
    tm = torch.linalg.solve_triangular(eye_c + a, eye_c.expand(NT, C, C), upper=False, unitriangular=True)
    w2 = tm @ Wb
    hc = eye_k - W.transpose(1, 2) @ w2                      # [NT, K, K]
    qw = torch.tril(Q @ W.transpose(1, 2))
    wbk = torch.tril(Wb @ Kc.transpose(1, 2), -1)
    tw = tm @ wbk
    qt = Q - qw @ w2
    kt = Kc - tw.transpose(1, 2) @ W
    adiag = torch.tril(Q @ Kc.transpose(1, 2) - qw @ tw)    # [NT, C, C]
    # chunks padded to NS * R with identity transitions (and zero rows) past the end
    pad = NS * R - NT
    if pad:
        hc = torch.cat([hc, eye_k.expand(pad, K, K)], 0)
        qt = torch.cat([qt, qt.new_zeros(pad, C, K)], 0)
        kt = torch.cat([kt, kt.new_zeros(pad, C, K)], 0)
        adiag = torch.cat([adiag, adiag.new_zeros(pad, C, C)], 0)
    hp, qtp, ktp = hc.reshape(NS, R, K, K), qt.reshape(NS, R, C, K), kt.reshape(NS, R, C, K)
    # SUF (top-down) and PRE (bottom-up) inside each large chunk; HL the whole product
    suf = [None] * R
    suf[R - 1] = eye_k.expand(NS, K, K)
    for r in range(R - 2, -1, -1):
        suf[r] = suf[r + 1] @ hp[:, r + 1]
    pre = [eye_k.expand(NS, K, K)]
    for r in range(1, R):
        pre.append(hp[:, r - 1] @ pre[r - 1])
    SUF, PRE = torch.stack(suf, 1), torch.stack(pre, 1)    # [NS, R, K, K]
    HL = SUF[:, 0] @ hp[:, 0]                                # [NS, K, K]
    KL = ktp @ SUF.transpose(-1, -2)                         # [NS, R, C, K]
    # same large chunk: X[d][s, rI] = q~_I Hc_{I-1} ... Hc_{I-d}; block (rI, rJ) uses d = rI-1-rJ
    ridx = torch.arange(R, device=dev)
    X = [qtp]
    for d in range(1, R):
        X.append(X[-1] @ hp[:, (ridx - d).clamp(min=0)])
    Xs = torch.stack(X, 2)                                   # [NS, R(rI), R(d), C, K]
    didx = (ridx[:, None] - 1 - ridx[None, :]).clamp(min=0)  # [rI, rJ]
    Xg = Xs[:, ridx[:, None], didx]                          # [NS, R, R, C, K]
    win = Xg @ ktp[:, None].transpose(-1, -2)                # [NS, rI, rJ, C, C]
    diag = torch.eye(R, dtype=torch.bool, device=dev)[None, :, :, None, None]
    win = torch.where(diag, adiag.reshape(NS, R, 1, C, C), win)
    win = win.permute(0, 1, 3, 2, 4).reshape(NS, S, S)       # rows (rI, c), cols (rJ, d)
    # earlier large chunks, key chunk s descending: x carries each query down to s's top
    x = (qtp @ PRE).reshape(NS, S, K)                        # q~_I PRE_I
    srow = torch.arange(NS, device=dev)
    cols = []
    for s in range(NS - 1, -1, -1):
        cross = (x @ KL[s].reshape(S, K).T)                  # [NS, S, S]
        blk = torch.where((srow > s)[:, None, None], cross, torch.zeros((), dtype=dt, device=dev))
        blk = torch.where((srow == s)[:, None, None], win[s].expand(NS, S, S), blk)
        cols.append(blk)
        if s > 0:
            x = torch.where((srow > s)[:, None, None], x @ HL[s], x)
    A = torch.cat(cols[::-1], 2).reshape(NS * S, NS * S)
    return A[:T, :T]


def path_head_dense(q, k, v, w, beta, scale=None, C=64, S=512, softmax=False):
    """O [T, V] of one query head (q [T, K]) over its kv head's k, v, w [T, *], beta [T]:
    LUCID-Path ``(I + L)^-1 V`` or (``softmax``) PaTH softmax attention.  Differentiable."""
    T, K = k.shape
    scale = K ** -0.5 if scale is None else scale
    A = path_logits_dense(q, k, w, beta, C, S)
    if softmax:
        ninf = torch.full((T, T), float("-inf"), dtype=A.dtype, device=A.device).triu_(1)
        p = torch.softmax(A * scale + ninf, dim=-1)
        return p @ v
    L = torch.tril(torch.exp(A * scale - 1.0 / scale), -1)
    return torch.linalg.solve_triangular(L, v, upper=False, unitriangular=True)


def path_attention_dense(q, k, v, w, beta, do=None, scale=None, C=64, S=512, softmax=False, heads=None):
    """[B, T, H*, K] inputs (any device), one query head at a time; returns O [B, T, HQ, V] and,
    with ``do``, the gradients (dq, dk, dv, dw, dbeta) with the GQA sums applied (float64 autograd).
    ``heads``: the query heads to evaluate (default all); the others' outputs and gradient
    contributions are left zero."""
    B, T, HQ, K = q.shape
    H = k.shape[2]
    G = HQ // H
    q, k, v, w, beta = (x.double() for x in (q, k, v, w, beta))
    o = torch.zeros(B, T, HQ, v.shape[-1], dtype=torch.float64, device=q.device)
    grads = None
    if do is not None:
        do = do.double()
        grads = [torch.zeros_like(x) for x in (q, k, v, w, beta)]
    for b in range(B):
        for hq in (range(HQ) if heads is None else heads):
            h = hq // G
            leaves = [x.detach().clone().requires_grad_(do is not None)
                      for x in (q[b, :, hq], k[b, :, h], v[b, :, h], w[b, :, h], beta[b, :, h])]
            ob = path_head_dense(*leaves, scale=scale, C=C, S=S, softmax=softmax)
            o[b, :, hq] = ob.detach()
            if do is not None:
                g = torch.autograd.grad(ob, leaves, do[b, :, hq])
                grads[0][b, :, hq] += g[0]
                for i in range(1, 5):
                    grads[i][b, :, h] += g[i]
            del ob, leaves
    return o if do is None else (o, tuple(grads))
