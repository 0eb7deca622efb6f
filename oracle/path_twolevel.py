"""Two-level (small chunk C, large chunk S) LUCID-Path algorithm, float64, one head at a time.

Test infrastructure only (see oracle/__init__.py).  This is the decomposition the
HIP kernels in lucid_amd/csrc/path_*.hip implement, written out with explicit
forward and backward so that every intermediate the kernels produce can be
checked, and so that the decomposition itself is pinned against float64 autograd
of ``path_ref.path_attention_chunked`` (tests/test_oracle_path_twolevel.py).

Notation (rows are time positions; every transport is a right-multiplication of
row vectors by d x d matrices):
  Hc_c  = I - W_c^T W2_c                 product of the Householders of small chunk c
  HL_s  = Hc_{top} ... Hc_{bottom}        product over large chunk s
  SUF_c = Hc_{top} ... Hc_{c+1},  PRE_c = Hc_{c-1} ... Hc_{bottom}   (inside c's large chunk)
  KL_j  = k~_j SUF_c^T                   key carried to the top of its large chunk
  QS_I^(c) = q~_I Hc_{I-1} ... Hc_{c+1}  query carried down to the top of chunk c (same large chunk)
  QB_I^(s) = q~_I PRE_I HL_{sI-1} ... HL_{s+1}   query carried down to the top of large chunk s
  A_IJ = QB_I^(sJ) KL_J^T if sJ < sI else QS_I^(J) k~_J^T   (every inter-chunk pair is one GEMM)
Reference: parallel.py:27-177 (stage order), cumprod_householder_fwd.py:13-79,
transform_q.py:15-61, triangular_solve_fwd.py:99-225, intra_chunk_preprocess_bwd.py:14-110.
"""
from __future__ import annotations

import torch


def _ltri_inv_unit(a):
    c = a.shape[0]
    eye = torch.eye(c, dtype=a.dtype)
    return torch.linalg.solve_triangular(eye + a, eye, upper=False, unitriangular=True)


def chunk_prep(q, k, w, beta, scale, C):
    """Per small chunk: T_inv, W2, Hc, q~, k~, A_diag and Y = (I + stril exp(s A_diag - 1/s))^-1."""
    T, d = k.shape
    out = []
    for c in range(T // C):
        sl = slice(c * C, (c + 1) * C)
        W, b, qc, kc = w[sl], beta[sl], q[sl], k[sl]
        Wb = W * b[:, None]
        tm = _ltri_inv_unit(torch.tril(Wb @ W.T, -1))
        w2 = tm @ Wb
        qw = torch.tril(qc @ W.T)
        wbk = torch.tril(Wb @ kc.T, -1)
        tw = tm @ wbk
        adiag = torch.tril(qc @ kc.T - qw @ tw)
        ld = torch.tril(torch.exp(adiag * scale - 1.0 / scale), -1)
        out.append(dict(W=W, b=b, Wb=Wb, tm=tm, w2=w2, Hc=torch.eye(d, dtype=k.dtype) - W.T @ w2,
                        qw=qw, wbk=wbk, tw=tw, qt=qc - qw @ w2, kt=kc - tw.T @ W, ld=ld, adiag=adiag,
                        Y=_ltri_inv_unit(ld)))
    return out


def large_prep(ch, R):
    """Per large chunk (R small chunks): SUF, PRE, HL and the carried keys KL."""
    NT = len(ch)
    d = ch[0]["Hc"].shape[0]
    eye = torch.eye(d, dtype=ch[0]["Hc"].dtype)
    SUF, PRE, HL, KL = [None] * NT, [None] * NT, [], [None] * NT
    for s in range((NT + R - 1) // R):
        c0, c1 = s * R, min(s * R + R, NT) - 1
        SUF[c1] = eye
        for c in range(c1 - 1, c0 - 1, -1):
            SUF[c] = SUF[c + 1] @ ch[c + 1]["Hc"]
        PRE[c0] = eye
        for c in range(c0 + 1, c1 + 1):
            PRE[c] = ch[c - 1]["Hc"] @ PRE[c - 1]
        HL.append(SUF[c0] @ ch[c0]["Hc"])
        for c in range(c0, c1 + 1):
            KL[c] = ch[c]["kt"] @ SUF[c].T
    return SUF, PRE, HL, KL


def query_transport(ch, HL, R):
    """QS[I][c] (c in I's large chunk, c < I) and QB[I][s] (s < I's large chunk)."""
    NT = len(ch)
    QS, QB = [dict() for _ in range(NT)], [dict() for _ in range(NT)]
    for I in range(NT):
        sI, c0 = I // R, (I // R) * R
        x = ch[I]["qt"]
        for c in range(I - 1, c0 - 1, -1):
            QS[I][c] = x
            x = x @ ch[c]["Hc"]
        for s in range(sI - 1, -1, -1):
            QB[I][s] = x
            x = x @ HL[s]
    return QS, QB


def forward(q, k, v, w, beta, scale, C=64, S=512, softmax=False):
    """O for one query head (kv tensors of its kv head); returns (O, state for backward).

    ``softmax=False``: LUCID-Path, the chained solve (I + L) O = V.
    ``softmax=True``: PaTH softmax attention over the same logits, diagonal included:
    O_I = sum_{J<=I} P_IJ V_J with P = exp(s A - lse) (row-wise log-sum-exp).
    """
    T = k.shape[0]
    R = S // C
    NT = T // C
    ch = chunk_prep(q, k, w, beta, scale, C)
    SUF, PRE, HL, KL = large_prep(ch, R)
    QS, QB = query_transport(ch, HL, R)

    def logits(I, J):
        if J // R < I // R:
            return QB[I][J // R] @ KL[J].T
        return QS[I][J] @ ch[J]["kt"].T

    L = {}
    O = []
    st = dict(ch=ch, SUF=SUF, PRE=PRE, HL=HL, KL=KL, QS=QS, QB=QB, L=L, O=O, R=R, C=C, scale=scale,
              softmax=softmax)
    if softmax:
        mask = torch.ones(C, C, dtype=torch.bool).tril()
        Vb = [v[J * C:(J + 1) * C] for J in range(NT)]
        Pd, lse = [], []
        for I in range(NT):
            blocks = [logits(I, J) * scale for J in range(I)]
            blocks.append((ch[I]["adiag"] * scale).masked_fill(~mask, float("-inf")))
            full = torch.cat(blocks, 1)
            ls = torch.logsumexp(full, dim=-1)
            for J in range(I):
                L[(I, J)] = torch.exp(blocks[J] - ls[:, None])
            Pd.append(torch.exp(blocks[I] - ls[:, None]))
            O.append(sum(L[(I, J)] @ Vb[J] for J in range(I)) + Pd[I] @ Vb[I])
            lse.append(ls)
        st.update(Pd=Pd, V=Vb, lse=torch.cat(lse))
        return torch.cat(O, 0), st
    for I in range(NT):
        r = v[I * C:(I + 1) * C].clone()
        for J in range(I):
            L[(I, J)] = torch.exp(logits(I, J) * scale - 1.0 / scale)
            r -= L[(I, J)] @ O[J]
        O.append(ch[I]["Y"] @ r)
    return torch.cat(O, 0), st


def backward(st, do):
    """(dq, dk, dv, dw, dbeta) for one query head from the two-level state."""
    ch, SUF, HL, KL, QS, QB, L, O = (st[x] for x in ("ch", "SUF", "HL", "KL", "QS", "QB", "L", "O"))
    R, C, scale = st["R"], st["C"], st["scale"]
    NT = len(ch)
    d = ch[0]["Hc"].shape[0]
    z = lambda *s: torch.zeros(*s, dtype=do.dtype)  # noqa: E731
    if st["softmax"]:
        # ---- softmax: dP = dO V^T, dA = s P (dP - delta), dV_J = sum_{I>=J} P_IJ^T dO_I ----
        Vb, Pd = st["V"], st["Pd"]
        dOb = [do[I * C:(I + 1) * C] for I in range(NT)]
        delta = [(dOb[I] * O[I]).sum(-1, keepdim=True) for I in range(NT)]
        dA = {(I, J): scale * L[(I, J)] * (dOb[I] @ Vb[J].T - delta[I]) for (I, J) in L}
        dAd = [scale * Pd[c] * (dOb[c] @ Vb[c].T - delta[c]) for c in range(NT)]
        dV = [Pd[J].T @ dOb[J] + sum((L[(I, J)].T @ dOb[I] for I in range(J + 1, NT)), z(C, d))
              for J in range(NT)]
        return _logit_backward(st, dA, dAd, dV, z)
    # ---- dV = (I + L)^-T dO, last block first ----
    dV = [None] * NT
    for J in range(NT - 1, -1, -1):
        r = do[J * C:(J + 1) * C].clone()
        for I in range(J + 1, NT):
            r -= L[(I, J)].T @ dV[I]
        dV[J] = ch[J]["Y"].T @ r
    dA = {(I, J): -scale * (dV[I] @ O[J].T) * L[(I, J)] for (I, J) in L}
    dAd = [-scale * (dV[c] @ O[c].T) * ch[c]["ld"] for c in range(NT)]
    return _logit_backward(st, dA, dAd, dV, z)


def _logit_backward(st, dA, dAd, dV, z):
    """Gradients of the inputs given dA (inter-chunk blocks), dAd (in-chunk, lower incl. the
    diagonal) and dV: the row sweep, the column sweep, the products and the WY backward."""
    ch, SUF, HL, KL, QS, QB = (st[x] for x in ("ch", "SUF", "HL", "KL", "QS", "QB"))
    R, C = st["R"], st["C"]
    NT = len(ch)
    d = ch[0]["Hc"].shape[0]
    # ---- row sweep: gradient of the query transports ----
    dHL = [z(d, d) for _ in HL]
    dHc = [z(d, d) for _ in range(NT)]
    dqt = [None] * NT
    for I in range(NT):
        sI, c0 = I // R, (I // R) * R
        G = z(C, d)
        for s in range(sI):
            if s > 0:
                dHL[s] += QB[I][s].T @ G
                G = G @ HL[s].T
            for J in range(s * R, s * R + R):
                G += dA[(I, J)] @ KL[J]
        for c in range(c0, I):
            if sI > 0 or c > c0:
                dHc[c] += QS[I][c].T @ G
                G = G @ ch[c]["Hc"].T
            G += dA[(I, c)] @ ch[c]["kt"]
        dqt[I] = G
    # ---- column sweep: gradient of the carried keys ----
    dkt = [z(C, d) for _ in range(NT)]
    dSUF = [z(d, d) for _ in range(NT)]
    for J in range(NT):
        sJ = J // R
        dKL = z(C, d)
        for I in range(J + 1, NT):
            if I // R > sJ:
                dKL += dA[(I, J)].T @ QB[I][sJ]
            else:
                dkt[J] += dA[(I, J)].T @ QS[I][J]
        dkt[J] += dKL @ SUF[J]
        dSUF[J] += dKL.T @ ch[J]["kt"]
    # ---- products backward inside each large chunk ----
    for s in range(len(HL)):
        c0, c1 = s * R, min(s * R + R, NT) - 1
        F = dHL[s].clone()
        for c in range(c0, c1 + 1):
            dHc[c] += SUF[c].T @ F
            F = F @ ch[c]["Hc"].T + dSUF[c]
    # ---- WY backward per chunk ----
    dq, dk, dw, db = [], [], [], []
    for c in range(NT):
        x = ch[c]
        W, Wb, tm, w2, qw, wbk, tw = x["W"], x["Wb"], x["tm"], x["w2"], x["qw"], x["wbk"], x["tw"]
        sl = slice(c * C, (c + 1) * C)
        dW = -w2 @ dHc[c].T
        dW2 = -W @ dHc[c]
        # q~ = q - QW W2
        dqc = dqt[c].clone()
        dQW = -dqt[c] @ w2.T
        dW2 = dW2 - qw.T @ dqt[c]
        # k~ = k - TW^T W
        dkc = dkt[c].clone()
        dTW = -W @ dkt[c].T
        dW = dW - tw @ dkt[c]
        # A_diag (lower part incl. the diagonal; LUCID-Path's dAd vanishes on the diagonal)
        qrows, krows = st_rows(st, c)
        dqc += dAd[c] @ krows
        dkc += dAd[c].T @ qrows
        dQW = dQW - dAd[c] @ tw.T
        dTW = dTW - qw.T @ dAd[c]
        # QW = tril(q W^T)
        dQW = torch.tril(dQW)
        dqc += dQW @ W
        dW = dW + dQW.T @ qrows
        # TW = Tm WBK
        dTm = dTW @ wbk.T
        dWBK = torch.tril(tm.T @ dTW, -1)
        dWb = dWBK @ krows
        dkc += dWBK.T @ Wb
        # W2 = Tm Wb
        dTm = dTm + dW2 @ Wb.T
        dWb = dWb + tm.T @ dW2
        # Tm = (I + a)^-1, a = stril(Wb W^T)
        da = torch.tril(-tm.T @ dTm @ tm.T, -1)
        dWb = dWb + da @ W
        dW = dW + da.T @ Wb
        # Wb = diag(beta) W
        dW = dW + x["b"][:, None] * dWb
        db.append((dWb * W).sum(-1))
        dq.append(dqc)
        dk.append(dkc)
        dw.append(dW)
    return (torch.cat(dq), torch.cat(dk), torch.cat(dV), torch.cat(dw), torch.cat(db))


def st_rows(st, c):
    C = st["C"]
    return st["q"][c * C:(c + 1) * C], st["k"][c * C:(c + 1) * C]


def path_attention_twolevel(q, k, v, w, beta, do=None, scale=None, C=64, S=512, softmax=False):
    """Forward (and backward if ``do`` is given) over [B,T,H*,K] tensors, looping over heads.

    Returns O [B,T,HQ,V] and, with ``do``, (dq, dk, dv, dw, dbeta) with the GQA sums applied.
    """
    B, T, HQ, K = q.shape
    H = k.shape[2]
    G = HQ // H
    scale = K ** -0.5 if scale is None else scale
    o = torch.zeros(B, T, HQ, v.shape[-1], dtype=q.dtype)
    grads = None
    if do is not None:
        grads = [torch.zeros_like(q), torch.zeros_like(k), torch.zeros_like(v), torch.zeros_like(w),
                 torch.zeros_like(beta)]
    for b in range(B):
        for hq in range(HQ):
            h = hq // G
            ob, st = forward(q[b, :, hq], k[b, :, h], v[b, :, h], w[b, :, h], beta[b, :, h], scale, C, S, softmax)
            o[b, :, hq] = ob
            if do is not None:
                st["q"], st["k"] = q[b, :, hq], k[b, :, h]
                dq, dk, dv, dw, db = backward(st, do[b, :, hq])
                grads[0][b, :, hq] += dq
                grads[1][b, :, h] += dk
                grads[2][b, :, h] += dv
                grads[3][b, :, h] += dw
                grads[4][b, :, h] += db
    return o if do is None else (o, tuple(grads))
