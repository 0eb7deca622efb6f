"""Pins the LUCID-Path oracle (oracle/path_ref.py).

The reference has no tests or golden vectors for this path, and its chunk helpers
come from an unpinned third-party package (flash-linear-attention:
chunk_scaled_dot_kkt_fwd, solve_tril), so the oracle is pinned here by the
definition itself (explicit Householder products), identities of the WY form,
special cases and float64 gradcheck.
"""
import math

import pytest
import torch

from oracle import path_ref as P

F64 = torch.float64


def _inputs(B, T, H, G, K, seed, q_is_k=False):
    g = torch.Generator().manual_seed(seed)
    k = torch.randn(B, T, H, K, generator=g, dtype=F64)
    v = torch.randn(B, T, H, K, generator=g, dtype=F64)
    w = torch.randn(B, T, H, K, generator=g, dtype=F64)
    w = w / w.norm(dim=-1, keepdim=True)
    beta = 2 * torch.sigmoid(torch.randn(B, T, H, generator=g, dtype=F64))
    q = k.clone() if q_is_k else torch.randn(B, T, H * G, K, generator=g, dtype=F64)
    return q, k, v, w, beta


def test_householder_definition():
    g = torch.Generator().manual_seed(0)
    w = torch.randn(6, generator=g, dtype=F64)
    w = w / w.norm()
    x = torch.randn(6, generator=g, dtype=F64)
    beta = torch.tensor(1.3, dtype=F64)
    h = torch.eye(6, dtype=F64) - beta * torch.outer(w, w)
    torch.testing.assert_close(P.householder_apply(x, w, beta), h @ x)


def test_wy_identity_matches_explicit_product():
    # I - W^T T_inv (beta W) == H_e ... H_s (H_s applied first to a column vector)
    g = torch.Generator().manual_seed(1)
    C, K = 8, 5
    w = torch.randn(C, K, generator=g, dtype=F64)
    w = w / w.norm(dim=-1, keepdim=True)
    b = 2 * torch.sigmoid(torch.randn(C, generator=g, dtype=F64))
    t_inv, w2 = P.wy_chunk(w, b)
    prod = torch.eye(K, dtype=F64)
    for t in range(C):
        prod = (torch.eye(K, dtype=F64) - b[t] * torch.outer(w[t], w[t])) @ prod
    torch.testing.assert_close(torch.eye(K, dtype=F64) - w.T @ w2, prod)


def test_beta_zero_reduces_to_plain_logits():
    q, k, v, w, beta = _inputs(1, 12, 1, 1, 4, 2)
    A = P.path_logits_bruteforce(q, k, w, torch.zeros_like(beta))
    ref = torch.tril(q[0, :, 0] @ k[0, :, 0].T, -1)
    torch.testing.assert_close(A[0, 0], ref)


def test_single_reflection_closed_form():
    # T = 2: A_10 = q_1^T H_1 k_0
    q, k, v, w, beta = _inputs(1, 2, 1, 1, 4, 3)
    A = P.path_logits_bruteforce(q, k, w, beta)
    h1 = torch.eye(4, dtype=F64) - beta[0, 1, 0] * torch.outer(w[0, 1, 0], w[0, 1, 0])
    torch.testing.assert_close(A[0, 0, 1, 0], q[0, 1, 0] @ h1 @ k[0, 0, 0])


@pytest.mark.parametrize("T,C,G", [(16, 4, 1), (24, 8, 2), (32, 16, 1), (64, 16, 2)])
def test_chunked_equals_bruteforce(T, C, G):
    q, k, v, w, beta = _inputs(2, T, 2, G, 8, T + C)
    scale = 8 ** -0.5
    o_bf = P.path_attention_bruteforce(q, k, v, w, beta, scale)
    o_ch = P.path_attention_chunked(q, k, v, w, beta, scale, C=C)
    torch.testing.assert_close(o_ch, o_bf, rtol=1e-10, atol=1e-10)


def test_solve_residual_unit_diagonal():
    q, k, v, w, beta = _inputs(1, 20, 1, 1, 4, 4)
    scale = 0.5
    A = P.path_logits_bruteforce(q, k, w, beta)[0, 0]
    L = torch.tril(torch.exp(A * scale - 1 / scale), -1)
    o = P.path_attention_bruteforce(q, k, v, w, beta, scale)[0, :, 0]
    torch.testing.assert_close((torch.eye(20, dtype=F64) + L) @ o, v[0, :, 0])
    # row 0 has no predecessors: O_0 = V_0
    torch.testing.assert_close(o[0], v[0, 0, 0])


def test_q_defaults_to_k():
    q, k, v, w, beta = _inputs(1, 16, 1, 1, 4, 5, q_is_k=True)
    A = P.path_logits_bruteforce(k, k, w, beta)
    assert torch.equal(A, P.path_logits_bruteforce(q, k, w, beta))


def test_kcache_decode_identity():
    # A_{T,j} for a new token equals (H_T q_T) . k_cache_j
    q, k, v, w, beta = _inputs(1, 10, 1, 1, 4, 6)
    A = P.path_logits_bruteforce(q, k, w, beta)[0, 0]
    kc = P.path_kcache_bruteforce(k[:, :9], w[:, :9], beta[:, :9])
    qT = P.householder_apply(q[0, 9, 0], w[0, 9, 0], beta[0, 9, 0])
    torch.testing.assert_close(kc[0, :, 0] @ qT, A[9, :9])


def test_gradcheck_bruteforce():
    q, k, v, w, beta = _inputs(1, 5, 1, 1, 3, 7)
    leaves = [t.clone().requires_grad_() for t in (q, k, v, w, beta)]
    assert torch.autograd.gradcheck(lambda *a: P.path_attention_bruteforce(*a, scale=0.7), leaves)


def test_chunked_grads_match_bruteforce_grads():
    q, k, v, w, beta = _inputs(1, 16, 1, 2, 4, 8)
    do = torch.randn(1, 16, 2, 4, generator=torch.Generator().manual_seed(9), dtype=F64)
    g_ch = P.path_attention_grads(q, k, v, w, beta, do, scale=0.6, C=4)
    leaves = [t.clone().requires_grad_() for t in (q, k, v, w, beta)]
    (P.path_attention_bruteforce(*leaves, scale=0.6) * do).sum().backward()
    for a, b in zip(g_ch, leaves):
        torch.testing.assert_close(a, b.grad, rtol=1e-9, atol=1e-10)


# ---- PaTH softmax attention (softmax over the same path logits, diagonal included) ----

def test_softmax_logits_diagonal_and_beta_zero():
    q, k, v, w, beta = _inputs(1, 9, 1, 2, 4, 20)
    A = P.path_softmax_logits_bruteforce(q, k, w, beta)
    for hq in range(2):
        torch.testing.assert_close(torch.diagonal(A[0, hq]), (q[0, :, hq] * k[0, :, 0]).sum(-1))
        assert torch.equal(torch.tril(A[0, hq], -1), P.path_logits_bruteforce(q, k, w, beta)[0, hq])
    A0 = P.path_softmax_logits_bruteforce(q, k, w, torch.zeros_like(beta))
    torch.testing.assert_close(A0[0, 1], torch.tril(q[0, :, 1] @ k[0, :, 0].T))


@pytest.mark.parametrize("G", [1, 2])
def test_softmax_beta_zero_is_causal_sdpa(G):
    # no reflections: plain causal softmax attention, checked against torch's SDPA (float64)
    q, k, v, w, beta = _inputs(2, 14, 2, G, 8, 21 + G)
    o = P.path_softmax_bruteforce(q, k, v, w, torch.zeros_like(beta), scale=0.3)
    kk, vv = (x.repeat_interleave(G, dim=2).transpose(1, 2) for x in (k, v))
    ref = torch.nn.functional.scaled_dot_product_attention(q.transpose(1, 2), kk, vv, is_causal=True, scale=0.3)
    torch.testing.assert_close(o, ref.transpose(1, 2), rtol=1e-12, atol=1e-12)


def test_softmax_first_row_is_v0():
    q, k, v, w, beta = _inputs(1, 6, 1, 1, 4, 23)
    o = P.path_softmax_bruteforce(q, k, v, w, beta)
    torch.testing.assert_close(o[0, 0, 0], v[0, 0, 0])


@pytest.mark.parametrize("T,C,G", [(16, 4, 1), (24, 8, 2), (32, 16, 1), (64, 16, 2)])
def test_softmax_chunked_equals_bruteforce(T, C, G):
    q, k, v, w, beta = _inputs(2, T, 2, G, 8, 30 + T + C)
    scale = 8 ** -0.5
    o_bf, lse = P.path_softmax_bruteforce(q, k, v, w, beta, scale, return_lse=True)
    o_ch, lse2 = P.path_softmax_chunked(q, k, v, w, beta, scale, C=C)
    torch.testing.assert_close(o_ch, o_bf, rtol=1e-10, atol=1e-10)
    # the reference's L_new is log2(l) + m in the exp2 domain = lse / ln 2
    torch.testing.assert_close(lse2 * math.log(2.0), lse.permute(0, 2, 1), rtol=1e-10, atol=1e-10)


def test_softmax_gradcheck_bruteforce():
    q, k, v, w, beta = _inputs(1, 5, 1, 1, 3, 24)
    leaves = [t.clone().requires_grad_() for t in (q, k, v, w, beta)]
    assert torch.autograd.gradcheck(lambda *a: P.path_softmax_bruteforce(*a, scale=0.7), leaves)
