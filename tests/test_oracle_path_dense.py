"""Pins oracle/path_dense.py (the vectorised full-size ground truth of the LUCID-Path and PaTH
softmax GPU tests) against the chunked restatement (pinned against the brute-force definition in
test_oracle_path.py) and its float64 autograd gradients, and against the softmax brute force.
Sizes span several large chunks with a partial last one (T not a multiple of S)."""
import pytest
import torch

from oracle import path_dense as PD
from oracle import path_ref as P


def _inputs(B, T, H, G, seed, K=16):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, T, H * G, K, generator=g, dtype=torch.float64)
    k = torch.randn(B, T, H, K, generator=g, dtype=torch.float64)
    v = torch.randn(B, T, H, K, generator=g, dtype=torch.float64)
    w = torch.randn(B, T, H, K, generator=g, dtype=torch.float64)
    w = w / w.norm(dim=-1, keepdim=True)
    beta = 2 * torch.sigmoid(torch.randn(B, T, H, generator=g, dtype=torch.float64))
    do = torch.randn(B, T, H * G, K, generator=g, dtype=torch.float64)
    return q, k, v, w, beta, do


@pytest.mark.parametrize("T,C,S", [(80, 8, 32), (96, 16, 32), (40, 8, 8), (64, 8, 64)])
def test_dense_path_equals_chunked_forward_and_gradients(T, C, S):
    q, k, v, w, beta, do = _inputs(1, T, 2, 2, seed=T + C + S)
    scale = 0.4
    ref = P.path_attention_chunked(q, k, v, w, beta, scale=scale, C=C)
    o, grads = PD.path_attention_dense(q, k, v, w, beta, do=do, scale=scale, C=C, S=S)
    assert torch.allclose(o, ref, rtol=1e-10, atol=1e-10)
    gref = P.path_attention_grads(q, k, v, w, beta, do, scale=scale, C=C)
    for name, a, b in zip(("dq", "dk", "dv", "dw", "dbeta"), grads, gref):
        assert torch.allclose(a, b, rtol=1e-9, atol=1e-9), name


def test_dense_path_logits_equal_bruteforce():
    q, k, v, w, beta, _ = _inputs(1, 48, 1, 1, seed=3, K=8)
    A = PD.path_logits_dense(q[0, :, 0], k[0, :, 0], w[0, :, 0], beta[0, :, 0], C=8, S=16)
    ref = P.path_logits_bruteforce(q, k, w, beta)[0, 0]
    mask = torch.ones(48, 48, dtype=torch.bool).tril(-1)
    assert torch.allclose(A[mask], ref[mask], rtol=1e-10, atol=1e-10)
    # the in-chunk diagonal is q_i . k_i (no transport)
    assert torch.allclose(A.diagonal(), (q[0, :, 0] * k[0, :, 0]).sum(-1), rtol=1e-12, atol=1e-12)


def test_dense_softmax_equals_bruteforce():
    q, k, v, w, beta, do = _inputs(1, 48, 1, 2, seed=5, K=8)
    ref = P.path_softmax_bruteforce(q, k, v, w, beta, scale=0.5)
    o, grads = PD.path_attention_dense(q, k, v, w, beta, do=do, scale=0.5, C=8, S=16, softmax=True)
    assert torch.allclose(o, ref, rtol=1e-10, atol=1e-10)
    gref = P.path_softmax_grads(q, k, v, w, beta, do, scale=0.5)
    for name, a, b in zip(("dq", "dk", "dv", "dw", "dbeta"), grads, gref):
        assert torch.allclose(a, b, rtol=1e-9, atol=1e-9), name


def test_dense_heads_subset_leaves_other_heads_zero():
    q, k, v, w, beta, do = _inputs(1, 32, 1, 2, seed=9, K=8)
    o, grads = PD.path_attention_dense(q, k, v, w, beta, do=do, scale=0.5, C=8, S=16, heads=[1])
    assert torch.count_nonzero(o[:, :, 0]) == 0 and torch.count_nonzero(grads[0][:, :, 0]) == 0
    full, _ = PD.path_attention_dense(q, k, v, w, beta, do=do, scale=0.5, C=8, S=16)
    assert torch.equal(o[:, :, 1], full[:, :, 1])
