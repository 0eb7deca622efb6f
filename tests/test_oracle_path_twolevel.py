"""The two-level decomposition implemented by the HIP kernels equals float64 autograd of the
chunked LUCID-Path restatement (itself pinned against the brute-force definition)."""
import pytest
import torch

from oracle import path_ref as P
from oracle import path_twolevel as TL

F64 = torch.float64


def _inputs(B, T, H, G, K, seed):
    g = torch.Generator().manual_seed(seed)
    k = torch.randn(B, T, H, K, generator=g, dtype=F64)
    v = torch.randn(B, T, H, K, generator=g, dtype=F64)
    w = torch.randn(B, T, H, K, generator=g, dtype=F64)
    w = w / w.norm(dim=-1, keepdim=True)
    beta = 2 * torch.sigmoid(torch.randn(B, T, H, generator=g, dtype=F64))
    q = torch.randn(B, T, H * G, K, generator=g, dtype=F64)
    do = torch.randn(B, T, H * G, K, generator=g, dtype=F64)
    return q, k, v, w, beta, do


@pytest.mark.parametrize("T,C,S,G", [(64, 4, 16, 1), (48, 8, 16, 2), (40, 4, 16, 1), (96, 8, 32, 2)])
def test_twolevel_matches_autograd(T, C, S, G):
    q, k, v, w, beta, do = _inputs(1, T, 2, G, 8, T + C + S)
    scale = 8 ** -0.5
    o, grads = TL.path_attention_twolevel(q, k, v, w, beta, do, scale=scale, C=C, S=S)
    torch.testing.assert_close(o, P.path_attention_chunked(q, k, v, w, beta, scale, C=C), rtol=1e-10, atol=1e-10)
    ref = P.path_attention_grads(q, k, v, w, beta, do, scale=scale, C=C)
    for name, a, b in zip(("dq", "dk", "dv", "dw", "dbeta"), grads, ref):
        torch.testing.assert_close(a, b, rtol=1e-8, atol=1e-9, msg=name)


@pytest.mark.parametrize("T,C,S,G", [(64, 4, 16, 1), (48, 8, 16, 2), (40, 4, 16, 1)])
def test_twolevel_softmax_matches_bruteforce_autograd(T, C, S, G):
    # PaTH softmax attention: same decomposition, dA from the softmax backward
    q, k, v, w, beta, do = _inputs(1, T, 2, G, 8, 100 + T + C + S)
    scale = 8 ** -0.5
    o, grads = TL.path_attention_twolevel(q, k, v, w, beta, do, scale=scale, C=C, S=S, softmax=True)
    torch.testing.assert_close(o, P.path_softmax_bruteforce(q, k, v, w, beta, scale), rtol=1e-10, atol=1e-10)
    ref = P.path_softmax_grads(q, k, v, w, beta, do, scale=scale)
    for name, a, b in zip(("dq", "dk", "dv", "dw", "dbeta"), grads, ref):
        torch.testing.assert_close(a, b, rtol=1e-8, atol=1e-9, msg=name)
