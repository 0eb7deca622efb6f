"""GPU parity of LUCID-Path and PaTH softmax attention at head dims 16 and 32.

The reference entry point takes head dims 16, 32, 64 and 128 for q/k/w and for v
independently (lucid_path/triton_code/parallel.py:230-232).  Here 16 and 32 run on rows
zero-padded to the kernels' 64; the float64 oracle computes at the true dims and the
default scale 1/sqrt(K) of the true K, so a padded coordinate leaking into the logits, the
scale, an output or a gradient would show.  Bars: tests/bars.py (bf16 against float64 on
the same bf16-rounded inputs).
"""
import pytest
import torch

from bars import check
from oracle import path_ref as P

pytestmark = pytest.mark.gpu


def _inputs(B, T, H, G, K, V, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, T, H * G, K, generator=g)
    k = torch.randn(B, T, H, K, generator=g)
    v = torch.randn(B, T, H, V, generator=g)
    w = torch.randn(B, T, H, K, generator=g)
    w = w / w.norm(dim=-1, keepdim=True)
    beta = 2 * torch.sigmoid(torch.randn(B, T, H, generator=g))
    do = torch.randn(B, T, H * G, V, generator=g)
    return [x.to(torch.bfloat16) for x in (q, k, v, w, beta, do)]


def _f64(x):
    return x.detach().cpu().double()


def _pad_t(x, Tp):
    return torch.nn.functional.pad(_f64(x), [0, 0] * (x.dim() - 2) + [0, Tp - x.shape[1]])


@pytest.mark.parametrize("B,T,H,G,K,V", [(1, 256, 2, 1, 32, 32), (1, 200, 1, 2, 16, 16), (2, 192, 1, 1, 32, 64),
                                         (1, 128, 1, 1, 64, 16)])
def test_lucid_path_small_head_dims(B, T, H, G, K, V):
    from lucid_amd.lucid_path import parallel_lucid_path_attention
    q, k, v, w, beta, do = _inputs(B, T, H, G, K, V, seed=T + K + V)
    print(f"case path head dims B={B} T={T} H={H} G={G} K={K} V={V}", flush=True)
    leaves = [x.cuda().requires_grad_() for x in (q, k, v, w, beta)]
    o, kc = parallel_lucid_path_attention(leaves[1], leaves[2], leaves[3], leaves[4], q=leaves[0], use_cache=True)
    assert o.shape == (B, T, H * G, V) and kc.shape == (B, T, H, K)
    o.backward(do.cuda())
    torch.cuda.synchronize()
    Tp = (T + 63) // 64 * 64
    s = K ** -0.5
    ref = P.path_attention_chunked(*(_pad_t(x, Tp) for x in (q, k, v, w, beta)), scale=s, C=64)[:, :T]
    err = (o.detach().cpu().double() - ref).abs().max().item()
    print(f"  o: max err {err:.2e} max|ref| {ref.abs().max().item():.2e}", flush=True)
    check("o", err, ref.abs().max().item())
    if T <= 256:
        kc_ref = P.path_kcache_bruteforce(_f64(k), _f64(w), _f64(beta))
        check("k_cache", (kc.cpu().double() - kc_ref).abs().max().item(), kc_ref.abs().max().item())
    grads = P.path_attention_grads(*(_pad_t(x, Tp) for x in (q, k, v, w, beta)), _pad_t(do, Tp), scale=s, C=64)
    for name, got, r in zip(("dq", "dk", "dv", "dw", "dbeta"), leaves, grads):
        r = r[:, :T]
        assert got.grad.shape == r.shape, name
        err = (got.grad.cpu().double() - r).abs().max().item()
        print(f"  {name}: max err {err:.2e} max|ref| {r.abs().max().item():.2e}", flush=True)
        check(name, err, r.abs().max().item())


@pytest.mark.parametrize("B,T,H,G,K,V", [(1, 192, 1, 2, 32, 32), (1, 128, 2, 1, 16, 32)])
def test_path_softmax_small_head_dims(B, T, H, G, K, V):
    from lucid_amd.lucid_path import parallel_path_attention
    q, k, v, w, beta, do = _inputs(B, T, H, G, K, V, seed=7 * T + K + V)
    print(f"case path softmax head dims B={B} T={T} H={H} G={G} K={K} V={V}", flush=True)
    leaves = [x.cuda().requires_grad_() for x in (q, k, v, w, beta)]
    o, _ = parallel_path_attention(*leaves)
    assert o.shape == (B, T, H * G, V)
    o.backward(do.cuda())
    torch.cuda.synchronize()
    s = K ** -0.5
    ref = P.path_softmax_bruteforce(*(_f64(x) for x in (q, k, v, w, beta)), scale=s)
    err = (o.detach().cpu().double() - ref).abs().max().item()
    print(f"  o: max err {err:.2e} max|ref| {ref.abs().max().item():.2e}", flush=True)
    check("o", err, ref.abs().max().item())
    grads = P.path_softmax_grads(*(_f64(x) for x in (q, k, v, w, beta)), _f64(do), scale=s)
    for name, got, r in zip(("dq", "dk", "dv", "dw", "dbeta"), leaves, grads):
        err = (got.grad.cpu().double() - r).abs().max().item()
        print(f"  {name}: max err {err:.2e} max|ref| {r.abs().max().item():.2e}", flush=True)
        check(name, err, r.abs().max().item())


def test_lucid_path_rejects_unsupported_head_dim():
    """A head dim outside the reference's [16, 32, 64, 128] fails its assert."""
    from lucid_amd.lucid_path import parallel_lucid_path_attention
    q, k, v, w, beta, _ = _inputs(1, 64, 1, 1, 48, 48, seed=1)
    with pytest.raises(AssertionError, match="only support head_dim"):
        parallel_lucid_path_attention(k.cuda(), v.cuda(), w.cuda(), beta.cuda(), q=q.cuda())
