"""GPU parity of PaTH softmax attention (lucid_amd.lucid_path.parallel_path_attention)
against the float64 CPU oracle.

Inputs as BASELINE config 4 (q, k, v, w ~ N(0,1), w L2-normalised, beta = 2 sigmoid(N(0,1)),
scale 1/sqrt(64)).  Forward reference: ``path_ref.path_softmax_chunked`` (the chunk algebra
of the reference's two forward kernels, pinned against the brute-force definition);
gradients: ``path_twolevel`` in softmax mode (pinned against float64 autograd of the brute
force).  Tolerance (bf16 against float64 on the same bf16-rounded inputs): max |x - ref|
<= 2e-2 for outputs, 2e-2 * max(1, max |ref|) for gradients.
"""
import pytest
import torch

from oracle import path_ref as P
from oracle import path_twolevel as TL

from bars import check  # noqa: E402

pytestmark = pytest.mark.gpu

TOL = 2e-2


def _inputs(B, T, H, G, seed, K=64, beta_zero=False):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, T, H * G, K, generator=g)
    k = torch.randn(B, T, H, K, generator=g)
    v = torch.randn(B, T, H, K, generator=g)
    w = torch.randn(B, T, H, K, generator=g)
    w = w / w.norm(dim=-1, keepdim=True)
    beta = 2 * torch.sigmoid(torch.randn(B, T, H, generator=g))
    if beta_zero:
        beta = torch.zeros_like(beta)
    do = torch.randn(B, T, H * G, K, generator=g)
    return [x.to(torch.bfloat16) for x in (q, k, v, w, beta, do)]


def _f64(x):
    return x.detach().cpu().double()


def _padded(x, Tp):
    return torch.nn.functional.pad(_f64(x), [0, 0] * (x.dim() - 2) + [0, Tp - x.shape[1]])


@pytest.mark.parametrize("B,T,H,G", [(1, 256, 2, 1), (1, 1024, 1, 2), (2, 640, 1, 1), (1, 200, 1, 1),
                                     (1, 576, 1, 1)])
def test_path_softmax_forward_matches_oracle(B, T, H, G):
    from lucid_amd.lucid_path import parallel_path_attention
    q, k, v, w, beta, _ = _inputs(B, T, H, G, seed=40 + T + G)
    print(f"case path softmax fwd B={B} T={T} H={H} G={G}", flush=True)
    o, kc = parallel_path_attention(q.cuda(), k.cuda(), v.cuda(), w.cuda(), beta.cuda())
    torch.cuda.synchronize()
    assert kc is None
    Tp = (T + 63) // 64 * 64
    ref, _ = P.path_softmax_chunked(*(_padded(x, Tp) for x in (q, k, v, w, beta)), scale=0.125, C=64)
    err = (o.cpu().double() - ref[:, :T]).abs().max().item()
    assert err <= TOL, f"max err {err:.3e}"


@pytest.mark.parametrize("B,T,H,G", [(1, 256, 1, 1), (1, 1024, 1, 2), (1, 576, 2, 1), (1, 200, 1, 1)])
def test_path_softmax_backward_matches_oracle(B, T, H, G):
    from lucid_amd.lucid_path import parallel_path_attention
    q, k, v, w, beta, do = _inputs(B, T, H, G, seed=50 + T + G)
    print(f"case path softmax bwd B={B} T={T} H={H} G={G}", flush=True)
    leaves = [x.cuda().requires_grad_() for x in (q, k, v, w, beta)]
    o, _ = parallel_path_attention(*leaves)
    o.backward(do.cuda())
    torch.cuda.synchronize()
    Tp = (T + 63) // 64 * 64
    _, ref = TL.path_attention_twolevel(*(_padded(x, Tp) for x in (q, k, v, w, beta)), do=_padded(do, Tp),
                                        scale=0.125, C=64, S=512, softmax=True)
    for name, x, r in zip(("dq", "dk", "dv", "dw", "dbeta"), leaves, ref):
        r = r[:, :T]
        err = (x.grad.cpu().double() - r).abs().max().item()
        check(name, err, r.abs().max().item())


def test_path_softmax_beta_zero_is_causal_attention():
    """beta = 0 removes every reflection: plain causal softmax attention (GQA), checked against
    torch SDPA in float32 at T = 4096 (8 large chunks), forward and the q, k, v gradients."""
    from lucid_amd.lucid_path import parallel_path_attention
    T, H, G = 4096, 2, 2
    q, k, v, w, beta, do = _inputs(1, T, H, G, seed=61, beta_zero=True)
    print(f"case path softmax beta=0 T={T}", flush=True)
    leaves = [x.cuda().requires_grad_() for x in (q, k, v)]
    o, _ = parallel_path_attention(*leaves, w.cuda(), beta.cuda())
    o.backward(do.cuda())
    ref_leaves = [x.cuda().float().requires_grad_() for x in (q, k, v)]
    qr, kr, vr = ref_leaves
    kk, vv = (x.repeat_interleave(G, dim=2).transpose(1, 2) for x in (kr, vr))
    ref = torch.nn.functional.scaled_dot_product_attention(qr.transpose(1, 2), kk, vv, is_causal=True, scale=0.125)
    ref = ref.transpose(1, 2)
    ref.backward(do.cuda().float())
    torch.cuda.synchronize()
    assert (o.float() - ref).abs().max().item() <= TOL
    for name, a, r in zip(("dq", "dk", "dv"), leaves, ref_leaves):
        err = (a.grad.float() - r.grad).abs().max().item()
        check(name, err, r.grad.abs().max().item())


def test_path_softmax_long_sequence_sampled_rows():
    """T = 8192 (16 large chunks): sampled output rows recomputed from the definition, with the
    path logits of each row obtained by explicit fp32 Householder transport of its query."""
    from lucid_amd.lucid_path import parallel_path_attention
    T = 8192
    q, k, v, w, beta, _ = _inputs(1, T, 1, 1, seed=71)
    qc, kc_, vc, wc, bc = (x.cuda() for x in (q, k, v, w, beta))
    print(f"case path softmax sampled rows T={T}", flush=True)
    o, _ = parallel_path_attention(qc, kc_, vc, wc, bc)
    torch.cuda.synchronize()
    kf, wf, bf, vf = kc_[0, :, 0].float(), wc[0, :, 0].float(), bc[0, :, 0].float(), vc[0, :, 0].float()
    for i in (0, 1, 63, 64, 700, 4100, T - 1):
        x = qc[0, i, 0].float()
        row = torch.empty(i + 1, device="cuda")
        row[i] = x @ kf[i]
        for j in range(i - 1, -1, -1):  # x <- H_{j+1} x, then A_ij = x . k_j
            x = x - bf[j + 1] * (x @ wf[j + 1]) * wf[j + 1]
            row[j] = x @ kf[j]
        ref = torch.softmax(row * 0.125, dim=0) @ vf[: i + 1]
        err = (o[0, i, 0].float() - ref).abs().max().item()
        assert err <= TOL, f"row {i}: max err {err:.3e}"


@pytest.mark.parametrize("softmax", [False, True])
def test_varlen_packed_sequences(softmax):
    """cu_seqlens (packed sequences, B = 1): each sequence independent; outputs and gradients
    against the float64 oracle of every sequence on its own (lengths span several buckets)."""
    from lucid_amd.lucid_path import parallel_lucid_path_attention, parallel_path_attention
    bounds = [0, 100, 228, 740, 800, 864]
    T = bounds[-1]
    q, k, v, w, beta, do = _inputs(1, T, 2, 1, seed=81 + softmax)
    print(f"case varlen softmax={softmax} bounds={bounds}", flush=True)
    leaves = [x.cuda().requires_grad_() for x in (q, k, v, w, beta)]
    cu = torch.tensor(bounds, dtype=torch.int32, device="cuda")
    if softmax:
        o, kc = parallel_path_attention(*leaves, cu_seqlens=cu, use_cache=True)
    else:
        qq, kk, vv, ww, bb = leaves
        o, kc = parallel_lucid_path_attention(kk, vv, ww, bb, q=qq, cu_seqlens=cu, use_cache=True)
    o.backward(do.cuda())
    torch.cuda.synchronize()
    assert o.shape == (1, T, 2, 64) and kc.shape == (1, T, 2, 64)
    for s0, s1 in zip(bounds[:-1], bounds[1:]):
        n = s1 - s0
        tp = (n + 63) // 64 * 64
        seg = [_padded(x[:, s0:s1], tp) for x in (q, k, v, w, beta)]
        o_ref, g_ref = TL.path_attention_twolevel(*seg, do=_padded(do[:, s0:s1], tp), scale=0.125, C=64, S=512,
                                                  softmax=softmax)
        err = (o[:, s0:s1].detach().cpu().double() - o_ref[:, :n]).abs().max().item()
        assert err <= TOL, f"seq [{s0},{s1}) O err {err:.3e}"
        for name, x, r in zip(("dq", "dk", "dv", "dw", "dbeta"), leaves, g_ref):
            r = r[:, :n]
            e = (x.grad[:, s0:s1].cpu().double() - r).abs().max().item()
            check(f"seq [{s0},{s1}) {name}", e, r.abs().max().item())
        kc_ref = P.path_kcache_bruteforce(_f64(k[:, s0:s1]), _f64(w[:, s0:s1]), _f64(beta[:, s0:s1])) if n <= 128 \
            else None
        if kc_ref is not None:
            e = (kc[:, s0:s1].cpu().double() - kc_ref).abs().max().item()
            check(f"seq [{s0},{s1}) k_cache", e, kc_ref.abs().max().item())


def test_empty_sequence_returns_empty():
    from lucid_amd.lucid_path import parallel_lucid_path_attention, parallel_path_attention
    q, k, v, w, beta, _ = _inputs(1, 0, 2, 1, seed=1)
    leaves = [x.cuda().requires_grad_() for x in (q, k, v, w, beta)]
    o, kc = parallel_path_attention(*leaves, use_cache=True)
    assert o.shape == (1, 0, 2, 64) and kc.shape == (1, 0, 2, 64)
    o.sum().backward()
    assert all(x.grad is not None and x.grad.shape == x.shape for x in leaves)
    o2, kc2 = parallel_lucid_path_attention(*leaves[1:], q=leaves[0])
    assert o2.shape == (1, 0, 2, 64) and kc2 is None
