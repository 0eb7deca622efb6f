"""GPU parity of LUCID-Path and PaTH softmax attention on the head-dim-128 kernels.

The reference entry point takes head dim 128 for q/k/w and for v
(lucid_path/triton_code/parallel.py:230-232).  Here K = V = 128 runs on its own kernels
(128 x 128 transport products, 128-wide query transport and solve), and a K/V pair whose
larger member exceeds 64 runs on rows zero-padded to 128.  Oracles: the float64 chunked
restatement (oracle/path_ref.py) on the CPU for short sequences, the float64 dense oracle
(oracle/path_dense.py, pinned in tests/test_oracle_path_dense.py) on the GPU for long ones;
the decode key cache against the brute-force reflection product.  Bars: tests/bars.py
(bf16 against float64 on the same bf16-rounded inputs).
"""
import pytest
import torch

from bars import check
from oracle import path_dense as PD
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


@pytest.mark.parametrize("B,T,H,G,K,V", [(1, 256, 1, 1, 128, 128), (2, 192, 2, 2, 128, 128),
                                         (1, 200, 1, 1, 64, 128), (1, 128, 2, 1, 128, 32)])
def test_lucid_path_d128_forward_short(B, T, H, G, K, V):
    from lucid_amd.lucid_path import parallel_lucid_path_attention
    q, k, v, w, beta, _ = _inputs(B, T, H, G, K, V, seed=11 * T + K + V)
    print(f"case path d128 fwd B={B} T={T} H={H} G={G} K={K} V={V}", flush=True)
    with torch.no_grad():
        o, kc = parallel_lucid_path_attention(k.cuda(), v.cuda(), w.cuda(), beta.cuda(), q=q.cuda(),
                                              use_cache=True)
    torch.cuda.synchronize()
    assert o.shape == (B, T, H * G, V) and kc.shape == (B, T, H, K)
    Tp = (T + 63) // 64 * 64
    ref = P.path_attention_chunked(*(_pad_t(x, Tp) for x in (q, k, v, w, beta)), scale=K ** -0.5, C=64)[:, :T]
    err = (o.cpu().double() - ref).abs().max().item()
    print(f"  o: max err {err:.2e} max|ref| {ref.abs().max().item():.2e}", flush=True)
    check("o", err, ref.abs().max().item())
    kc_ref = P.path_kcache_bruteforce(_f64(k), _f64(w), _f64(beta))
    err = (kc.cpu().double() - kc_ref).abs().max().item()
    print(f"  k_cache: max err {err:.2e} max|ref| {kc_ref.abs().max().item():.2e}", flush=True)
    check("k_cache", err, kc_ref.abs().max().item())


@pytest.mark.parametrize("B,T,H,G", [(1, 1024, 2, 2), (1, 8192, 1, 1)])
def test_lucid_path_d128_forward_long(B, T, H, G):
    """Several super-chunks (S = 512 positions): the large-chunk products, the query transport
    across super-chunks and the chained solve over up to 128 chunks."""
    from lucid_amd.lucid_path import parallel_lucid_path_attention
    q, k, v, w, beta, _ = (x.cuda() for x in _inputs(B, T, H, G, 128, 128, seed=T + G))
    print(f"case path d128 fwd long B={B} T={T} H={H} G={G}", flush=True)
    with torch.no_grad():
        o, _ = parallel_lucid_path_attention(k, v, w, beta, q=q)
    torch.cuda.synchronize()
    heads = range(H * G) if T <= 1024 else [0]
    ref = PD.path_attention_dense(q, k, v, w, beta, scale=128 ** -0.5, heads=heads)
    for hq in heads:
        err = (o[:, :, hq].double() - ref[:, :, hq]).abs().max().item()
        print(f"  head {hq} o: max err {err:.2e} max|ref| {ref[:, :, hq].abs().max().item():.2e}", flush=True)
        check(f"o[{hq}]", err, ref[:, :, hq].abs().max().item())


@pytest.mark.parametrize("B,T,H,G,K,V", [(1, 256, 1, 1, 128, 128), (2, 192, 2, 2, 128, 128),
                                         (1, 200, 1, 1, 64, 128), (1, 128, 2, 1, 128, 32)])
def test_lucid_path_d128_backward_short(B, T, H, G, K, V):
    from lucid_amd.lucid_path import parallel_lucid_path_attention
    q, k, v, w, beta, do = _inputs(B, T, H, G, K, V, seed=13 * T + K + V)
    print(f"case path d128 bwd B={B} T={T} H={H} G={G} K={K} V={V}", flush=True)
    leaves = [x.cuda().requires_grad_() for x in (q, k, v, w, beta)]
    o, _ = parallel_lucid_path_attention(leaves[1], leaves[2], leaves[3], leaves[4], q=leaves[0])
    o.backward(do.cuda())
    torch.cuda.synchronize()
    Tp = (T + 63) // 64 * 64
    s = K ** -0.5
    ref = P.path_attention_chunked(*(_pad_t(x, Tp) for x in (q, k, v, w, beta)), scale=s, C=64)[:, :T]
    check("o", (o.detach().cpu().double() - ref).abs().max().item(), ref.abs().max().item())
    grads = P.path_attention_grads(*(_pad_t(x, Tp) for x in (q, k, v, w, beta)), _pad_t(do, Tp), scale=s, C=64)
    for name, got, r in zip(("dq", "dk", "dv", "dw", "dbeta"), leaves, grads):
        r = r[:, :T]
        assert got.grad.shape == r.shape, name
        err = (got.grad.cpu().double() - r).abs().max().item()
        print(f"  {name}: max err {err:.2e} max|ref| {r.abs().max().item():.2e}", flush=True)
        check(name, err, r.abs().max().item())


@pytest.mark.parametrize("B,T,H,G", [(1, 1024, 2, 2), (1, 8192, 1, 1)])
def test_lucid_path_d128_backward_long(B, T, H, G):
    """Gradients across super-chunks: the row and column sweeps over QB / QS operands, the
    128 x 128 transport gradients (dHL, dHc) and the products backward."""
    from lucid_amd.lucid_path import parallel_lucid_path_attention
    q, k, v, w, beta, do = (x.cuda() for x in _inputs(B, T, H, G, 128, 128, seed=3 * T + G))
    print(f"case path d128 bwd long B={B} T={T} H={H} G={G}", flush=True)
    leaves = [x.clone().requires_grad_() for x in (q, k, v, w, beta)]
    o, _ = parallel_lucid_path_attention(leaves[1], leaves[2], leaves[3], leaves[4], q=leaves[0])
    o.backward(do)
    torch.cuda.synchronize()
    ref_o, ref_g = PD.path_attention_dense(q, k, v, w, beta, do=do, scale=128 ** -0.5)
    check("o", (o.detach().double() - ref_o).abs().max().item(), ref_o.abs().max().item())
    for name, got, r in zip(("dq", "dk", "dv", "dw", "dbeta"), leaves, ref_g):
        err = (got.grad.double() - r).abs().max().item()
        print(f"  {name}: max err {err:.2e} max|ref| {r.abs().max().item():.2e}", flush=True)
        check(name, err, r.abs().max().item())


@pytest.mark.parametrize("B,T,H,G,K,V", [(1, 256, 1, 1, 128, 128), (1, 192, 1, 2, 128, 128), (1, 128, 2, 1, 64, 128)])
def test_path_softmax_d128_short(B, T, H, G, K, V):
    """PaTH softmax attention on the head-dim-128 kernels against the brute-force float64
    oracle (explicit Householder products), forward and backward."""
    from lucid_amd.lucid_path import parallel_path_attention
    q, k, v, w, beta, do = _inputs(B, T, H, G, K, V, seed=17 * T + K + V)
    print(f"case path softmax d128 B={B} T={T} H={H} G={G} K={K} V={V}", flush=True)
    leaves = [x.cuda().requires_grad_() for x in (q, k, v, w, beta)]
    o, _ = parallel_path_attention(*leaves)
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


@pytest.mark.parametrize("B,T,H,G", [(1, 1024, 2, 2), (1, 4096, 1, 1)])
def test_path_softmax_d128_long(B, T, H, G):
    from lucid_amd.lucid_path import parallel_path_attention
    q, k, v, w, beta, do = (x.cuda() for x in _inputs(B, T, H, G, 128, 128, seed=5 * T + G))
    print(f"case path softmax d128 long B={B} T={T} H={H} G={G}", flush=True)
    leaves = [x.clone().requires_grad_() for x in (q, k, v, w, beta)]
    o, _ = parallel_path_attention(*leaves)
    o.backward(do)
    torch.cuda.synchronize()
    ref_o, ref_g = PD.path_attention_dense(q, k, v, w, beta, do=do, scale=128 ** -0.5, softmax=True)
    err = (o.detach().double() - ref_o).abs().max().item()
    print(f"  o: max err {err:.2e} max|ref| {ref_o.abs().max().item():.2e}", flush=True)
    check("o", err, ref_o.abs().max().item())
    for name, got, r in zip(("dq", "dk", "dv", "dw", "dbeta"), leaves, ref_g):
        err = (got.grad.double() - r).abs().max().item()
        print(f"  {name}: max err {err:.2e} max|ref| {r.abs().max().item():.2e}", flush=True)
        check(name, err, r.abs().max().item())


@pytest.mark.parametrize("softmax", [False, True])
def test_path_d128_varlen_packed_sequences(softmax):
    """cu_seqlens at head dim 128: every packed sequence against its own float64 oracle."""
    from lucid_amd.lucid_path import parallel_lucid_path_attention, parallel_path_attention
    bounds = [0, 90, 218, 300]
    T = bounds[-1]
    q, k, v, w, beta, do = _inputs(1, T, 2, 1, 128, 128, seed=41 + softmax)
    print(f"case path d128 varlen softmax={softmax} bounds={bounds}", flush=True)
    leaves = [x.cuda().requires_grad_() for x in (q, k, v, w, beta)]
    cu = torch.tensor(bounds, dtype=torch.int32, device="cuda")
    if softmax:
        o, kc = parallel_path_attention(*leaves, cu_seqlens=cu, use_cache=True)
    else:
        o, kc = parallel_lucid_path_attention(leaves[1], leaves[2], leaves[3], leaves[4], q=leaves[0], cu_seqlens=cu,
                                              use_cache=True)
    o.backward(do.cuda())
    torch.cuda.synchronize()
    s = 128 ** -0.5
    for s0, s1 in zip(bounds[:-1], bounds[1:]):
        seg = [_f64(x[:, s0:s1]) for x in (q, k, v, w, beta)]
        if softmax:
            o_ref = P.path_softmax_bruteforce(*seg, scale=s)
            g_ref = P.path_softmax_grads(*seg, _f64(do[:, s0:s1]), scale=s)
        else:
            n = s1 - s0
            tp = (n + 63) // 64 * 64
            segp = [_pad_t(x, tp) for x in seg]
            o_ref = P.path_attention_chunked(*segp, scale=s, C=64)[:, :n]
            g_ref = [r[:, :n] for r in P.path_attention_grads(*segp, _pad_t(do[:, s0:s1], tp), scale=s, C=64)]
        check(f"seq [{s0},{s1}) o", (o[:, s0:s1].detach().cpu().double() - o_ref).abs().max().item(),
              o_ref.abs().max().item())
        kc_ref = P.path_kcache_bruteforce(seg[1], seg[3], seg[4])
        check(f"seq [{s0},{s1}) k_cache", (kc[:, s0:s1].cpu().double() - kc_ref).abs().max().item(),
              kc_ref.abs().max().item())
        for name, x, r in zip(("dq", "dk", "dv", "dw", "dbeta"), leaves, g_ref):
            check(f"seq [{s0},{s1}) {name}", (x.grad[:, s0:s1].cpu().double() - r).abs().max().item(),
                  r.abs().max().item())
