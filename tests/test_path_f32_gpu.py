"""GPU parity of LUCID-Path and PaTH softmax attention on fp32 inputs.

The reference's LUCID-Path model is fp32 (lucid_path/config/config.json:5, head dim
2048 / 32 = 64) and its Triton entry point takes fp32 tensors (parallel.py:180-241).  Here
fp32 runs the same kernels with every bf16 operand kept as hi / lo planes and every product
taken as a 3-term split, so the bar is the north star's fp32 tolerance: max |x - ref| <=
1e-4 max |ref| against the float64 oracles on the same fp32 inputs (tests/bars.py
check_f32), forward and every gradient.  Oracles: oracle/path_ref.py (chunked restatement
and brute force, pinned in tests/test_oracle_path.py) on the CPU for short sequences, the
dense oracle oracle/path_dense.py (pinned in tests/test_oracle_path_dense.py) on the GPU for
long ones.
"""
import pytest
import torch

from bars import check_f32
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
    return [x.float() for x in (q, k, v, w, beta, do)]


def _f64(x):
    return x.detach().cpu().double()


def _pad_t(x, Tp):
    return torch.nn.functional.pad(_f64(x), [0, 0] * (x.dim() - 2) + [0, Tp - x.shape[1]])


def _cmp(name, got, ref):
    err = (got.detach().cpu().double() - ref.cpu()).abs().max().item()
    scale = ref.abs().max().item()
    print(f"  {name}: max err {err:.2e} max|ref| {scale:.2e} rel {err / scale:.1e}", flush=True)
    check_f32(name, err, scale)


@pytest.mark.parametrize("B,T,H,G,K,V", [(1, 256, 2, 1, 64, 64), (1, 200, 1, 2, 32, 32), (2, 640, 1, 1, 64, 64),
                                         (1, 576, 1, 2, 64, 16)])
def test_lucid_path_f32_matches_oracle(B, T, H, G, K, V):
    from lucid_amd.lucid_path import parallel_lucid_path_attention
    q, k, v, w, beta, do = _inputs(B, T, H, G, K, V, seed=19 * T + K + V)
    print(f"case path f32 B={B} T={T} H={H} G={G} K={K} V={V}", flush=True)
    leaves = [x.cuda().requires_grad_() for x in (q, k, v, w, beta)]
    o, kc = parallel_lucid_path_attention(leaves[1], leaves[2], leaves[3], leaves[4], q=leaves[0], use_cache=True)
    assert o.dtype == torch.float32 and kc.dtype == torch.float32
    o.backward(do.cuda())
    torch.cuda.synchronize()
    Tp = (T + 63) // 64 * 64
    s = K ** -0.5
    ref = P.path_attention_chunked(*(_pad_t(x, Tp) for x in (q, k, v, w, beta)), scale=s, C=64)[:, :T]
    _cmp("o", o, ref)
    if T <= 256:
        _cmp("k_cache", kc, P.path_kcache_bruteforce(_f64(k), _f64(w), _f64(beta)))
    grads = P.path_attention_grads(*(_pad_t(x, Tp) for x in (q, k, v, w, beta)), _pad_t(do, Tp), scale=s, C=64)
    for name, got, r in zip(("dq", "dk", "dv", "dw", "dbeta"), leaves, grads):
        assert got.grad.dtype == torch.float32
        _cmp(name, got.grad, r[:, :T])


@pytest.mark.parametrize("B,T,H,G", [(1, 4096, 2, 2)])
def test_lucid_path_f32_long(B, T, H, G):
    """Several super-chunks (QB operands, HL transitions, the chained solve over 64 chunks)
    against the dense float64 oracle on the GPU, every head."""
    from lucid_amd.lucid_path import parallel_lucid_path_attention
    q, k, v, w, beta, do = (x.cuda() for x in _inputs(B, T, H, G, 64, 64, seed=7 * T + G))
    print(f"case path f32 long B={B} T={T} H={H} G={G}", flush=True)
    leaves = [x.clone().requires_grad_() for x in (q, k, v, w, beta)]
    o, _ = parallel_lucid_path_attention(leaves[1], leaves[2], leaves[3], leaves[4], q=leaves[0])
    o.backward(do)
    torch.cuda.synchronize()
    ref_o, ref_g = PD.path_attention_dense(q, k, v, w, beta, do=do, scale=0.125)
    _cmp("o", o, ref_o)
    for name, got, r in zip(("dq", "dk", "dv", "dw", "dbeta"), leaves, ref_g):
        _cmp(name, got.grad, r)


@pytest.mark.parametrize("B,T,H,G,K,V", [(1, 256, 1, 1, 64, 64), (1, 192, 1, 2, 32, 64)])
def test_path_softmax_f32_matches_oracle(B, T, H, G, K, V):
    from lucid_amd.lucid_path import parallel_path_attention
    q, k, v, w, beta, do = _inputs(B, T, H, G, K, V, seed=23 * T + K + V)
    print(f"case path softmax f32 B={B} T={T} H={H} G={G} K={K} V={V}", flush=True)
    leaves = [x.cuda().requires_grad_() for x in (q, k, v, w, beta)]
    o, _ = parallel_path_attention(*leaves)
    o.backward(do.cuda())
    torch.cuda.synchronize()
    s = K ** -0.5
    _cmp("o", o, P.path_softmax_bruteforce(*(_f64(x) for x in (q, k, v, w, beta)), scale=s))
    grads = P.path_softmax_grads(*(_f64(x) for x in (q, k, v, w, beta)), _f64(do), scale=s)
    for name, got, r in zip(("dq", "dk", "dv", "dw", "dbeta"), leaves, grads):
        _cmp(name, got.grad, r)


def test_path_softmax_f32_long():
    from lucid_amd.lucid_path import parallel_path_attention
    q, k, v, w, beta, do = (x.cuda() for x in _inputs(1, 2048, 2, 2, 64, 64, seed=99))
    print("case path softmax f32 long B=1 T=2048 H=2 G=2", flush=True)
    leaves = [x.clone().requires_grad_() for x in (q, k, v, w, beta)]
    o, _ = parallel_path_attention(*leaves)
    o.backward(do)
    torch.cuda.synchronize()
    ref_o, ref_g = PD.path_attention_dense(q, k, v, w, beta, do=do, scale=0.125, softmax=True)
    _cmp("o", o, ref_o)
    for name, got, r in zip(("dq", "dk", "dv", "dw", "dbeta"), leaves, ref_g):
        _cmp(name, got.grad, r)


def test_path_f32_rejects_wide_heads_and_mixed_dtypes():
    from lucid_amd.lucid_path import parallel_lucid_path_attention
    q, k, v, w, beta, _ = (x.cuda() for x in _inputs(1, 64, 1, 1, 128, 128, seed=1))
    with pytest.raises(NotImplementedError, match="fp32"):
        parallel_lucid_path_attention(k, v, w, beta, q=q)
    q, k, v, w, beta, _ = (x.cuda() for x in _inputs(1, 64, 1, 1, 64, 64, seed=1))
    with pytest.raises(TypeError, match="dtype"):
        parallel_lucid_path_attention(k, v.bfloat16(), w, beta, q=q)


@pytest.mark.parametrize("softmax", [False, True])
def test_path_f32_varlen_packed_sequences(softmax):
    """cu_seqlens on fp32 inputs: every packed sequence against its own float64 oracle at the
    fp32 bar (lengths in three 64-position buckets, one ragged)."""
    from lucid_amd.lucid_path import parallel_lucid_path_attention, parallel_path_attention
    bounds = [0, 70, 198, 262]
    T = bounds[-1]
    q, k, v, w, beta, do = _inputs(1, T, 2, 1, 64, 64, seed=31 + softmax)
    print(f"case path f32 varlen softmax={softmax} bounds={bounds}", flush=True)
    leaves = [x.cuda().requires_grad_() for x in (q, k, v, w, beta)]
    cu = torch.tensor(bounds, dtype=torch.int32, device="cuda")
    if softmax:
        o, kc = parallel_path_attention(*leaves, cu_seqlens=cu, use_cache=True)
    else:
        o, kc = parallel_lucid_path_attention(leaves[1], leaves[2], leaves[3], leaves[4], q=leaves[0], cu_seqlens=cu,
                                              use_cache=True)
    o.backward(do.cuda())
    torch.cuda.synchronize()
    for s0, s1 in zip(bounds[:-1], bounds[1:]):
        seg = [_f64(x[:, s0:s1]) for x in (q, k, v, w, beta)]
        if softmax:
            o_ref = P.path_softmax_bruteforce(*seg, scale=0.125)
            g_ref = P.path_softmax_grads(*seg, _f64(do[:, s0:s1]), scale=0.125)
        else:
            n = s1 - s0
            tp = (n + 63) // 64 * 64
            segp = [_pad_t(x, tp) for x in seg]
            o_ref = P.path_attention_chunked(*segp, scale=0.125, C=64)[:, :n]
            g_ref = [r[:, :n] for r in P.path_attention_grads(*segp, _pad_t(do[:, s0:s1], tp), scale=0.125, C=64)]
        _cmp(f"seq [{s0},{s1}) o", o[:, s0:s1], o_ref)
        _cmp(f"seq [{s0},{s1}) k_cache", kc[:, s0:s1], P.path_kcache_bruteforce(*seg[1:2], seg[3], seg[4]))
        for name, x, r in zip(("dq", "dk", "dv", "dw", "dbeta"), leaves, g_ref):
            _cmp(f"seq [{s0},{s1}) {name}", x.grad[:, s0:s1], r)


def test_path_f32_empty_sequence():
    from lucid_amd.lucid_path import parallel_lucid_path_attention, parallel_path_attention
    leaves = [x.cuda().requires_grad_() for x in _inputs(1, 0, 2, 1, 64, 64, seed=1)[:5]]
    o, kc = parallel_path_attention(*leaves, use_cache=True)
    assert o.shape == (1, 0, 2, 64) and o.dtype == torch.float32 and kc.shape == (1, 0, 2, 64)
    o.sum().backward()
    assert all(x.grad is not None and x.grad.shape == x.shape for x in leaves)
    o2, kc2 = parallel_lucid_path_attention(*leaves[1:], q=leaves[0])
    assert o2.shape == (1, 0, 2, 64) and kc2 is None
