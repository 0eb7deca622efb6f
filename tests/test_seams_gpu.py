"""GPU parity of the two operator seams, get_v_prime and eager_lucid_attention_forward, used
separately and composed the way LucidAttention.forward composes them (modeling_lucid.py:461-496):

    v_prime = get_v_prime(key, value, scaling, attention_mask)
    attn_output, _ = eager_lucid_attention_forward(query, key, v_prime, scaling, attention_mask)

Checked against the fused lucid_attention (same kernels in one call) and against the float64
oracle (tests/bars.py bars), forward and gradients.  Plain causal attention on the same
kernels (V' = V) is checked against float32 SDPA on the CPU.
"""
import numpy as np
import pytest
import torch

from bars import check
from oracle import lucid_ref as R

pytestmark = pytest.mark.gpu


def _inputs(B, Hq, Hkv, T, D, seed, correlated=False):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, Hq, T, D, generator=g)
    if correlated:
        k = torch.randn(B, Hkv, 1, D, generator=g) + 0.1 * torch.randn(B, Hkv, T, D, generator=g)
    else:
        k = torch.randn(B, Hkv, T, D, generator=g)
    v = torch.randn(B, Hkv, T, D, generator=g) / 8
    do = torch.randn(B, T, Hq, D, generator=g)
    return [x.to(torch.bfloat16) for x in (q, k, v, do)]


def _np(t):
    return t.detach().float().cpu().double().numpy()


def _err(x, ref):
    return float(np.abs(_np(x) - ref).max())


CASES = [
    # B, Hq, Hkv, T, D, correlated keys (the exact chains)
    (1, 2, 2, 256, 64, False),
    (2, 4, 2, 384, 64, False),
    (1, 2, 1, 200, 64, False),
    (1, 2, 2, 256, 128, False),
    (1, 2, 2, 512, 64, True),
]


@pytest.mark.parametrize("B,Hq,Hkv,T,D,corr", CASES)
def test_seams_composed_like_lucid_attention(B, Hq, Hkv, T, D, corr):
    from lucid_amd import eager_lucid_attention_forward, get_v_prime, lucid_attention, set_fused_forward
    q, k, v, do = _inputs(B, Hq, Hkv, T, D, seed=T + D + corr, correlated=corr)
    print(f"case seams B={B} Hq={Hq} Hkv={Hkv} T={T} D={D} correlated={corr}", flush=True)
    s = D ** -0.5
    mask = torch.ones(T, T, dtype=torch.bool, device="cuda").tril()[None, None].expand(B, 1, T, T)
    qg, kg, vg = (t.cuda().requires_grad_() for t in (q, k, v))
    v_prime = get_v_prime(kg, vg, s, mask)
    assert v_prime.dtype == torch.bfloat16 and v_prime.requires_grad
    o, w = eager_lucid_attention_forward(qg, kg, v_prime, s, mask)
    assert w is None and o.shape == (B, T, Hq, D)
    o.backward(do.cuda())
    # the fused op on the same inputs, with the two-kernel forward (chain, then attention: the
    # kernels the seams run)
    qf, kf, vf = (t.cuda().requires_grad_() for t in (q, k, v))
    set_fused_forward(False)
    try:
        of, vpf = lucid_attention(qf, kf, vf, s, return_vprime=True)
    finally:
        set_fused_forward(True)
    of.backward(do.cuda())
    # and with the default schedule (at Hq == Hkv the fused chain + attention kernel)
    o_def, vp_def = lucid_attention(q.cuda(), k.cuda(), v.cuda(), s, return_vprime=True)
    torch.cuda.synchronize()
    # the seam's V' is the fused op's V' rounded to the value dtype, and the attention kernels
    # read the same bf16 V' in both, so O agrees exactly
    assert torch.equal(v_prime.detach(), vpf.to(torch.bfloat16))
    assert torch.equal(o.detach(), of.detach())
    # the fused kernel sums in another order and rounds only the scaled row key of the chain's
    # exponents to bf16 (the chain kernel also the staged K^ rows): V' agrees to ~1e-4
    # relative, O to one bf16 rounding step
    assert float((vp_def - vpf).abs().max()) <= 5e-4 * float(vpf.abs().max())
    assert float((o_def.float() - of.float()).abs().max()) <= 1e-2 * float(of.float().abs().max())
    o_ref, vp_ref = R.lucid_attention(_np(q), _np(k), _np(v), s, 1e-5)
    grads = R.lucid_attention_grads(_np(q), _np(k), _np(v), _np(do), s, 1e-5)
    check("o", _err(o, o_ref), float(np.abs(o_ref).max()))
    check("vprime", _err(v_prime, vp_ref), float(np.abs(vp_ref).max()))
    for name, got, fused, ref in zip(("dq", "dk", "dv"), (qg, kg, vg), (qf, kf, vf), grads):
        scale = float(np.abs(ref).max())
        check(name, _err(got.grad, ref), scale)
        # composed and fused differ only by the bf16 rounding of dV' between the seams
        check(name + " vs fused", float((got.grad.float() - fused.grad.float()).abs().max()), scale)


@pytest.mark.parametrize("corr", [False, True])
def test_get_v_prime_gradient_alone(corr):
    """d/dK and d/dV of sum(V' * W) through get_v_prime alone: dV = P^-T W and the k_norm
    backward of -s (M K^ + M^T K^), against the oracle's closed forms."""
    from lucid_amd import get_v_prime
    B, H, T, D = 1, 2, 384, 64
    _, k, v, _ = _inputs(B, H, H, T, D, seed=31 + corr, correlated=corr)
    wgt = torch.randn(B, H, T, D, generator=torch.Generator().manual_seed(5))
    print(f"case get_v_prime grad correlated={corr}", flush=True)
    kg, vg = k.cuda().requires_grad_(), v.cuda().requires_grad_()
    vp = get_v_prime(kg, vg)
    (vp.float() * wgt.cuda()).sum().backward()
    torch.cuda.synchronize()
    s = D ** -0.5
    kn, vn, wn = _np(k), _np(v), wgt.double().numpy()
    kh = R.k_hat(kn, 1e-5)
    dk_ref = np.empty_like(kn)
    dv_ref = np.empty_like(vn)
    for h in range(H):
        vp_ref = R.vprime_dense(kn[:, h:h + 1], vn[:, h:h + 1], s, 1e-5)[0, 0]
        dkh, dv_ref[0, h] = R.precond_backward(kh[0, h], vp_ref, wn[0, h], s)
        dk_ref[0, h] = R.rmsnorm_backward(kn[0, h], dkh, 1e-5)
    check("dk", _err(kg.grad, dk_ref), float(np.abs(dk_ref).max()))
    check("dv", _err(vg.grad, dv_ref), float(np.abs(dv_ref).max()))


@pytest.mark.parametrize("B,Hq,Hkv,T,D", [(1, 2, 2, 256, 64), (2, 4, 2, 200, 64), (1, 2, 1, 256, 128)])
def test_causal_attention_matches_sdpa(B, Hq, Hkv, T, D):
    """The attention kernels with V' = V are plain causal softmax attention: O and the gradients
    against float32 SDPA on the CPU (GQA expanded by repeat_interleave)."""
    from lucid_amd import causal_attention
    q, k, v, do = _inputs(B, Hq, Hkv, T, D, seed=41 + T)
    print(f"case causal B={B} Hq={Hq} Hkv={Hkv} T={T} D={D}", flush=True)
    qg, kg, vg = (t.cuda().requires_grad_() for t in (q, k, v))
    o = causal_attention(qg, kg, vg)
    o.backward(do.cuda())
    torch.cuda.synchronize()
    qr, kr, vr = (t.float().requires_grad_() for t in (q, k, v))
    G = Hq // Hkv
    ref = torch.nn.functional.scaled_dot_product_attention(qr, kr.repeat_interleave(G, 1), vr.repeat_interleave(G, 1),
                                                           is_causal=True).transpose(1, 2)
    ref.backward(do.float())
    check("o", float((o.float().cpu() - ref).abs().max()), float(ref.abs().max()))
    for name, got, r in (("dq", qg, qr), ("dk", kg, kr), ("dv", vg, vr)):
        check(name, float((got.grad.float().cpu() - r.grad).abs().max()), float(r.grad.abs().max()))


def test_seams_reject_a_non_causal_mask():
    from lucid_amd import eager_lucid_attention_forward, get_v_prime
    q, k, v, _ = (t.cuda() for t in _inputs(1, 2, 2, 128, 64, seed=1))
    full = torch.ones(1, 1, 128, 128, dtype=torch.bool, device="cuda")
    with pytest.raises(NotImplementedError):
        get_v_prime(k, v, None, full)
    with pytest.raises(NotImplementedError):
        eager_lucid_attention_forward(q, k, v, None, full)
    # the causal mask, and a float tensor in the mask slot, are told apart
    causal = full.tril()
    get_v_prime(k, v, None, causal)
    with pytest.raises(NotImplementedError):
        eager_lucid_attention_forward(q, k, v, None, 1e-5)


@pytest.mark.parametrize("dtype,B,Hq,Hkv,T,D", [(torch.bfloat16, 2, 4, 2, 200, 64),
                                                (torch.bfloat16, 3, 2, 2, 384, 64),
                                                (torch.bfloat16, 1, 4, 4, 256, 128),
                                                (torch.float32, 1, 4, 2, 256, 68)])
def test_gradients_follow_the_operand_layout(dtype, B, Hq, Hkv, T, D):
    """Operands given as [B, T, H, d] memory (the projections' view(...).transpose(1, 2)) get
    their gradients in that memory order (head dims 64 and 128, which are not copied into a
    padded buffer), and the values are those of the same call on contiguous [B, H, T, d]
    operands, bit for bit (the same kernels, other output strides)."""
    from lucid_amd import lucid_attention
    print(f"case layouts {dtype} B={B} Hq={Hq} Hkv={Hkv} T={T} D={D}", flush=True)
    q, k, v, do = (x.to(dtype).cuda() for x in _inputs(B, Hq, Hkv, T, D, 11))
    grads = {}
    for tm in (False, True):
        leaves = [(x.transpose(1, 2).contiguous() if tm else x.clone()).requires_grad_() for x in (q, k, v)]
        ops = [x.transpose(1, 2) if tm else x.view(x.shape) for x in leaves]  # non-leaf views
        seen = []
        for x in ops:  # the gradient as the attention backward returns it
            x.register_hook(lambda g_: seen.append((g_.stride(1) < g_.stride(2), g_.clone())))
        o = lucid_attention(*ops)
        o.backward(do)
        torch.cuda.synchronize()
        assert len(seen) == 3
        if D in (64, 128):  # other head dims pass through a zero-padded copy of the operands
            assert all(s_[0] == tm for s_ in seen), [s_[0] for s_ in seen]
        grads[tm] = [o.detach()] + [s_[1] for s_ in seen]
    for a, b in zip(grads[False], grads[True]):
        assert torch.equal(a, b)
