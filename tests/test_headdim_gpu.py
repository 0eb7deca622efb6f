"""GPU parity at head dims other than 64 and 128.

The reference model's shipped config uses head_dim 68 with GQA 32/4 in fp32
(lucid/config/config.json:9, :25) and its torch path takes any d.  These head dims run on
rows zero-padded to 64 or 128 columns with the RMS of k_norm over the true d; every case
is compared with the float64 oracle on the same inputs (the oracle computes at the true d,
so a padded column leaking into the RMS, the scale or an output would show here):
O, V', dQ, dK, dV at the bf16 bars of tests/bars.py, fp32 inputs at rel 1e-4, the two
operator seams composed like LucidAttention.forward, and decoded rows against the
prefill rows of the oracle.
"""
import numpy as np
import pytest
import torch

from bars import check, check_f32
from oracle import lucid_ref as R

pytestmark = pytest.mark.gpu


def _inputs(B, Hq, Hkv, T, D, seed, qk_std=None, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    s = D ** -0.5
    qs = s if qk_std is None else qk_std
    q = (torch.randn(B, Hq, T, D, generator=g) * qs).to(dtype)
    k = (torch.randn(B, Hkv, T, D, generator=g) * qs).to(dtype)
    v = (torch.randn(B, Hkv, T, D, generator=g) * s).to(dtype)
    do = torch.randn(B, T, Hq, D, generator=g).to(dtype)
    return q, k, v, do


def _np(t):
    return t.detach().float().cpu().double().numpy() if t.dtype != torch.float32 else t.detach().cpu().double().numpy()


CASES = [
    # B, Hq, Hkv, T, D, q/k std (None: 1/sqrt(d); 1.0: O(1) scores)
    (1, 8, 1, 300, 68, None),   # the reference model's head dim and GQA ratio (32/4), ragged T
    (1, 8, 1, 256, 68, 1.0),
    (2, 2, 2, 256, 32, 1.0),
    (1, 4, 2, 384, 96, None),
    (1, 2, 1, 256, 16, 1.0),
    (1, 2, 2, 128, 127, None),
    # edges of the active-column instances (80 columns up to d = 80, 96 up to 96, else 128),
    # the first with the reference model's 32 / 4 grouping
    (1, 32, 4, 256, 80, None),
    (1, 4, 2, 256, 81, 1.0),
    (1, 2, 1, 256, 97, None),
]


@pytest.mark.parametrize("B,Hq,Hkv,T,D,qk_std", CASES)
def test_padded_head_dim_matches_oracle(B, Hq, Hkv, T, D, qk_std):
    from lucid_amd import lucid_attention
    q, k, v, do = _inputs(B, Hq, Hkv, T, D, seed=T + 3 * D, qk_std=qk_std)
    print(f"case head dim B={B} Hq={Hq} Hkv={Hkv} T={T} D={D} qk_std={qk_std}", flush=True)
    qg, kg, vg = (t.cuda().requires_grad_() for t in (q, k, v))
    o, vp = lucid_attention(qg, kg, vg, return_vprime=True)
    assert o.shape == (B, T, Hq, D) and vp.shape == (B, Hkv, T, D)
    o.backward(do.cuda())
    torch.cuda.synchronize()
    s = D ** -0.5
    o_ref, vp_ref = R.lucid_attention(_np(q), _np(k), _np(v), s, 1e-5)
    refs = R.lucid_attention_grads(_np(q), _np(k), _np(v), _np(do), s, 1e-5)
    for name, got, ref in zip(("o", "vprime", "dq", "dk", "dv"), (o, vp, qg.grad, kg.grad, vg.grad),
                              (o_ref, vp_ref, *refs)):
        assert got.shape == ref.shape, name
        err = float(np.abs(_np(got) - ref).max())
        print(f"  {name}: max err {err:.2e} max|ref| {np.abs(ref).max():.2e}", flush=True)
        check(name, err, float(np.abs(ref).max()))


@pytest.mark.parametrize("B,Hq,Hkv,T,D", [(1, 2, 1, 512, 48), (1, 2, 2, 384, 20),
                                           (1, 4, 2, 256, 80), (1, 2, 2, 256, 81), (1, 2, 1, 256, 96)])
def test_padded_head_dim_fp32(B, Hq, Hkv, T, D):
    from lucid_amd import lucid_attention
    q, k, v, do = _inputs(B, Hq, Hkv, T, D, seed=5 * T + D, qk_std=1.0, dtype=torch.float32)
    print(f"case head dim fp32 B={B} Hq={Hq} Hkv={Hkv} T={T} D={D}", flush=True)
    qg, kg, vg = (t.cuda().requires_grad_() for t in (q, k, v))
    o, vp = lucid_attention(qg, kg, vg, return_vprime=True)
    assert o.dtype == torch.float32
    o.backward(do.cuda())
    torch.cuda.synchronize()
    s = D ** -0.5
    o_ref, vp_ref = R.lucid_attention(_np(q), _np(k), _np(v), s, 1e-5)
    refs = R.lucid_attention_grads(_np(q), _np(k), _np(v), _np(do), s, 1e-5)
    for name, got, ref in zip(("o", "vprime", "dq", "dk", "dv"), (o, vp, qg.grad, kg.grad, vg.grad),
                              (o_ref, vp_ref, *refs)):
        err = float(np.abs(_np(got) - ref).max())
        print(f"  {name}: max err {err:.2e} max|ref| {np.abs(ref).max():.2e}", flush=True)
        check_f32(name, err, float(np.abs(ref).max()))


def test_padded_head_dim_seams_composed():
    """get_v_prime and eager_lucid_attention_forward at d = 68, composed as
    LucidAttention.forward composes them (modeling_lucid.py:461-496), against the oracle and
    the fused op."""
    from lucid_amd import eager_lucid_attention_forward, get_v_prime, lucid_attention
    B, Hq, Hkv, T, D = 1, 4, 1, 256, 68
    q, k, v, do = _inputs(B, Hq, Hkv, T, D, seed=68, qk_std=1.0)
    print("case head dim seams D=68", flush=True)
    qg, kg, vg = (t.cuda().requires_grad_() for t in (q, k, v))
    vp = get_v_prime(kg, vg)
    assert vp.shape == (B, Hkv, T, D) and vp.dtype == torch.bfloat16
    o, none = eager_lucid_attention_forward(qg, kg, vp)
    assert none is None and o.shape == (B, T, Hq, D)
    o.backward(do.cuda())
    torch.cuda.synchronize()
    s = D ** -0.5
    o_ref, vp_ref = R.lucid_attention(_np(q), _np(k), _np(v), s, 1e-5)
    refs = R.lucid_attention_grads(_np(q), _np(k), _np(v), _np(do), s, 1e-5)
    for name, got, ref in zip(("o", "vprime", "dq", "dk", "dv"), (o, vp, qg.grad, kg.grad, vg.grad),
                              (o_ref, vp_ref, *refs)):
        err = float(np.abs(_np(got) - ref).max())
        print(f"  {name}: max err {err:.2e} max|ref| {np.abs(ref).max():.2e}", flush=True)
        check(name, err, float(np.abs(ref).max()))
    of = lucid_attention(q.cuda(), k.cuda(), v.cuda())
    assert torch.equal(of, o.detach())  # the same kernels on the same operands


@pytest.mark.parametrize("B,Hq,Hkv,T0,n,D", [(1, 8, 1, 200, 3, 68), (2, 2, 2, 64, 2, 40)])
def test_padded_head_dim_decode(B, Hq, Hkv, T0, n, D):
    """Prefill T0 rows, decode n more into padded cache buffers; the decoded O and V' rows
    equal the oracle's rows of the whole sequence."""
    from lucid_amd import lucid_attention, lucid_decode
    from lucid_amd.lucid import _padded_dim
    T = T0 + n
    q, k, v, _ = _inputs(B, Hq, Hkv, T, D, seed=T0 + D)
    print(f"case head dim decode B={B} Hq={Hq} Hkv={Hkv} T0={T0} n={n} D={D}", flush=True)
    qc, kc_, vc_ = q.cuda(), k.cuda(), v.cuda()
    dp = _padded_dim(D)
    kc = torch.zeros(B, Hkv, T + 5, dp, dtype=torch.bfloat16, device="cuda")
    vc = torch.zeros_like(kc)
    _, vp0 = lucid_attention(qc[:, :, :T0], kc_[:, :, :T0], vc_[:, :, :T0], return_vprime=True)
    kc[:, :, :T0, :D] = kc_[:, :, :T0]
    vc[:, :, :T0, :D] = vp0.to(torch.bfloat16)
    with pytest.raises(ValueError, match="cache buffers"):
        lucid_decode(qc[:, :, T0:T0 + 1], kc_[:, :, T0:T0 + 1], vc_[:, :, T0:T0 + 1], kc[..., :D], vc[..., :D], T0)
    outs, vps = [], []
    for t in range(T0, T):
        o, vp = lucid_decode(qc[:, :, t:t + 1], kc_[:, :, t:t + 1], vc_[:, :, t:t + 1], kc, vc, t)
        assert o.shape == (B, 1, Hq, D) and vp.shape == (B, Hkv, 1, D)
        outs.append(o)
        vps.append(vp)
    torch.cuda.synchronize()
    o_dec, vp_dec = torch.cat(outs, 1), torch.cat(vps, 2)
    o_ref, vp_ref = R.lucid_attention(_np(q), _np(k), _np(v), D ** -0.5, 1e-5)
    err_o = float(np.abs(_np(o_dec) - o_ref[:, T0:]).max())
    err_v = float(np.abs(_np(vp_dec) - vp_ref[:, :, T0:]).max())
    print(f"  o err {err_o:.2e} vprime err {err_v:.2e}", flush=True)
    check("o", err_o, float(np.abs(o_ref[:, T0:]).max()))
    check("vprime", err_v, float(np.abs(vp_ref[:, :, T0:]).max()))
    # the appended keys, and the padded columns of both caches stay zero
    assert torch.equal(kc[:, :, T0:T, :D], kc_[:, :, T0:T])
    assert not kc[..., D:].any() and not vc[..., D:].any()
