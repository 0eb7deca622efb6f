"""GPU parity of the Lucid_Tril_Solver seam (modeling_lucid.py:284-382): the solve on keys that
are already normalised, ``Lucid_Tril_Solver.apply(key_hat, value, scaling, BS)``, and its
gradient ``(grad_k_hat, grad_v)`` with no RMSNorm backward.

Ground truth: the float64 oracle ``precond_matrix`` / ``precond_backward`` on the same (bf16- or
fp32-valued) K^ and V.  The K^ fed in are RMS-normalised keys (the reference's only caller,
get_v_prime, :562-565) and, to show that nothing renormalises them, the same keys scaled by 0.6.
"""
import numpy as np
import pytest
import scipy.linalg as sla
import torch

from bars import check, check_f32
from oracle import lucid_ref as R

pytestmark = pytest.mark.gpu

CASES = [
    # B, Hkv, T, D, BS, key factor, dtype
    (1, 2, 1024, 64, 256, 1.0, torch.bfloat16),
    (2, 1, 512, 64, 128, 0.6, torch.bfloat16),
    (1, 2, 512, 128, 256, 1.0, torch.bfloat16),
    (1, 1, 384, 68, 128, 1.0, torch.bfloat16),
    (1, 2, 512, 64, 128, 1.0, torch.float32),
    (1, 1, 256, 40, 64, 0.6, torch.float32),
]


def _np(t):
    return t.detach().cpu().double().numpy()


@pytest.mark.parametrize("B,Hkv,T,D,BS,fac,dt", CASES)
def test_tril_solver_against_oracle(B, Hkv, T, D, BS, fac, dt):
    from lucid_amd.lucid import Lucid_Tril_Solver
    print(f"case tril_solver B={B} Hkv={Hkv} T={T} D={D} BS={BS} factor={fac} dtype={dt}", flush=True)
    g = torch.Generator().manual_seed(T + D)
    k = torch.randn(B, Hkv, T, D, generator=g)
    kh = fac * k * torch.rsqrt(k.pow(2).mean(-1, keepdim=True) + 1e-5)
    v = torch.randn(B, Hkv, T, D, generator=g) / 8
    dvp = torch.randn(B, Hkv, T, D, generator=g)
    kh, v, dvp = (x.to(dt) for x in (kh, v, dvp))
    s = D ** -0.5
    khg, vg = (x.cuda().requires_grad_() for x in (kh, v))
    v_before = vg.detach().clone()
    vp = Lucid_Tril_Solver.apply(khg, vg, s, BS)
    assert vp.dtype == dt and vp.shape == v.shape
    vp.backward(dvp.cuda())
    torch.cuda.synchronize()
    assert torch.equal(vg.detach(), v_before), "value must not be modified"
    khn, vn, dvn = _np(kh), _np(v), _np(dvp)
    errs = {}
    for b in range(B):
        for h in range(Hkv):
            p = R.precond_matrix(khn[b, h], s)
            vp_ref = sla.solve_triangular(p, vn[b, h], lower=True)
            dkh_ref, dv_ref = R.precond_backward(khn[b, h], vp_ref, dvn[b, h], s)
            for name, got, ref in (("vp", vp[b, h], vp_ref), ("dk_hat", khg.grad[b, h], dkh_ref),
                                   ("dv", vg.grad[b, h], dv_ref)):
                err, scale = float(np.abs(_np(got) - ref).max()), float(np.abs(ref).max())
                errs[f"{name}[{b},{h}]"] = (err, scale)
                if dt == torch.float32:
                    check_f32(name, err, scale)
                else:
                    check(name, err, scale)
    print("max errors:", {n: f"{e:.2e}/{s_:.2e}" for n, (e, s_) in errs.items()}, flush=True)


def test_tril_solver_matches_get_v_prime_on_normalised_keys():
    """get_v_prime(K) = Lucid_Tril_Solver(K^(K)) and the chain rule through k_norm links the two
    gradients: dK (get_v_prime) = RMSNorm backward of dK^ (solver)."""
    from lucid_amd.lucid import Lucid_Tril_Solver, get_v_prime
    g = torch.Generator().manual_seed(7)
    B, H, T, D = 1, 2, 512, 64
    k = torch.randn(B, H, T, D, generator=g, dtype=torch.float64)
    v = torch.randn(B, H, T, D, generator=g, dtype=torch.float64) / 8
    dvp = torch.randn(B, H, T, D, generator=g, dtype=torch.float64)
    s = D ** -0.5
    kc = k.float().cuda().requires_grad_()
    vc = v.float().cuda().requires_grad_()
    vp1 = get_v_prime(kc, vc, s)
    vp1.backward(dvp.float().cuda())
    kh = (k * torch.rsqrt(k.pow(2).mean(-1, keepdim=True) + 1e-5)).float().cuda().requires_grad_()
    vc2 = v.float().cuda().requires_grad_()
    vp2 = Lucid_Tril_Solver.apply(kh, vc2, s, 128)
    vp2.backward(dvp.float().cuda())
    torch.cuda.synchronize()
    scale = float(vp1.detach().abs().max())
    check_f32("vp", float((vp1 - vp2).detach().abs().max()), scale)
    check_f32("dv", float((vc.grad - vc2.grad).abs().max()), float(vc.grad.abs().max()))
    # The RMSNorm backward keeps only ~eps r^2 of dK^'s large diagonal term -2 s M_ii K^_i (which
    # lies along K^_i), so the chained solver gradient carries the fp32 error of dK^ itself:
    # the bar scales with r |dK^| rather than with the much smaller |dK|.
    dk_chain = R.rmsnorm_backward(_np(k), _np(kh.grad), 1e-5)
    r = R.rms_inv(_np(k), 1e-5)
    check_f32("dk", float(np.abs(_np(kc.grad) - dk_chain).max()), float(np.abs(_np(kh.grad) * r[..., None]).max()))
