"""Pins the float64 LUCID oracle (oracle/lucid_ref.py) before it is trusted as the checker.

The reference ships no tests, golden vectors or fixtures for this path, so each
oracle function is pinned here by closed forms, invariants, an independent
restatement from another reference file and float64 autograd.  Every check is
chosen so that a plausible mistake (wrong sign of the -1/s offset, a missing
scale, using K^ instead of raw K in the softmax, a transposed solve) fails it.
"""
import math

import numpy as np
import pytest
import scipy.linalg as sla
import torch

from oracle import lucid_ref as R


def _rand(shape, seed, scale=1.0):
    return np.random.default_rng(seed).standard_normal(shape) * scale


def test_t1_closed_form():
    # T = 1: V' = V / P_00 with P_00 = exp(s d ms/(ms+eps) - 1/s)  (non-unit diagonal)
    d, eps = 64, 1e-5
    k = _rand((1, 1, 1, d), 0, 0.05)
    v = _rand((1, 1, 1, d), 1)
    s = d ** -0.5
    ms = np.mean(k * k)
    p00 = math.exp(s * d * ms / (ms + eps) - 1 / s)
    assert p00 < 1.0  # eps makes the diagonal strictly below one
    np.testing.assert_allclose(R.vprime_dense(k, v, s, eps), v / p00, rtol=1e-13)


def test_identical_keys_first_difference():
    # All keys equal: P_ij = c for every j <= i, so V'_0 = V_0 / c and V'_i = (V_i - V_{i-1}) / c.
    t, d, eps = 17, 32, 1e-5
    row = _rand((d,), 2)
    k = np.broadcast_to(row, (1, 1, t, d)).copy()
    v = _rand((1, 1, t, d), 3)
    s = d ** -0.5
    ms = np.mean(row * row)
    c = math.exp(s * d * ms / (ms + eps) - 1 / s)
    expect = np.empty_like(v)
    expect[..., 0, :] = v[..., 0, :] / c
    expect[..., 1:, :] = (v[..., 1:, :] - v[..., :-1, :]) / c
    np.testing.assert_allclose(R.vprime_dense(k, v, s, eps), expect, rtol=1e-10, atol=1e-12)


def test_orthogonal_keys_diagonal():
    # Mutually orthogonal keys: P_ij = exp(-1/s) for j < i; with d large this is ~e^-8 off the diagonal.
    d, eps = 64, 1e-5
    k = np.eye(d)[None, None, :8] * 3.0
    v = _rand((1, 1, 8, d), 4)
    s = d ** -0.5
    p = R.precond_matrix(R.k_hat(k, eps)[0, 0], s)
    off = p[np.tril_indices(8, -1)]
    np.testing.assert_allclose(off, math.exp(-8.0), rtol=1e-12)
    vp = R.vprime_dense(k, v, s, eps)
    np.testing.assert_allclose(p @ vp[0, 0], v[0, 0], atol=1e-12)


@pytest.mark.parametrize("t,hkv,g", [(64, 1, 1), (96, 2, 2), (128, 1, 4)])
def test_solve_residual_and_bounds(t, hkv, g):
    d, eps = 64, 1e-5
    k = _rand((2, hkv, t, d), 5, 0.125)
    v = _rand((2, hkv, t, d), 6, 0.125)
    s = d ** -0.5
    vp = R.vprime_dense(k, v, s, eps)
    kh = R.k_hat(k, eps)
    for b in range(2):
        for h in range(hkv):
            p = R.precond_matrix(kh[b, h], s)
            assert np.all(p <= 1.0 + 1e-12) and np.all(p >= 0)  # Cauchy-Schwarz: s K^i.K^j <= s d = 1/s
            res = np.linalg.norm(p @ vp[b, h] - v[b, h]) / np.linalg.norm(v[b, h])
            assert res < 1e-12


@pytest.mark.parametrize("bs", [8, 16, 32, 64])
def test_blockwise_equals_dense(bs):
    t, d, eps = 128, 64, 1e-5
    k = _rand((1, 2, t, d), 7, 0.125)
    v = _rand((1, 2, t, d), 8, 0.125)
    s = d ** -0.5
    np.testing.assert_allclose(R.vprime_blockwise(k, v, s, eps, bs), R.vprime_dense(k, v, s, eps),
                               rtol=1e-10, atol=1e-12)


def test_against_unit_diagonal_restatement():
    # experiment1_cumavg.py:188-202 states the same preconditioner with a unit diagonal
    # (solve_triangular(..., unitriangular=True)).  With eps -> 0 the LUCID diagonal
    # exp(s d ms/(ms+eps) - 1/s) -> 1, so both statements must agree.
    t, d = 48, 16
    k = torch.from_numpy(_rand((1, 1, t, d), 9))
    v = torch.from_numpy(_rand((1, 1, t, d), 10))
    k_rms = k * torch.rsqrt(k.pow(2).mean(-1, keepdim=True))
    kkt = k_rms @ k_rms.transpose(-2, -1) / math.sqrt(d) - math.sqrt(d)
    mask = torch.triu(torch.ones(t, t), diagonal=1).bool()
    kkt = torch.exp(kkt.masked_fill(mask, -float("inf")))
    v_unit = torch.linalg.solve_triangular(kkt, v, upper=False, unitriangular=True).numpy()
    np.testing.assert_allclose(R.vprime_dense(k.numpy(), v.numpy(), d ** -0.5, 1e-14), v_unit,
                               rtol=1e-9, atol=1e-11)


def test_attention_matches_sdpa_and_first_row():
    t, d, g = 40, 32, 2
    q = _rand((1, 2 * g, t, d), 11)
    k = _rand((1, 2, t, d), 12)
    v = _rand((1, 2, t, d), 13)
    s = d ** -0.5
    o, vp = R.lucid_attention(q, k, v, s, 1e-5)
    # row 0 attends only to key 0 -> O_0 = V'_0 of its kv head
    for hq in range(2 * g):
        np.testing.assert_allclose(o[0, 0, hq], vp[0, hq // g, 0], rtol=1e-12)
    # library routine (torch SDPA, float64) on the oracle's V'
    ref = torch.nn.functional.scaled_dot_product_attention(
        torch.from_numpy(q), torch.from_numpy(np.repeat(k, g, 1)), torch.from_numpy(np.repeat(vp, g, 1)),
        is_causal=True, scale=s).transpose(1, 2).numpy()
    np.testing.assert_allclose(o, ref, rtol=1e-10, atol=1e-12)
    # raw K (not K^) feeds the softmax: a per-row rescale of K must change O
    o2, _ = R.lucid_attention(q, 2.0 * k, v, s, 1e-5)
    assert np.abs(o2 - o).max() > 1e-3


def test_torch_restatement_matches_numpy():
    t, d, g = 64, 32, 2
    q = _rand((2, 2 * g, t, d), 14)
    k = _rand((2, 2, t, d), 15, 0.3)
    v = _rand((2, 2, t, d), 16)
    o, vp = R.lucid_attention(q, k, v)
    ot, vpt = R.lucid_attention_torch(*(torch.from_numpy(x) for x in (q, k, v)))
    np.testing.assert_allclose(vpt.numpy(), vp, rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(ot.numpy(), o, rtol=1e-10, atol=1e-12)


def test_torch_restatement_gradcheck():
    t, d = 12, 8
    gen = torch.Generator().manual_seed(0)
    q = torch.randn(1, 2, t, d, generator=gen, dtype=torch.float64, requires_grad=True)
    k = torch.randn(1, 1, t, d, generator=gen, dtype=torch.float64, requires_grad=True)
    v = torch.randn(1, 1, t, d, generator=gen, dtype=torch.float64, requires_grad=True)
    assert torch.autograd.gradcheck(lambda a, b, c: R.lucid_attention_torch(a, b, c)[0], (q, k, v))


@pytest.mark.parametrize("t,hkv,g", [(32, 1, 1), (48, 2, 2)])
def test_closed_form_grads_match_autograd(t, hkv, g):
    d = 16
    q = _rand((2, hkv * g, t, d), 17)
    k = _rand((2, hkv, t, d), 18, 0.5)
    v = _rand((2, hkv, t, d), 19)
    do = _rand((2, t, hkv * g, d), 20)
    dq, dk, dv = R.lucid_attention_grads(q, k, v, do)
    qt, kt, vt = (torch.from_numpy(x).requires_grad_() for x in (q, k, v))
    o, _ = R.lucid_attention_torch(qt, kt, vt)
    (o * torch.from_numpy(do)).sum().backward()
    np.testing.assert_allclose(dq, qt.grad.numpy(), rtol=1e-9, atol=1e-11)
    np.testing.assert_allclose(dk, kt.grad.numpy(), rtol=1e-9, atol=1e-11)
    np.testing.assert_allclose(dv, vt.grad.numpy(), rtol=1e-9, atol=1e-11)


@pytest.mark.parametrize("bs", [8, 16])
def test_blockwise_backward_equals_dense(bs):
    t, d, eps = 64, 16, 1e-5
    k = _rand((t, d), 21, 0.5)
    kh = R.k_hat(k, eps)
    v = _rand((t, d), 22)
    s = d ** -0.5
    p = R.precond_matrix(kh, s)
    vp = sla.solve_triangular(p, v, lower=True)
    dvp = _rand((t, d), 23)
    dkh, dv = R.precond_backward(kh, vp, dvp, s)
    dkh_b, dv_b = R.precond_backward_blockwise(kh, vp, dvp, s, bs)
    np.testing.assert_allclose(dv_b, dv, rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(dkh_b, dkh, rtol=1e-10, atol=1e-12)


def test_rmsnorm_backward_matches_autograd():
    k = torch.from_numpy(_rand((5, 16), 24)).requires_grad_()
    dkh = _rand((5, 16), 25)
    kh = k * torch.rsqrt(k.pow(2).mean(-1, keepdim=True) + 1e-5)
    (kh * torch.from_numpy(dkh)).sum().backward()
    np.testing.assert_allclose(R.rmsnorm_backward(k.detach().numpy(), dkh, 1e-5), k.grad.numpy(),
                               rtol=1e-11, atol=1e-13)


def test_chain_block_coupling_identity():
    """The forward chain solves each 128-row block as V'_A = X_A R_A and
    V'_B = X_B R_B + Z V'_A with Z = -(X_B P_BA) precomputed (X = inverse of a 64x64
    diagonal block of P).  This pins that identity against a direct triangular solve of
    P's real 128x128 diagonal block, and its transpose form (dV_A = X_A^T R_A + W dV_B,
    W = -(X_A^T P_BA^T)) used by the backward column chain; a wrong sign, block or
    transpose fails it."""
    t, d, eps = 128, 64, 1e-5
    k = _rand((1, 1, t, d), 21, 0.125)[0, 0]
    r = _rand((1, 1, t, d), 22, 1.0)[0, 0]
    s = d ** -0.5
    p = R.precond_matrix(R.k_hat(k[None, None], eps)[0, 0], s)
    pa, pb, pba = p[:64, :64], p[64:, 64:], p[64:, :64]
    xa, xb = np.linalg.inv(pa), np.linalg.inv(pb)
    direct = sla.solve_triangular(p, r, lower=True)
    va = xa @ r[:64]
    z = -(xb @ pba)
    vb = xb @ r[64:] + z @ va
    np.testing.assert_allclose(np.concatenate([va, vb]), direct, rtol=1e-10, atol=1e-12)
    # the transposed (backward) solve P^T dV = R, last block first
    direct_t = sla.solve_triangular(p.T, r, lower=False)
    dvb = xb.T @ r[64:]
    w = -(xa.T @ pba.T)
    dva = xa.T @ r[:64] + w @ dvb
    np.testing.assert_allclose(np.concatenate([dva, dvb]), direct_t, rtol=1e-10, atol=1e-12)


@pytest.mark.parametrize("t,g", [(48, 1), (40, 3)])
def test_group_torch_matches_numpy_closed_forms(t, g):
    """lucid_group_torch (the full-size GPU ground truth) equals the numpy oracle, forward and
    gradients, for one kv head with g query heads; a missing GQA sum or transposed solve fails."""
    d = 16
    q = _rand((1, g, t, d), 26)
    k = _rand((1, 1, t, d), 27, 0.7)
    v = _rand((1, 1, t, d), 28)
    do = _rand((1, t, g, d), 29)
    o, vp = R.lucid_attention(q, k, v)
    dq, dk, dv = R.lucid_attention_grads(q, k, v, do)
    out = R.lucid_group_torch(torch.from_numpy(q[0]), torch.from_numpy(k[0, 0]), torch.from_numpy(v[0, 0]),
                              torch.from_numpy(do[0].transpose(1, 0, 2).copy()))
    np.testing.assert_allclose(out["vp"].numpy(), vp[0, 0], rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(out["o"].numpy(), o[0].transpose(1, 0, 2), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(out["dq"].numpy(), dq[0], rtol=1e-9, atol=1e-11)
    np.testing.assert_allclose(out["dk"].numpy(), dk[0, 0], rtol=1e-9, atol=1e-11)
    np.testing.assert_allclose(out["dv"].numpy(), dv[0, 0], rtol=1e-9, atol=1e-11)


def test_unit_variance_inputs_reject_scale_and_gradient_mistakes():
    """The GPU parity cases with unit-variance q and k put s q.k at O(1), so the softmax is far
    from uniform: there a doubled softmax scale moves O, and a halved dQ or dK misses, by more
    than the relative bar (2e-2 of max |ref|) -- unlike N(0,1)/sqrt(d) inputs, whose near-uniform
    softmax hides such mistakes."""
    t, d = 256, 64
    q = _rand((1, 1, t, d), 30)
    k = _rand((1, 1, t, d), 31)
    v = _rand((1, 1, t, d), 32, 0.125)
    do = _rand((1, t, 1, d), 33)
    s = d ** -0.5
    o, vp = R.lucid_attention(q, k, v, s)
    o2, _ = R.causal_attention(q, k, vp, 2 * s)
    assert np.abs(o2 - o).max() > 2e-2 * np.abs(o).max()
    dq, dk, _ = R.lucid_attention_grads(q, k, v, do, s)
    for ref in (dq, dk):
        assert np.abs(0.5 * ref - ref).max() > 2e-2 * np.abs(ref).max()
    # the same mistake hides under the small-score inputs at the absolute bar
    qs, ks = q / 8, k / 8
    o_s, vp_s = R.lucid_attention(qs, ks, v, s)
    o2_s, _ = R.causal_attention(qs, ks, vp_s, 2 * s)
    assert np.abs(o2_s - o_s).max() < 2e-2
