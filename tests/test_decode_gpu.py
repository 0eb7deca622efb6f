"""GPU parity of the LUCID decoding step (lucid_amd.lucid.lucid_decode).

Decode parity is defined mathematically: a token decoded against the (K, V') cache of
the earlier tokens must reproduce the same row of the full-sequence forward (P has a
non-unit diagonal, modeling_lucid.py:565-569, which the step keeps).  Each case checks
the decoded O and V' rows against the float64 oracle of the whole sequence
(``oracle.lucid_ref.lucid_attention``) and against the HIP prefill of the whole sequence.
Tolerance: max |x - ref| <= 2e-2 (bf16 against float64 on the same bf16 inputs).
"""
import pytest
import torch

from oracle import lucid_ref as R

pytestmark = pytest.mark.gpu

TOL = 2e-2


def _inputs(B, Hq, Hkv, T, D, seed):
    g = torch.Generator().manual_seed(seed)
    s = D ** -0.5
    q = (torch.randn(B, Hq, T, D, generator=g) * s).to(torch.bfloat16)
    k = (torch.randn(B, Hkv, T, D, generator=g) * s).to(torch.bfloat16)
    v = (torch.randn(B, Hkv, T, D, generator=g) * s).to(torch.bfloat16)
    return q, k, v


def _decode_tail(q, k, v, t0, cap):
    """Prefill rows [0, t0) with the fused op, then decode rows t0.. one at a time."""
    from lucid_amd import lucid_attention, lucid_decode
    B, Hkv, T, D = k.shape
    kc = torch.zeros(B, Hkv, cap, D, dtype=torch.bfloat16, device="cuda")
    vc = torch.zeros_like(kc)
    if t0 > 0:
        _, vp0 = lucid_attention(q[:, :, :t0], k[:, :, :t0], v[:, :, :t0], return_vprime=True)
        kc[:, :, :t0] = k[:, :, :t0]
        vc[:, :, :t0] = vp0.to(torch.bfloat16)
    outs, vps = [], []
    for t in range(t0, T):
        o, vp = lucid_decode(q[:, :, t:t + 1], k[:, :, t:t + 1], v[:, :, t:t + 1], kc, vc, t)
        outs.append(o)
        vps.append(vp)
    torch.cuda.synchronize()
    return torch.cat(outs, 1), torch.cat(vps, 2), kc, vc


@pytest.mark.parametrize("B,Hq,Hkv,T0,n,D", [(2, 4, 2, 300, 3, 64), (1, 8, 1, 1000, 2, 128), (1, 2, 2, 0, 5, 64),
                                            (1, 4, 4, 130, 2, 64), (2, 4, 1, 77, 2, 128)])
def test_decode_rows_match_oracle_and_prefill(B, Hq, Hkv, T0, n, D):
    from lucid_amd import lucid_attention
    T = T0 + n
    q, k, v = _inputs(B, Hq, Hkv, T, D, seed=T0 + n + D)
    print(f"case decode B={B} Hq={Hq} Hkv={Hkv} T0={T0} n={n} D={D}", flush=True)
    qc, kc_, vc_ = q.cuda(), k.cuda(), v.cuda()
    o_dec, vp_dec, kcache, vcache = _decode_tail(qc, kc_, vc_, T0, T + 7)
    o_ref, vp_ref = R.lucid_attention(q.double().numpy(), k.double().numpy(), v.double().numpy())
    o_ref, vp_ref = torch.from_numpy(o_ref), torch.from_numpy(vp_ref)
    err_o = (o_dec.cpu().double() - o_ref[:, T0:]).abs().max().item()
    err_v = (vp_dec.cpu().double() - vp_ref[:, :, T0:]).abs().max().item()
    assert err_o <= TOL and err_v <= TOL, f"O err {err_o:.3e}, V' err {err_v:.3e}"
    # against the HIP prefill of the whole sequence, and the cache holds the appended rows
    o_full, vp_full = lucid_attention(qc, kc_, vc_, return_vprime=True)
    torch.cuda.synchronize()
    assert (o_dec.float() - o_full[:, T0:].float()).abs().max().item() <= TOL
    assert (vp_dec - vp_full[:, :, T0:]).abs().max().item() <= TOL
    assert torch.equal(kcache[:, :, :T], kc_)
    assert (vcache[:, :, T0:T].float() - vp_dec).abs().max().item() <= 1e-2 * max(1.0, vp_dec.abs().max().item())


def test_decode_long_cache_matches_prefill():
    """T = 20000 cached rows (the split path with many splits): decoded rows against the
    HIP prefill of the whole sequence."""
    from lucid_amd import lucid_attention
    B, Hq, Hkv, T0, n, D = 1, 4, 2, 20000, 2, 64
    q, k, v = _inputs(B, Hq, Hkv, T0 + n, D, seed=9)
    print(f"case decode long T0={T0}", flush=True)
    qc, kc_, vc_ = q.cuda(), k.cuda(), v.cuda()
    o_dec, vp_dec, _, _ = _decode_tail(qc, kc_, vc_, T0, T0 + n)
    o_full, vp_full = lucid_attention(qc, kc_, vc_, return_vprime=True)
    torch.cuda.synchronize()
    assert (o_dec.float() - o_full[:, T0:].float()).abs().max().item() <= TOL
    assert (vp_dec - vp_full[:, :, T0:]).abs().max().item() <= TOL


def test_decode_rejects_full_cache():
    from lucid_amd import lucid_decode
    q, k, v = (x.cuda() for x in _inputs(1, 2, 2, 1, 64, seed=1))
    kc = torch.zeros(1, 2, 4, 64, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError, match="cache is too small"):
        lucid_decode(q, k, v, kc, kc.clone(), 4)
    # several tokens must fit as a whole: 3 new rows after 2 cached ones do not fit 4 rows
    q, k, v = (x.cuda() for x in _inputs(1, 2, 2, 3, 64, seed=2))
    with pytest.raises(ValueError, match="cache is too small"):
        lucid_decode(q, k, v, kc, kc.clone(), 2)


@pytest.mark.parametrize("B,Hq,Hkv,T0,n,D", [
    (1, 4, 4, 300, 20, 64),    # G = 1: 16 tokens per pass, two passes
    (2, 8, 2, 130, 13, 64),    # G = 4: 6 tokens per pass, three passes (the last one token)
    (1, 8, 1, 1000, 7, 128),   # G = 8: 3 tokens per pass
    (1, 4, 2, 0, 9, 64),       # empty cache: the first pass has no split partials
    (1, 2, 1, 77, 5, 68),      # a padded head dim
    # groupings without their own instance: the generic one (group size at run time)
    (1, 6, 2, 200, 10, 64),    # G = 3: 8 tokens per pass
    (1, 12, 2, 65, 5, 128),    # G = 6: 4 tokens per pass
    (2, 12, 1, 300, 4, 64),    # G = 12: 2 tokens per pass
    (1, 40, 1, 129, 3, 64),    # G = 40: two chunks of 20 query heads, 1 token per pass
    (2, 64, 2, 70, 2, 68),     # G = 32 (multi-query with 32 heads per kv head): chunks of 16
    (1, 33, 1, 90, 2, 64),     # G = 33: chunks of 17 and 16 with the passes of the larger
])
def test_decode_several_tokens_in_one_call(B, Hq, Hkv, T0, n, D):
    """n new tokens in one call (get_new_v_prime with L_k = n): every decoded O and V' row
    equals the float64 oracle's row of the whole sequence, i.e. the new tokens are coupled to
    the cache and to each other, and attend causally among themselves."""
    from lucid_amd import lucid_attention, lucid_decode
    from lucid_amd.lucid import _padded_dim
    T = T0 + n
    q, k, v = _inputs(B, Hq, Hkv, T, D, seed=11 * T0 + n + D)
    print(f"case decode tokens B={B} Hq={Hq} Hkv={Hkv} T0={T0} n={n} D={D}", flush=True)
    qc, kc_, vc_ = q.cuda(), k.cuda(), v.cuda()
    dp = _padded_dim(D)
    kc = torch.zeros(B, Hkv, T + 3, dp, dtype=torch.bfloat16, device="cuda")
    vc = torch.zeros_like(kc)
    if T0 > 0:
        _, vp0 = lucid_attention(qc[:, :, :T0], kc_[:, :, :T0], vc_[:, :, :T0], return_vprime=True)
        kc[:, :, :T0, :D] = kc_[:, :, :T0]
        vc[:, :, :T0, :D] = vp0.to(torch.bfloat16)
    o_dec, vp_dec = lucid_decode(qc[:, :, T0:], kc_[:, :, T0:], vc_[:, :, T0:], kc, vc, T0)
    torch.cuda.synchronize()
    assert o_dec.shape == (B, n, Hq, D) and vp_dec.shape == (B, Hkv, n, D)
    o_ref, vp_ref = R.lucid_attention(q.double().numpy(), k.double().numpy(), v.double().numpy(), D ** -0.5, 1e-5)
    o_ref, vp_ref = torch.from_numpy(o_ref), torch.from_numpy(vp_ref)
    err_o = (o_dec.cpu().double() - o_ref[:, T0:]).abs().max().item()
    err_v = (vp_dec.cpu().double() - vp_ref[:, :, T0:]).abs().max().item()
    print(f"  o err {err_o:.2e} vprime err {err_v:.2e}", flush=True)
    assert err_o <= TOL and err_v <= TOL, f"O err {err_o:.3e}, V' err {err_v:.3e}"
    assert torch.equal(kc[:, :, T0:T, :D], kc_[:, :, T0:])
    assert (vc[:, :, T0:T, :D].float() - vp_dec).abs().max().item() <= 1e-2 * max(1.0, vp_dec.abs().max().item())
    # one call equals the same tokens decoded one at a time
    kc1 = torch.zeros_like(kc)
    vc1 = torch.zeros_like(vc)
    kc1[:, :, :T0], vc1[:, :, :T0] = kc[:, :, :T0], vc[:, :, :T0]
    outs = [lucid_decode(qc[:, :, t:t + 1], kc_[:, :, t:t + 1], vc_[:, :, t:t + 1], kc1, vc1, t)[0]
            for t in range(T0, T)]
    torch.cuda.synchronize()
    assert (torch.cat(outs, 1).float() - o_dec.float()).abs().max().item() <= TOL
