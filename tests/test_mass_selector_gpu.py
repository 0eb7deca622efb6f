"""The per-head chain precision selector against repeated keys it cannot see by construction.

The row-mass pass (lucid_mass_kernel) sums a row's own 64-block exactly and samples the earlier
keys.  These cases place one key direction u (a token repeated, as in the reference's shipped
LUCID model, which runs without RoPE: lucid/config/config.json:31) three times in most 64-blocks,
at row offsets chosen so that no sampled key of any row holding u is a copy of u, and at most
two earlier copies share a row's own block.  The rows holding u then have a true mass
sum_{j<i} P_ij^2 in the hundreds (P ~ 1 between copies) while the sampled estimate stays near 2.
O, V' and every gradient must still meet the bf16 bars against the float64 ground truth.
"""
import pytest
import torch

from bars import check
from oracle import lucid_ref as R

pytestmark = pytest.mark.gpu

OFFS = (1, 9, 17)  # rows of u inside a block


def _sample_offset(blk):
    """Row offset the mass pass samples in every earlier block of query block ``blk``."""
    return (blk * 29) & 63


def _repeat_blocks(T):
    """Blocks holding u: those whose own sample offset is not a row of u, so that a row holding
    u never samples a copy of u (every sampled key of its block sits at that offset)."""
    return [b for b in range(T // 64) if _sample_offset(b) not in OFFS]


def _inputs(T, D, seed, adversarial):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(1, 1, T, D, generator=g)
    k = torch.randn(1, 1, T, D, generator=g)
    v = torch.randn(1, 1, T, D, generator=g) / 8
    do = torch.randn(1, T, 1, D, generator=g)
    if adversarial:
        u = torch.randn(D, generator=g)
        for b in _repeat_blocks(T):
            for o in OFFS:
                k[0, 0, b * 64 + o] = u
    return q, k, v, do


@pytest.mark.parametrize("T,D", [(8192, 64), (4096, 128)])
def test_repeated_keys_hidden_from_the_sample(T, D):
    from lucid_amd import lucid_attention
    from lucid_amd.lucid import _fwd, head_row_mass
    print(f"case mass selector adversarial T={T} D={D}", flush=True)
    q, k, v, do = _inputs(T, D, seed=T + D, adversarial=True)
    # the construction hides u from every sample of a row holding u
    assert all(_sample_offset(b) not in OFFS for b in _repeat_blocks(T))
    qb, kb, vb, dob = (x.to(torch.bfloat16) for x in (q, k, v, do))
    s = D ** -0.5
    # true and sampled row masses
    kd = kb[0, 0].double().cuda()
    kh = kd * torch.rsqrt(kd.pow(2).mean(-1, keepdim=True) + 1e-5)
    p = torch.tril(torch.exp(kh @ kh.T * s - 1 / s), -1)
    true_mass = (p * p).sum(-1).max().item()
    del p
    qc, kc, vc = (x.cuda() for x in (qb, kb, vb))
    _, _, _, ws = _fwd(qc, kc, vc, s, 1e-5, D)
    sampled = head_row_mass(ws, 1, 1, 1, T, D).item()
    print(f"  true max row mass {true_mass:.1f}, sampled {sampled:.2f}", flush=True)
    assert true_mass > 100
    # parity of the whole op
    qg, kg, vg = (x.cuda().requires_grad_() for x in (qb, kb, vb))
    o, vp = lucid_attention(qg, kg, vg, return_vprime=True)
    o.backward(dob.cuda())
    torch.cuda.synchronize()
    ref = R.lucid_group_torch(qb[0].cuda(), kb[0, 0].cuda(), vb[0, 0].cuda(), dob[0].permute(1, 0, 2).cuda(), s)
    errs = {
        "o": ((o[0, :, 0].double() - ref["o"][0]).abs().max().item(), ref["o"].abs().max().item()),
        "vprime": ((vp[0, 0].double() - ref["vp"]).abs().max().item(), ref["vp"].abs().max().item()),
        "dq": ((qg.grad[0, 0].double() - ref["dq"][0]).abs().max().item(), ref["dq"].abs().max().item()),
        "dk": ((kg.grad[0, 0].double() - ref["dk"]).abs().max().item(), ref["dk"].abs().max().item()),
        "dv": ((vg.grad[0, 0].double() - ref["dv"]).abs().max().item(), ref["dv"].abs().max().item()),
    }
    print("  max errors (err, max|ref|):", {n: (f"{e:.2e}", f"{m:.2e}") for n, (e, m) in errs.items()}, flush=True)
    for name, (err, scale) in errs.items():
        check(name, err, scale)
