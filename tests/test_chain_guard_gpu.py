"""Bounded chain waits on the GPU, forced from the host: with a wait limit of 1 us (a chain
hand-off takes microseconds to tens of microseconds) waits give up, every kernel still
finishes, and the give-up is reported as RuntimeError; with the limit restored the same call
is correct again.  No wait is left unbounded, so nothing can hang."""
import pytest
import torch

from bars import check

pytestmark = pytest.mark.gpu


def _restore(lib, setter, status):
    setter(2.0)
    torch.cuda.synchronize()
    status()  # drop any flag left by the forced run


def test_lucid_chain_give_up_is_reported_and_recovers():
    from lucid_amd import _lib, lucid_attention
    lib = _lib.load()
    g = torch.Generator().manual_seed(3)
    q, k, v = ((torch.randn(1, 2, 16384, 64, generator=g) / 8).to(torch.bfloat16).cuda() for _ in range(3))
    print("case chain give-up lucid", flush=True)
    ref = lucid_attention(q, k, v)
    _lib.chain_status()
    assert lib.lucid_set_chain_wait_limit(1e-6) == 0
    try:
        lucid_attention(q, k, v)
        torch.cuda.synchronize()
        with pytest.raises(RuntimeError, match="chain wait gave up"):
            _lib.chain_status()
    finally:
        _restore(lib, lib.lucid_set_chain_wait_limit, lib.lucid_chain_status)
    again = lucid_attention(q, k, v)
    _lib.chain_status()
    check("o after recovery", float((again.float() - ref.float()).abs().max()), float(ref.float().abs().max()))


def test_path_chain_give_up_is_reported_and_recovers():
    from lucid_amd import _lib
    from lucid_amd.lucid_path import parallel_lucid_path_attention
    lib = _lib.load("liblucid_path.so")
    g = torch.Generator().manual_seed(4)
    T, H = 4096, 2
    q, k, v, w = (torch.randn(1, T, H, 64, generator=g) for _ in range(4))
    w = w / w.norm(dim=-1, keepdim=True)
    beta = 2 * torch.sigmoid(torch.randn(1, T, H, generator=g))
    q, k, v, w, beta = (x.to(torch.bfloat16).cuda() for x in (q, k, v, w, beta))
    print("case chain give-up path", flush=True)
    ref, _ = parallel_lucid_path_attention(k, v, w, beta, q=q)
    _lib.chain_status()
    assert lib.lucid_path_set_chain_wait_limit(1e-6) == 0
    try:
        parallel_lucid_path_attention(k, v, w, beta, q=q)
        torch.cuda.synchronize()
        with pytest.raises(RuntimeError, match="chain wait gave up"):
            _lib.chain_status()
    finally:
        _restore(lib, lib.lucid_path_set_chain_wait_limit, lib.lucid_path_chain_status)
    again, _ = parallel_lucid_path_attention(k, v, w, beta, q=q)
    _lib.chain_status()
    check("o after recovery", float((again.float() - ref.float()).abs().max()), float(ref.float().abs().max()))
