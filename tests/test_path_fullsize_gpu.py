"""Full-shape LUCID-Path parity on the GPU against the float64 dense oracle (oracle/path_dense.py,
pinned in tests/test_oracle_path_dense.py), evaluated on the GPU one query head at a time:

* config 4 at its full shape, B1 H16 T32768 d64 bf16, forward and backward: O, dq, dk, dv, dw
  and dbeta of every head (16 chains of 512 chunks running at once, the full query transport);
* the reference LUCID-Path model's grouping, 32 query heads over 4 kv heads (G = 8,
  lucid_path/config/config.json:8-9), at T = 4096: the GQA reduction and the first-query-head
  writes of the kv-head operands;
* PaTH softmax attention at config 4's shape, every head.

Inputs follow config 4: q, k, v, w ~ N(0,1) with w L2-normalised per token/head,
beta = 2 sigmoid(N(0,1)), dO ~ N(0,1), scale 1/8; bars as tests/bars.py (bf16 against float64
ground truth on the same bf16-rounded inputs).
"""
import time

import pytest
import torch

from bars import check
from oracle import path_dense as PD

pytestmark = pytest.mark.gpu


def _inputs(B, T, H, G, seed, K=64):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, T, H * G, K, generator=g)
    k = torch.randn(B, T, H, K, generator=g)
    v = torch.randn(B, T, H, K, generator=g)
    w = torch.randn(B, T, H, K, generator=g)
    w = w / w.norm(dim=-1, keepdim=True)
    beta = 2 * torch.sigmoid(torch.randn(B, T, H, generator=g))
    do = torch.randn(B, T, H * G, K, generator=g)
    return [x.to(torch.bfloat16).cuda() for x in (q, k, v, w, beta, do)]


def _run(fn, B, T, H, G, seed, heads=None, softmax=False):
    q, k, v, w, beta, do = _inputs(B, T, H, G, seed)
    leaves = [x.clone().requires_grad_() for x in (q, k, v, w, beta)]
    if softmax:
        o, _ = fn(leaves[0], leaves[1], leaves[2], leaves[3], leaves[4])
    else:
        o, _ = fn(leaves[1], leaves[2], leaves[3], leaves[4], q=leaves[0])
    o.backward(do)
    torch.cuda.synchronize()
    got = [o.detach()] + [x.grad for x in leaves]
    HQ = H * G
    report = {}
    t0 = time.time()
    for hq in (range(HQ) if heads is None else heads):
        h = hq // G
        ref_o, ref_g = PD.path_attention_dense(q[:, :, hq:hq + 1], k[:, :, h:h + 1], v[:, :, h:h + 1],
                                                w[:, :, h:h + 1], beta[:, :, h:h + 1], do=do[:, :, hq:hq + 1],
                                                scale=0.125, softmax=softmax)
        refs = {"o": ref_o[:, :, 0], "dq": ref_g[0][:, :, 0]}
        if G == 1:  # kv-head gradients of one query head only when it is the whole group
            refs.update(dk=ref_g[1][:, :, 0], dv=ref_g[2][:, :, 0], dw=ref_g[3][:, :, 0], dbeta=ref_g[4][:, :, 0])
        mine = {"o": got[0][:, :, hq], "dq": got[1][:, :, hq], "dk": got[2][:, :, h], "dv": got[3][:, :, h],
                "dw": got[4][:, :, h], "dbeta": got[5][:, :, h]}
        for name, r in refs.items():
            err = (mine[name].double() - r).abs().max().item()
            report[(name, hq)] = (err, r.abs().max().item())
        del ref_o, ref_g, refs
        torch.cuda.empty_cache()
    return report, time.time() - t0, (q, k, v, w, beta, do, got)


def _check_all(report):
    worst = {}
    for (name, hq), (err, scale) in report.items():
        if name not in worst or err / max(scale, 1e-30) > worst[name][0] / max(worst[name][1], 1e-30):
            worst[name] = (err, scale, hq)
    print("worst (err, max|ref|, head):", {n: (f"{e:.2e}", f"{s:.2e}", h) for n, (e, s, h) in worst.items()},
          flush=True)
    for (name, hq), (err, scale) in report.items():
        check(f"{name}[head {hq}]", err, scale)


def test_path_config4_full_shape_every_head():
    from lucid_amd.lucid_path import parallel_lucid_path_attention
    print("case path config 4 full shape B=1 T=32768 H=16 G=1", flush=True)
    report, secs, _ = _run(parallel_lucid_path_attention, 1, 32768, 16, 1, seed=4)
    print(f"oracle {secs:.1f} s for 16 heads", flush=True)
    _check_all(report)


def test_path_reference_model_grouping_g8():
    """HQ 32 over H 4 (G = 8) at T = 4096: every query head's O and dq, and the kv-head
    gradients summed over each group of eight."""
    from lucid_amd.lucid_path import parallel_lucid_path_attention
    B, T, H, G = 1, 4096, 4, 8
    print(f"case path G=8 B={B} T={T} H={H} HQ={H * G}", flush=True)
    report, _, (q, k, v, w, beta, do, got) = _run(parallel_lucid_path_attention, B, T, H, G, seed=48)
    _check_all(report)
    _, grads = PD.path_attention_dense(q, k, v, w, beta, do=do, scale=0.125)
    for name, mine, ref in zip(("dk", "dv", "dw", "dbeta"), got[2:], grads[1:]):
        check(name, (mine.double() - ref).abs().max().item(), ref.abs().max().item())


def test_path_softmax_config4_shape():
    from lucid_amd.lucid_path import parallel_path_attention
    print("case PaTH softmax config 4 shape B=1 T=32768 H=16", flush=True)
    report, secs, _ = _run(parallel_path_attention, 1, 32768, 16, 1, seed=5, softmax=True)
    print(f"oracle {secs:.1f} s for 16 heads", flush=True)
    _check_all(report)
