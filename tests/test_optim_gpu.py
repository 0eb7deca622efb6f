"""GPU parity of lucid_amd.optim.AdamW (one HIP pass per step) against torch.optim.AdamW, the
optimizer of the reference's Trainer runs (run_clm_chunk.py:776):

    fp32 parameters: max |ours - torch| <= 1e-6 * max |p| after several steps (fp32 rounding
    of the same update; torch's single-tensor loop is the reference)
    bf16 parameters and states: within two bf16 ulps of torch's fused bf16 kernel per element
    (of the larger of the two values: an update below half an ulp can round either way, and
    a value at a binade edge has the coarser ulp on one side; plus a floor at the scale of
    the steps for values that cancel to ~0), and on average no further than torch's kernel
    from the fp32 update

Tensor sizes cover the 8-element vector path, scalar tails, empty tensors, more tensors than
one launch holds (48), and parameters without gradients.
"""
import pytest
import torch

from lucid_amd.optim import AdamW

pytestmark = pytest.mark.gpu

SIZES = [(1000003,), (7,), (3, 2048), (0,), (64, 33), (129,)] + [(17 + i,) for i in range(50)]


def _params(dtype, seed):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(*s, generator=g).to(dtype).cuda() for s in SIZES]


def _run(opt_cls, params, grads_per_step, **kw):
    ps = [torch.nn.Parameter(p.clone()) for p in params]
    opt = opt_cls(ps, **kw)
    for grads in grads_per_step:
        for p, gr in zip(ps, grads):
            p.grad = None if gr is None else gr.clone()
        opt.step()
    torch.cuda.synchronize()
    return ps, opt


def _grads(dtype, steps, seed):
    g = torch.Generator().manual_seed(seed)
    out = []
    for _ in range(steps):
        gs = [torch.randn(*s, generator=g).to(dtype).cuda() for s in SIZES]
        gs[5] = None  # a parameter without a gradient is left alone
        out.append(gs)
    return out


def test_adamw_fp32_matches_torch():
    print("case adamw fp32", flush=True)
    kw = dict(lr=3e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)
    params, grads = _params(torch.float32, 0), _grads(torch.float32, 5, 1)
    ours, opt = _run(AdamW, params, grads, **kw)
    ref, ropt = _run(torch.optim.AdamW, params, grads, foreach=False, **kw)
    for a, b, p0 in zip(ours, ref, params):
        if p0.numel():
            err = (a.detach() - b.detach()).abs().max().item()
            assert err <= 1e-6 * max(1.0, p0.abs().max().item()), err
    assert torch.equal(ours[5].detach(), params[5])
    # the state dict has torch's layout: torch's optimizer resumes from it
    sd = opt.state_dict()
    ropt2 = torch.optim.AdamW([torch.nn.Parameter(p.detach().clone()) for p in ours], foreach=False, **kw)
    ropt2.load_state_dict(sd)
    st = ropt2.state[ropt2.param_groups[0]["params"][0]]
    assert int(st["step"]) == 5 and st["exp_avg"].shape == params[0].shape


def test_adamw_bf16_matches_torch_fused():
    print("case adamw bf16", flush=True)
    kw = dict(lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01)
    params, grads = _params(torch.bfloat16, 2), _grads(torch.bfloat16, 4, 3)
    ours, opt = _run(AdamW, params, grads, **kw)
    ref, ropt = _run(torch.optim.AdamW, params, grads, fused=True, **kw)
    exact, eopt = _run(torch.optim.AdamW, [p.float() for p in params],
                    [[None if g is None else g.float() for g in gs] for gs in grads], foreach=False, **kw)
    floor = 2.0 ** -6 * 4 * kw["lr"]  # values that cancel to ~0 were rounded at the scale of the steps
    # summed |error| against the fp32 update, ours and torch's bf16 kernel, over every tensor
    err = {"param": [0.0, 0.0], "exp_avg": [0.0, 0.0], "exp_avg_sq": [0.0, 0.0]}
    for a, b, e in zip(ours, ref, exact):
        a, b, e = a.detach().float(), b.detach().float(), e.detach().float()
        assert bool(((a - b).abs() <= 2.0 ** -6 * torch.maximum(a.abs(), b.abs()) + floor).all()), \
            (a - b).abs().max().item()
        err["param"][0] += (a - e).abs().sum().item()
        err["param"][1] += (b - e).abs().sum().item()
    for p_o, p_r, p_e in zip(ours, ref, exact):
        so, sr, se = opt.state.get(p_o), ropt.state.get(p_r), eopt.state.get(p_e)
        if not so or not p_o.numel():
            continue
        for key in ("exp_avg", "exp_avg_sq"):
            x, y, z = so[key].float(), sr[key].float(), se[key].float()
            # a moment that cancels to ~0 carries the roundings of its earlier, larger values
            fl = 2.0 ** -7 * y.abs().max().item()
            assert bool(((x - y).abs() <= 2.0 ** -6 * torch.maximum(x.abs(), y.abs()) + fl).all()), key
            err[key][0] += (x - z).abs().sum().item()
            err[key][1] += (y - z).abs().sum().item()
    print({k: (f"{v[0]:.4e}", f"{v[1]:.4e}") for k, v in err.items()}, flush=True)
    for key, (e_ours, e_torch) in err.items():  # no less accurate than torch's own bf16 kernel
        assert e_ours <= 1.05 * e_torch, (key, e_ours, e_torch)


def test_adamw_refuses_amsgrad_groups_from_torch_state_dicts():
    p = torch.nn.Parameter(torch.randn(16, device="cuda"))
    p.grad = torch.randn(16, device="cuda")
    opt = AdamW([p])
    sd = torch.optim.AdamW([torch.nn.Parameter(torch.randn(16, device="cuda"))], amsgrad=True).state_dict()
    opt.load_state_dict(sd)
    with pytest.raises(ValueError):
        opt.step()


def test_adamw_rejects_cpu_and_fp16_parameters():
    p = torch.nn.Parameter(torch.randn(8))
    p.grad = torch.randn(8)
    with pytest.raises(TypeError):
        AdamW([p]).step()
    q = torch.nn.Parameter(torch.randn(8, dtype=torch.float16, device="cuda"))
    q.grad = torch.randn(8, dtype=torch.float16, device="cuda")
    with pytest.raises(TypeError):
        AdamW([q]).step()


def test_adamw_skips_empty_and_gradless_parameters():
    empty = torch.nn.Parameter(torch.zeros(0, device="cuda"))
    empty.grad = torch.zeros(0, device="cuda")
    idle = torch.nn.Parameter(torch.ones(8, device="cuda"))
    opt = AdamW([empty, idle], lr=0.1)
    opt.step()
    torch.cuda.synchronize()
    assert bool((idle.detach() == 1).all()) and idle not in opt.state
    assert int(opt.state[empty]["step"]) == 1
