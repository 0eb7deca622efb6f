"""AdamW on one HIP kernel pass per step (``lucid_adamw_step``).

The reference trains through the HF ``Trainer`` (``run_clm_chunk.py:776``), whose default
optimizer is ``torch.optim.AdamW``.  :class:`AdamW` is a drop-in for it on GPU parameters
(bf16 or fp32, with states in the parameter dtype as torch keeps them): the update of every
parameter tensor -- weight decay, both moment updates and the bias-corrected step -- is one
read of (p, grad, exp_avg, exp_avg_sq) and one write of (p, exp_avg, exp_avg_sq), in fp32,
up to 48 tensors per launch.  Same hyper-parameters, defaults and state-dict layout
(``step``, ``exp_avg``, ``exp_avg_sq`` per parameter) as ``torch.optim.AdamW``; no amsgrad,
no maximize, no sparse or complex parameters (they raise).
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib

_DTYPES = {torch.bfloat16: 0, torch.float32: 1}


class AdamW(torch.optim.Optimizer):
    def __init__(self, params, lr: float = 1e-3, betas=(0.9, 0.999), eps: float = 1e-8,
                 weight_decay: float = 1e-2):
        if not 0.0 <= lr:
            raise ValueError(f"Invalid learning rate: {lr}")
        if not 0.0 <= eps:
            raise ValueError(f"Invalid epsilon value: {eps}")
        if not 0.0 <= betas[0] < 1.0 or not 0.0 <= betas[1] < 1.0:
            raise ValueError(f"Invalid beta parameters: {betas}")
        if not 0.0 <= weight_decay:
            raise ValueError(f"Invalid weight_decay value: {weight_decay}")
        super().__init__(params, dict(lr=lr, betas=betas, eps=eps, weight_decay=weight_decay))

    @torch.no_grad()
    def step(self, closure=None):
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        lib = _lib.load()
        for group in self.param_groups:
            # groups loaded from a torch.optim.AdamW state dict carry its flags: refuse the
            # variants this update does not implement rather than ignore them
            if group.get("amsgrad") or group.get("maximize"):
                raise ValueError("lucid_amd.optim.AdamW: amsgrad and maximize are not supported")
            # one C call per (device, dtype, step count): the bias corrections are per call
            batches: dict[tuple, list] = {}
            for p in group["params"]:
                if p.grad is None:
                    continue
                g = p.grad
                if g.is_sparse or p.is_complex():
                    raise RuntimeError("lucid_amd.optim.AdamW: sparse and complex parameters are not supported")
                if not p.is_cuda or p.dtype not in _DTYPES:
                    raise TypeError(f"lucid_amd.optim.AdamW: bf16 or fp32 GPU parameters, got {p.dtype} on {p.device}")
                if not p.is_contiguous():
                    raise ValueError("lucid_amd.optim.AdamW: parameters must be contiguous")
                if g.dtype != p.dtype:
                    raise TypeError(f"lucid_amd.optim.AdamW: grad dtype {g.dtype} differs from the parameter's {p.dtype}")
                if not g.is_contiguous():
                    g = g.contiguous()
                state = self.state[p]
                if not state:
                    state["step"] = torch.tensor(0.0)
                    state["exp_avg"] = torch.zeros_like(p, memory_format=torch.contiguous_format)
                    state["exp_avg_sq"] = torch.zeros_like(p, memory_format=torch.contiguous_format)
                state["step"] += 1
                key = (p.device, p.dtype, int(state["step"].item()))
                batches.setdefault(key, []).append((p, g, state["exp_avg"], state["exp_avg_sq"]))
            beta1, beta2 = group["betas"]
            for (dev, dtype, step), items in batches.items():
                n = len(items)
                arrs = [(ctypes.c_void_p * n)(*(t[j].data_ptr() for t in items)) for j in range(4)]
                numels = (ctypes.c_int64 * n)(*(t[0].numel() for t in items))
                rc = lib.lucid_adamw_step(n, arrs[0], arrs[1], arrs[2], arrs[3], numels, _DTYPES[dtype],
                                          float(group["lr"]), float(beta1), float(beta2), float(group["eps"]),
                                          float(group["weight_decay"]), step, _lib.stream_handle(dev))
                _lib.check(lib, rc, "lucid_adamw_step")
        return loss
