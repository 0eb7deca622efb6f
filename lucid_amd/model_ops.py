"""Fused RMSNorm and rotary-embedding layers of the Llama-LUCID decoder on HIP kernels.

The reference model (``modeling_lucid.py:58-75`` RMSNorm, ``:112-145`` rotate_half /
apply_rotary_pos_emb) writes both as chains of torch elementwise ops, each a full pass over
the activations in HBM.  Here each is one kernel pass forward and one backward:

* :func:`rms_norm` -- y = w * bf16(x * rstd) with rstd = 1 / sqrt(mean(x^2) + eps) in fp32
  (the reference's statistics and rounding points); backward dx = rstd (g - xn mean(g xn)),
  g = bf16(dy w), and dw summed over row blocks in a fixed order (deterministic).
* :func:`apply_rope` -- x cos + rotate_half(x) sin on a ``[B, H, T, 64]`` view of the
  ``[B, T, H, 64]`` projection output, written as ``[B, T, H, 64]`` (returned as the same
  transposed view), rounded to bf16 once; backward applies the transposed rotation.

Both take bf16 GPU tensors only (hidden sizes 512, 1024, 2048 or 4096; head dim 64) and
raise otherwise; :func:`rms_norm_supported` / :func:`rope_supported` tell the model which
inputs they cover.
"""
from __future__ import annotations

import torch

from . import _lib

_NORM_H = (512, 1024, 2048, 4096)


def _aligned(t: torch.Tensor) -> torch.Tensor:
    """Contiguous with a 16-byte aligned base (the kernels load 8 bf16 at a time)."""
    t = t.contiguous()
    return t if t.data_ptr() % 16 == 0 else t.clone()


def rms_norm_supported(x: torch.Tensor, weight: torch.Tensor) -> bool:
    return (x.is_cuda and x.dtype == torch.bfloat16 and weight.dtype == torch.bfloat16
            and x.shape[-1] in _NORM_H and weight.shape == (x.shape[-1],))


def rope_supported(x: torch.Tensor, cos: torch.Tensor) -> bool:
    return x.is_cuda and x.dtype == torch.bfloat16 and cos.dtype == torch.bfloat16 and x.dim() == 4 \
        and x.shape[-1] == 64


class RMSNormFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x: torch.Tensor, weight: torch.Tensor, eps: float):
        if not rms_norm_supported(x, weight):
            raise TypeError("lucid_amd.rms_norm: bf16 GPU input and weight with hidden size in "
                            f"{_NORM_H}, got {x.dtype} {tuple(x.shape)} / {weight.dtype}")
        H = x.shape[-1]
        x2 = _aligned(x.reshape(-1, H))
        w = _aligned(weight)
        N = x2.shape[0]
        y = torch.empty_like(x2)
        rstd = torch.empty(N, dtype=torch.float32, device=x.device)
        lib = _lib.load()
        rc = lib.lucid_rmsnorm_fwd(_lib.ptr(x2), _lib.ptr(w), _lib.ptr(y), _lib.ptr(rstd), N, H, float(eps),
                                   _lib.stream_handle(x.device))
        _lib.check(lib, rc, "lucid_rmsnorm_fwd")
        ctx.save_for_backward(x2, w, rstd)
        ctx.shape = x.shape
        return y.view(x.shape)

    @staticmethod
    def backward(ctx, dy: torch.Tensor):
        x2, w, rstd = ctx.saved_tensors
        N, H = x2.shape
        dy2 = _aligned(dy.reshape(N, H))
        dx = torch.empty_like(x2)
        dw = torch.empty_like(w)
        lib = _lib.load()
        nbytes = lib.lucid_rmsnorm_bwd_workspace_bytes(N, H)
        ws = torch.empty(max(nbytes // 4, 1), dtype=torch.float32, device=x2.device)
        rc = lib.lucid_rmsnorm_bwd(_lib.ptr(x2), _lib.ptr(w), _lib.ptr(dy2), _lib.ptr(rstd), _lib.ptr(dx),
                                   _lib.ptr(dw), _lib.ptr(ws), N, H, _lib.stream_handle(x2.device))
        _lib.check(lib, rc, "lucid_rmsnorm_bwd")
        return dx.view(ctx.shape), dw, None


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """RMSNorm over the last axis (``LlamaRMSNorm.forward``, modeling_lucid.py:58-75)."""
    return RMSNormFunction.apply(x, weight, eps)


def _rows(t: torch.Tensor):
    """``t`` [B, H, T, 64] viewed as rows in [B, T, H] order: (tensor, row stride); copies
    when the three leading axes do not collapse into one stride."""
    B, Hn, T, _ = t.shape
    s = t.stride()
    if s[3] == 1 and s[1] % 8 == 0 and s[2] == Hn * s[1] and (B == 1 or s[0] == T * s[2]) \
            and t.data_ptr() % 16 == 0:
        return t, s[1]
    return t.transpose(1, 2).contiguous().transpose(1, 2), 64


def _tokens(c: torch.Tensor, B: int, T: int) -> torch.Tensor:
    """cos / sin [B or 1, T, 64] as B*T contiguous token rows."""
    if c.dim() == 2:
        c = c.unsqueeze(0)
    return c.expand(B, T, c.shape[-1]).contiguous()


def _rope_launch(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, transpose: int) -> torch.Tensor:
    B, Hn, T, D = x.shape
    xr, xs = _rows(x)
    out = torch.empty(B, T, Hn, D, dtype=x.dtype, device=x.device)
    lib = _lib.load()
    rc = lib.lucid_rope(_lib.ptr(xr), xs, B * T * Hn, Hn, _lib.ptr(cos), _lib.ptr(sin), _lib.ptr(out), D, transpose,
                        _lib.stream_handle(x.device))
    _lib.check(lib, rc, "lucid_rope")
    return out.transpose(1, 2)


class RopeFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor):
        if not rope_supported(x, cos) or sin.dtype != cos.dtype:
            raise TypeError(f"lucid_amd.apply_rope: bf16 GPU [B, H, T, 64] input, got {x.dtype} {tuple(x.shape)}")
        B, _, T, _ = x.shape
        c, s = _tokens(cos, B, T), _tokens(sin, B, T)
        ctx.save_for_backward(c, s)
        return _rope_launch(x, c, s, 0)

    @staticmethod
    def backward(ctx, g: torch.Tensor):
        c, s = ctx.saved_tensors
        return _rope_launch(g, c, s, 1), None, None


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """x cos + rotate_half(x) sin for x [B, H, T, 64] and cos / sin [B or 1, T, 64]
    (modeling_lucid.py:118-145 with unsqueeze_dim 1)."""
    return RopeFunction.apply(x, cos, sin)
