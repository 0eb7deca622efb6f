"""Fused elementwise layers of the Llama-LUCID decoder on HIP kernels.

The reference model (``modeling_lucid.py:58-75`` RMSNorm, ``:112-145`` rotate_half /
apply_rotary_pos_emb, ``:155-167`` the SwiGLU MLP, ``:847-967`` the loss) writes these as
chains of torch elementwise ops, each a full pass over the activations in HBM.  Here each is
one kernel pass forward and one backward:

* :func:`rms_norm` -- y = w * bf16(x * rstd) with rstd = 1 / sqrt(mean(x^2) + eps) in fp32
  (the reference's statistics and rounding points); backward dx = rstd (g - xn mean(g xn)),
  g = bf16(dy w), and dw summed over row blocks in a fixed order (deterministic).
* :func:`apply_rope` -- x cos + rotate_half(x) sin on a ``[B, H, T, 64]`` view of the
  ``[B, T, H, 64]`` projection output (any strides that are multiples of 8), written as
  ``[B, T, H, 64]`` (returned as the same transposed view), rounded to bf16 once; backward
  applies the transposed rotation.

* :func:`swiglu` -- silu(g) * u of the MLP, one pass each way with fp32 inside (the
  reference rounds silu(g) to bf16 before the product).
* :func:`causal_lm_loss` -- the shifted cross entropy on bf16 logits, one read of the logits
  forward (per-row logsumexp) and one read + write backward, instead of fp32 copies of them.

All take bf16 GPU tensors only (RMSNorm: hidden sizes 512, 1024, 2048 or 4096; RoPE: head
dim 64; the loss: a vocabulary that is a multiple of 8) and raise otherwise; the
``*_supported`` predicates tell the model which inputs they cover.
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


def _strided(t: torch.Tensor) -> torch.Tensor:
    """``t`` [B, H, T, 64] as the kernel reads it: unit stride on the head axis, the other
    strides multiples of 8 elements, a 16-byte aligned base (copied otherwise)."""
    if t.stride(3) == 1 and all(s % 8 == 0 for s in t.stride()[:3]) and t.data_ptr() % 16 == 0:
        return t
    return t.contiguous()


def _tokens(c: torch.Tensor, B: int, T: int) -> torch.Tensor:
    """cos / sin [B or 1, T, 64] as B*T contiguous token rows."""
    if c.dim() == 2:
        c = c.unsqueeze(0)
    return _aligned(c.expand(B, T, c.shape[-1]))


def _rope_launch(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, transpose: int,
                 out: torch.Tensor | None = None) -> torch.Tensor:
    """x [B, H, T, 64] rotated into ``out`` ([B, H, T, 64], strides multiples of 8; default: a
    new [B, T, H, 64] buffer seen as [B, H, T, 64])."""
    B, Hn, T, D = x.shape
    xr = _strided(x)
    if out is None:
        out = torch.empty(B, T, Hn, D, dtype=x.dtype, device=x.device).transpose(1, 2)
    lib = _lib.load()
    rc = lib.lucid_rope(_lib.ptr(xr), _lib.strides3(xr, (0, 1, 2)), B, Hn, T, _lib.ptr(cos), _lib.ptr(sin),
                        _lib.ptr(out), _lib.strides3(out, (0, 1, 2)), D, transpose, _lib.stream_handle(x.device))
    _lib.check(lib, rc, "lucid_rope")
    return out


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


class QKVRopeFunction(torch.autograd.Function):
    """The stacked projection output qkv [B, T, (Hq + 2 Hkv) 64] split into q, k, v, with the
    rotary embedding applied to q and k.  Its backward writes the rotated-back dq, dk and dv
    straight into one [B, T, (Hq + 2 Hkv) 64] gradient, so that no concatenation of the three
    follows (the split's own backward would concatenate them)."""

    @staticmethod
    def forward(ctx, qkv: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, nq: int, nk: int):
        B, T, N = qkv.shape
        if not (qkv.is_cuda and qkv.dtype == torch.bfloat16 and cos.dtype == torch.bfloat16
                and nq % 64 == 0 and nk % 64 == 0 and N == nq + 2 * nk):
            raise TypeError("lucid_amd.qkv_rope: bf16 GPU [B, T, (Hq + 2 Hkv) 64] projections")
        hq, hk = nq // 64, nk // 64

        def heads(t, h):
            return t.view(B, T, h, 64).transpose(1, 2)

        c, s = _tokens(cos, B, T), _tokens(sin, B, T)
        q = _rope_launch(heads(qkv[..., :nq], hq), c, s, 0)
        k = _rope_launch(heads(qkv[..., nq:nq + nk], hk), c, s, 0)
        v = heads(qkv[..., nq + nk:], hk)
        ctx.save_for_backward(c, s)
        ctx.dims = (B, T, N, nq, nk)
        return q, k, v

    @staticmethod
    def backward(ctx, dq, dk, dv):
        c, s = ctx.saved_tensors
        B, T, N, nq, nk = ctx.dims
        dev = c.device
        g = torch.empty(B, T, N, dtype=torch.bfloat16, device=dev)

        def heads(t, h):
            return t.view(B, T, h, 64).transpose(1, 2)

        for grad, lo, n in ((dq, 0, nq), (dk, nq, nk)):
            if grad is None:
                g[..., lo:lo + n].zero_()
            else:
                _rope_launch(grad, c, s, 1, out=heads(g[..., lo:lo + n], n // 64))
        if dv is None:
            g[..., nq + nk:].zero_()
        else:
            heads(g[..., nq + nk:], nk // 64).copy_(dv)
        return g, None, None, None, None


def qkv_rope(qkv: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, nq: int, nk: int):
    """(q, k, v) [B, H, T, 64] from the stacked projection output, q and k rotated
    (apply_rotary_pos_emb, modeling_lucid.py:118-145)."""
    return QKVRopeFunction.apply(qkv, cos, sin, nq, nk)


def swiglu_supported(g: torch.Tensor, u: torch.Tensor) -> bool:
    return g.is_cuda and g.dtype == torch.bfloat16 and u.dtype == torch.bfloat16 and g.shape == u.shape


class SwiGLUFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, g: torch.Tensor, u: torch.Tensor):
        if not swiglu_supported(g, u):
            raise TypeError(f"lucid_amd.swiglu: bf16 GPU gate and up of one shape, got {g.dtype} {tuple(g.shape)} / "
                            f"{u.dtype} {tuple(u.shape)}")
        g2, u2 = _aligned(g), _aligned(u)
        h = torch.empty_like(g2)
        lib = _lib.load()
        rc = lib.lucid_swiglu_fwd(_lib.ptr(g2), _lib.ptr(u2), _lib.ptr(h), g2.numel(), _lib.stream_handle(g.device))
        _lib.check(lib, rc, "lucid_swiglu_fwd")
        ctx.save_for_backward(g2, u2)
        return h

    @staticmethod
    def backward(ctx, dh: torch.Tensor):
        g2, u2 = ctx.saved_tensors
        dh2 = _aligned(dh)
        dg, du = torch.empty_like(g2), torch.empty_like(u2)
        lib = _lib.load()
        rc = lib.lucid_swiglu_bwd(_lib.ptr(g2), _lib.ptr(u2), _lib.ptr(dh2), _lib.ptr(dg), _lib.ptr(du), g2.numel(),
                                  _lib.stream_handle(g2.device))
        _lib.check(lib, rc, "lucid_swiglu_bwd")
        return dg, du


def swiglu(g: torch.Tensor, u: torch.Tensor) -> torch.Tensor:
    """silu(g) * u (the gated activation of ``LlamaMLP.forward``, modeling_lucid.py:155-167)."""
    return SwiGLUFunction.apply(g, u)


IGNORE_INDEX = -100


def causal_lm_loss_supported(logits: torch.Tensor, labels: torch.Tensor) -> bool:
    return (logits.is_cuda and logits.dtype == torch.bfloat16 and logits.dim() == 3 and logits.shape[-1] % 8 == 0
            and labels.shape == logits.shape[:2] and labels.dtype == torch.int64)


class CausalLMLossFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, logits: torch.Tensor, labels: torch.Tensor):
        if not causal_lm_loss_supported(logits, labels):
            raise TypeError("lucid_amd.causal_lm_loss: bf16 GPU logits [B, T, V] (V a multiple of 8) and int64 "
                            f"labels [B, T], got {logits.dtype} {tuple(logits.shape)} / {labels.dtype}")
        B, T, V = logits.shape
        lg = _aligned(logits.reshape(B * T, V))
        lb = labels.reshape(-1).contiguous()
        R = B * T
        lse, per_row, valid = (torch.empty(R, dtype=torch.float32, device=logits.device) for _ in range(3))
        lib = _lib.load()
        rc = lib.lucid_causal_lm_loss_fwd(_lib.ptr(lg), V, _lib.ptr(lb), R, T, V, _lib.ptr(lse), _lib.ptr(per_row),
                                          _lib.ptr(valid), _lib.stream_handle(logits.device))
        _lib.check(lib, rc, "lucid_causal_lm_loss_fwd")
        count = valid.sum()
        ctx.save_for_backward(lg, lb, lse, valid, count)
        ctx.dims = (B, T, V)
        return per_row.sum() / count

    @staticmethod
    def backward(ctx, dloss: torch.Tensor):
        lg, lb, lse, valid, count = ctx.saved_tensors
        B, T, V = ctx.dims
        scale = (dloss.float() / count).reshape(1).contiguous()
        dlogits = torch.empty(B * T, V, dtype=torch.bfloat16, device=lg.device)
        lib = _lib.load()
        rc = lib.lucid_causal_lm_loss_bwd(_lib.ptr(lg), V, _lib.ptr(lb), B * T, T, V, _lib.ptr(lse), _lib.ptr(valid),
                                          _lib.ptr(scale), _lib.ptr(dlogits), _lib.stream_handle(lg.device))
        _lib.check(lib, rc, "lucid_causal_lm_loss_bwd")
        return dlogits.view(B, T, V), None


def causal_lm_loss(logits: torch.Tensor, labels: torch.Tensor) -> torch.Tensor:
    """Mean cross entropy of logits[:, :-1] against labels[:, 1:] with -100 ignored, computed in
    fp32 (``LlamaForCausalLM.forward``'s loss, modeling_lucid.py:847-967); a float32 scalar."""
    return CausalLMLossFunction.apply(logits, labels)
