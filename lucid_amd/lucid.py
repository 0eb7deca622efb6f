"""LUCID attention operators on the HIP kernels (MI355X / gfx950).

Python mirror of the reference operator seams in ``modeling_lucid.py``:

* :func:`get_v_prime`      -- ``LucidAttention.get_v_prime`` (:551-574): V' = P^-1 V
* :func:`eager_lucid_attention_forward` -- ``LucidAttention.eager_lucid_attention_forward``
  (:505-549) fused with the solve: O = softmax(s Q K^T, causal) V'
* :func:`lucid_attention`  -- both in one differentiable call (forward + backward kernels)

Layouts follow the reference: ``query [B, Hq, T, d]``, ``key/value [B, Hkv, T, d]``
(any strides with a contiguous last axis, e.g. the ``.view(...).transpose(1, 2)``
views LucidAttention builds), output ``[B, T, Hq, d]``.  Inputs must be bf16
CUDA(HIP) tensors with d in {64, 128}; anything else raises (there is no CPU or
eager fallback).  T that is not a multiple of 128 is zero-padded at the end,
which is exact for every real row because P and the attention mask are causal.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from . import _lib

_T_ALIGN = 128
_SUPPORTED_D = (64, 128)


def _check_inputs(q, k, v):
    for name, t in (("query", q), ("key", k), ("value", v)):
        if t is None:
            continue
        if not t.is_cuda:
            raise RuntimeError(f"lucid_amd: {name} must be a GPU tensor (no CPU path)")
        if t.dtype != torch.bfloat16:
            raise TypeError(f"lucid_amd: {name} must be bfloat16, got {t.dtype}")
        if t.dim() != 4:
            raise ValueError(f"lucid_amd: {name} must be 4-D [B, H, T, d]")
    if k.shape != v.shape:
        raise ValueError(f"lucid_amd: key {tuple(k.shape)} and value {tuple(v.shape)} must match")
    d = k.shape[-1]
    if d not in _SUPPORTED_D:
        raise ValueError(f"lucid_amd: head_dim {d} not supported (supported: {_SUPPORTED_D})")
    if q is not None:
        if q.shape[0] != k.shape[0] or q.shape[2] != k.shape[2] or q.shape[3] != d:
            raise ValueError("lucid_amd: query/key shapes disagree")
        if q.shape[1] % k.shape[1]:
            raise ValueError("lucid_amd: number of query heads must be a multiple of key/value heads")


def _prep(t: torch.Tensor, tp: int) -> torch.Tensor:
    """Pad the time axis (dim 2) to ``tp`` and make the last axis contiguous with 8-aligned strides."""
    if t.shape[2] != tp:
        t = F.pad(t, (0, 0, 0, tp - t.shape[2]))
    if t.stride(-1) != 1 or any(s % 8 for s in t.stride()[:3]) or t.data_ptr() % 16:
        t = t.contiguous()
    return t


def _padded_len(t: int) -> int:
    return (t + _T_ALIGN - 1) // _T_ALIGN * _T_ALIGN


def _fwd(q, k, v, scale, eps):
    lib = _lib.load()
    B, Hq, T, D = q.shape
    Hkv = k.shape[1]
    dev = q.device
    o = torch.empty(B, T, Hq, D, dtype=torch.bfloat16, device=dev)
    vprime = torch.empty(B, Hkv, T, D, dtype=torch.float32, device=dev)
    lse = torch.empty(B, Hq, T, dtype=torch.float32, device=dev)
    ws = torch.empty(lib.lucid_fwd_workspace_bytes(B, Hq, Hkv, T, D), dtype=torch.uint8, device=dev)
    rc = lib.lucid_attn_fwd(
        _lib.ptr(q), _lib.strides3(q, (0, 1, 2)), _lib.ptr(k), _lib.strides3(k, (0, 1, 2)),
        _lib.ptr(v), _lib.strides3(v, (0, 1, 2)), _lib.ptr(o), _lib.strides3(o, (0, 2, 1)),
        _lib.ptr(vprime), _lib.ptr(lse), _lib.ptr(ws), B, Hq, Hkv, T, D, float(scale), float(eps),
        _lib.stream_handle(dev))
    _lib.check(lib, rc, "lucid_attn_fwd")
    return o, vprime, lse, ws


def _bwd(do, q, k, o, lse, ws, scale, eps):
    lib = _lib.load()
    B, Hq, T, D = q.shape
    Hkv = k.shape[1]
    dev = q.device
    dq = torch.empty(B, Hq, T, D, dtype=torch.bfloat16, device=dev)
    dk = torch.empty(B, Hkv, T, D, dtype=torch.bfloat16, device=dev)
    dv = torch.empty(B, Hkv, T, D, dtype=torch.bfloat16, device=dev)
    bws = torch.empty(lib.lucid_bwd_workspace_bytes(B, Hq, Hkv, T, D), dtype=torch.uint8, device=dev)
    rc = lib.lucid_attn_bwd(
        _lib.ptr(do), _lib.strides3(do, (0, 2, 1)), _lib.ptr(q), _lib.strides3(q, (0, 1, 2)),
        _lib.ptr(k), _lib.strides3(k, (0, 1, 2)), _lib.ptr(o), _lib.strides3(o, (0, 2, 1)),
        _lib.ptr(lse), _lib.ptr(ws), _lib.ptr(dq), _lib.strides3(dq, (0, 1, 2)),
        _lib.ptr(dk), _lib.strides3(dk, (0, 1, 2)), _lib.ptr(dv), _lib.strides3(dv, (0, 1, 2)),
        _lib.ptr(bws), B, Hq, Hkv, T, D, float(scale), float(eps), _lib.stream_handle(dev))
    _lib.check(lib, rc, "lucid_attn_bwd")
    return dq, dk, dv


class LucidAttentionFunction(torch.autograd.Function):
    """O = softmax(s Q K^T, causal) (P^-1 V) with HIP forward and backward kernels.

    Gradients follow ``Lucid_Tril_Solver.backward`` (modeling_lucid.py:314-382)
    for the preconditioner and the softmax-attention backward for SDPA.
    """

    @staticmethod
    def forward(ctx, q, k, v, scale, eps):
        t = q.shape[2]
        ctx.empty = t == 0 or q.numel() == 0
        ctx.shapes = (q.shape, k.shape)
        if ctx.empty:  # the reference's torch ops return empty results (no kernel launch)
            B, Hq, _, D = q.shape
            return (q.new_empty(B, t, Hq, D),
                    torch.empty(B, k.shape[1], t, D, dtype=torch.float32, device=q.device))
        tp = _padded_len(t)
        qp, kp, vp_ = _prep(q, tp), _prep(k, tp), _prep(v, tp)
        o, vprime, lse, ws = _fwd(qp, kp, vp_, scale, eps)
        ctx.save_for_backward(qp, kp, o, lse, ws)
        ctx.scale, ctx.eps, ctx.t = scale, eps, t
        ctx.mark_non_differentiable(vprime)
        return o[:, :t], vprime[:, :, :t]

    @staticmethod
    def backward(ctx, do, _dvprime):
        if ctx.empty:
            return do.new_zeros(ctx.shapes[0]), do.new_zeros(ctx.shapes[1]), do.new_zeros(ctx.shapes[1]), None, None
        qp, kp, o, lse, ws = ctx.saved_tensors
        t, tp = ctx.t, qp.shape[2]
        if do.dtype != torch.bfloat16:
            do = do.to(torch.bfloat16)
        if t != tp:
            do = F.pad(do, (0, 0, 0, 0, 0, tp - t))
        if do.stride(-1) != 1 or any(s % 8 for s in do.stride()) or do.data_ptr() % 16:
            do = do.contiguous()
        dq, dk, dv = _bwd(do, qp, kp, o, lse, ws, ctx.scale, ctx.eps)
        return dq[:, :, :t], dk[:, :, :t], dv[:, :, :t], None, None


def lucid_attention(query, key, value, scaling=None, eps=1e-5, return_vprime=False):
    """LUCID attention: ``softmax(s Q K^T, causal) P^-1 V``; returns O ``[B, T, Hq, d]``.

    ``eps`` is the k_norm epsilon (``config.rms_norm_eps``, modeling_lucid.py:409).
    """
    _check_inputs(query, key, value)
    scale = query.shape[-1] ** -0.5 if scaling is None else float(scaling)
    o, vprime = LucidAttentionFunction.apply(query, key, value, scale, eps)
    return (o, vprime) if return_vprime else o


def get_v_prime(key, value, scaling=None, eps=1e-5):
    """``V' = P^-1 V`` (forward only), fp32 ``[B, Hkv, T, d]`` -- get_v_prime, modeling_lucid.py:551-574."""
    _check_inputs(None, key, value)
    B, Hkv, T, D = key.shape
    if T == 0 or key.numel() == 0:
        return torch.empty(B, Hkv, T, D, dtype=torch.float32, device=key.device)
    lib = _lib.load()
    tp = _padded_len(T)
    k, v = _prep(key, tp), _prep(value, tp)
    scale = D ** -0.5 if scaling is None else float(scaling)
    vprime = torch.empty(B, Hkv, tp, D, dtype=torch.float32, device=key.device)
    ws = torch.empty(lib.lucid_fwd_workspace_bytes(B, Hkv, Hkv, tp, D), dtype=torch.uint8, device=key.device)
    rc = lib.lucid_get_v_prime(_lib.ptr(k), _lib.strides3(k, (0, 1, 2)), _lib.ptr(v), _lib.strides3(v, (0, 1, 2)),
                               _lib.ptr(vprime), _lib.ptr(ws), B, Hkv, tp, D, scale, float(eps),
                               _lib.stream_handle(key.device))
    _lib.check(lib, rc, "lucid_get_v_prime")
    return vprime[:, :, :T]


def eager_lucid_attention_forward(query, key, value, scaling=None, eps=1e-5):
    """Drop-in for ``get_v_prime`` followed by ``eager_lucid_attention_forward``: returns ``(O, None)``."""
    return lucid_attention(query, key, value, scaling, eps), None


def lucid_decode(query, key, value, key_cache, vprime_cache, cache_len, scaling=None, eps=1e-5):
    """One decoding step for one new token per sequence (``get_new_v_prime`` and the cached
    attention of LucidAttention.forward, modeling_lucid.py:475-496, 576-598).

    ``query [B, Hq, 1, d]``, ``key/value [B, Hkv, 1, d]`` (bf16; keys with RoPE applied);
    ``key_cache`` / ``vprime_cache`` are bf16 buffers ``[B, Hkv, T_cap, d]`` whose first
    ``cache_len`` rows are valid.  The token's V' row (exact diagonal:
    ``v'_t = (v_t - sum_j P_tj v'_j) / P_tt``) and its key are written at row ``cache_len``
    of the caches in place.  Returns ``(O [B, 1, Hq, d], v'_t fp32 [B, Hkv, 1, d])``.
    """
    _check_inputs(None, key, value)
    for name, t in (("query", query), ("key_cache", key_cache), ("vprime_cache", vprime_cache)):
        if not t.is_cuda or t.dtype != torch.bfloat16 or t.dim() != 4:
            raise TypeError(f"lucid_amd: {name} must be a 4-D bfloat16 GPU tensor")
        if t.stride(-1) != 1 or any(s % 8 for s in t.stride()[:3]) or t.data_ptr() % 16:
            raise ValueError(f"lucid_amd: {name} needs a contiguous last axis and 8-element aligned strides")
    B, Hkv, tn, D = key.shape
    Hq = query.shape[1]
    if tn != 1 or query.shape[2] != 1:
        raise ValueError("lucid_amd: lucid_decode takes one new token per sequence")
    if key_cache.shape[:2] != (B, Hkv) or vprime_cache.shape != key_cache.shape or key_cache.shape[3] != D:
        raise ValueError("lucid_amd: cache shapes disagree with the new key")
    lib = _lib.load()
    cap = key_cache.shape[2]
    q, k, v = (_prep(t, 1) for t in (query, key, value))
    o = torch.empty(B, 1, Hq, D, dtype=torch.bfloat16, device=q.device)
    vp_new = torch.empty(B, Hkv, 1, D, dtype=torch.float32, device=q.device)
    ws = torch.empty(max(lib.lucid_decode_workspace_bytes(B, Hq, Hkv, cap, D), 256), dtype=torch.uint8,
                     device=q.device)
    scale = D ** -0.5 if scaling is None else float(scaling)
    rc = lib.lucid_decode(
        _lib.ptr(q), _lib.strides3(q, (0, 1, 2)), _lib.ptr(k), _lib.strides3(k, (0, 1, 2)),
        _lib.ptr(v), _lib.strides3(v, (0, 1, 2)), _lib.ptr(key_cache), _lib.strides3(key_cache, (0, 1, 2)),
        _lib.ptr(vprime_cache), _lib.strides3(vprime_cache, (0, 1, 2)), _lib.ptr(o), _lib.strides3(o, (0, 2, 1)),
        _lib.ptr(vp_new), _lib.ptr(ws), B, Hq, Hkv, int(cache_len), cap, D, scale, float(eps),
        _lib.stream_handle(q.device))
    _lib.check(lib, rc, "lucid_decode")
    return o, vp_new
