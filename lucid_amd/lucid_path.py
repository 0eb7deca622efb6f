"""LUCID-Path attention on the HIP kernels (MI355X / gfx950).

Python mirror of ``fla.ops.lucid_path`` (reference ``lucid_path/triton_code/parallel.py``):
:func:`parallel_lucid_path_attention` keeps the reference signature, defaults and
asserts (parallel.py:180-241) and returns ``(o, k_cache)``.

    O = (I + L)^-1 V,  L_ij = exp(s A_ij - 1/s) (j < i),  A_ij = q_i^T H_i ... H_{j+1} k_j,
    H_t = I - beta_t w_t w_t^T

:func:`parallel_path_attention` is PaTH softmax attention on the same path logits
(diagonal included), the softmax half of a LUCID-Path layer, whose forward the
reference ships as the kernels ``intra_chunk_preprocess_fwd.py`` and
``parallel_path_fwd.py`` (entry point and backward in the unvendored fla package):

    O_i = sum_{j <= i} softmax_j(s A_ij) v_j

Tensors are GPU tensors in the reference layout ``[B, T, H, K]``, all bf16 or all fp32 (the
reference's LUCID-Path model is fp32, lucid_path/config/config.json:5).  bf16 runs at
K = V = 64 and K = V = 128, fp32 at K = V = 64 (3-term bf16 split products on hi / lo copies
of every operand, ~fp32 accuracy), and the other head dims the reference's kernels take
(16, 32; a K/V pair that differs) run on rows zero-padded to the next supported one: the
reflections ``I - beta w w^T`` act as the identity on the padded coordinates, so the logits,
O and the gradients of the real coordinates are unchanged.  There is no CPU or Triton fallback.
"""
from __future__ import annotations

import ctypes
from typing import Optional

import torch
import torch.nn.functional as F

from . import _lib

_LIB = "liblucid_path.so"


def _pad_t(x: torch.Tensor, tp: int) -> torch.Tensor:
    t = x.shape[1]
    if t == tp:
        return x
    pad = [0, 0] * (x.dim() - 2) + [0, tp - t]
    return F.pad(x, pad)


def _ready(x: torch.Tensor) -> torch.Tensor:
    if x.stride(-1) != 1 or x.data_ptr() % 16 or any(s % 8 for s in x.stride()[:-1]):
        x = x.contiguous()
    return x


def _entry(softmax: bool, fwd: bool, dtype: torch.dtype) -> str:
    """C entry point name: lucid_path[_softmax]_{fwd,bwd}[_f32]."""
    return ("lucid_path_softmax_" if softmax else "lucid_path_") + ("fwd" if fwd else "bwd") + (
        "_f32" if dtype == torch.float32 else "")


def _fwd(q, k, v, w, beta, scale, use_cache, softmax=False):
    lib = _lib.load(_LIB)
    name = _entry(softmax, True, q.dtype)
    B, T, HQ, K = q.shape
    H = k.shape[2]
    dev = q.device
    o = torch.empty(B, T, HQ, v.shape[-1], dtype=q.dtype, device=dev)
    kc = torch.empty(B, T, H, K, dtype=q.dtype, device=dev) if use_cache else None
    ws = torch.empty(getattr(lib, name + "_workspace_bytes")(B, T, H, HQ, K), dtype=torch.uint8, device=dev)
    beta = beta.contiguous()
    st3 = lambda t: _lib.strides3(t, (0, 2, 1))  # noqa: E731  (batch, head, time)
    beta_strides = (ctypes.c_int64 * 3)(beta.stride(0), beta.stride(2), beta.stride(1))
    rc = getattr(lib, name)(
        _lib.ptr(q), st3(q), _lib.ptr(k), st3(k), _lib.ptr(v), st3(v), _lib.ptr(w), st3(w),
        _lib.ptr(beta), beta_strides, _lib.ptr(o), st3(o),
        _lib.ptr(kc) if kc is not None else None, st3(kc) if kc is not None else None,
        _lib.ptr(ws), B, T, H, HQ, K, float(scale), _lib.stream_handle(dev))
    _lib.check(lib, rc, name)
    return o, kc, ws


class ParallelLUCIDPathAttentionFunction(torch.autograd.Function):
    """Forward/backward of LUCID-Path (ParallelLUCIDPathAttentionFunction, parallel.py:27-177)."""

    @staticmethod
    def forward(ctx, q, k, v, w, beta, g, scale, cu_seqlens, use_cache=False):
        t = q.shape[1]
        tp = (t + 63) // 64 * 64
        q, k, v, w, beta = (_ready(_pad_t(x, tp)) for x in (q, k, v, w, beta))
        o, kc, ws = _fwd(q, k, v, w, beta, scale, use_cache)
        ctx.save_for_backward(q, k, v, w, beta, o, ws)
        ctx.scale, ctx.t = scale, t
        if kc is not None:
            kc = kc[:, :t]
            ctx.mark_non_differentiable(kc)
        return o[:, :t], kc

    @staticmethod
    def backward(ctx, do, dk_cache):
        # the k_cache output carries no gradient (parallel.py:78-81 ignores dk_new)
        q, k, v, w, beta, o, ws = ctx.saved_tensors
        t, tp = ctx.t, q.shape[1]
        if do.dtype != q.dtype:
            do = do.to(q.dtype)
        do = _ready(_pad_t(do, tp))
        lib = _lib.load(_LIB)
        name = _entry(False, False, q.dtype)
        B, T, HQ, K = q.shape
        H = k.shape[2]
        dq, dk, dv, dw = (torch.empty_like(x) for x in (q, k, v, w))
        db = torch.empty(B, T, H, dtype=q.dtype, device=q.device)
        bws = torch.empty(getattr(lib, name + "_workspace_bytes")(B, T, H, HQ, K), dtype=torch.uint8,
                          device=q.device)
        st3 = lambda x: _lib.strides3(x, (0, 2, 1))  # noqa: E731
        bst = lambda x: (ctypes.c_int64 * 3)(x.stride(0), x.stride(2), x.stride(1))  # noqa: E731
        rc = getattr(lib, name)(
            _lib.ptr(do), st3(do), _lib.ptr(q), st3(q), _lib.ptr(k), st3(k), _lib.ptr(w), st3(w),
            _lib.ptr(beta), bst(beta), _lib.ptr(o), st3(o), _lib.ptr(ws),
            _lib.ptr(dq), st3(dq), _lib.ptr(dk), st3(dk), _lib.ptr(dv), st3(dv), _lib.ptr(dw), st3(dw),
            _lib.ptr(db), bst(db), _lib.ptr(bws), B, T, H, HQ, K, float(ctx.scale), _lib.stream_handle(q.device))
        _lib.check(lib, rc, name)
        return (dq[:, :t], dk[:, :t], dv[:, :t], dw[:, :t], db[:, :t], None, None, None, None)


class ParallelPathAttentionFunction(torch.autograd.Function):
    """Forward/backward of PaTH softmax attention (forward: intra_chunk_preprocess_fwd.py:14-168
    then parallel_path_fwd.py:13-170; backward: softmax gradient of the same logits)."""

    @staticmethod
    def forward(ctx, q, k, v, w, beta, g, scale, cu_seqlens, use_cache=False):
        t = q.shape[1]
        tp = (t + 63) // 64 * 64
        q, k, v, w, beta = (_ready(_pad_t(x, tp)) for x in (q, k, v, w, beta))
        o, kc, ws = _fwd(q, k, v, w, beta, scale, use_cache, softmax=True)
        ctx.save_for_backward(q, k, v, w, beta, o, ws)
        ctx.scale, ctx.t = scale, t
        if kc is not None:
            kc = kc[:, :t]
            ctx.mark_non_differentiable(kc)
        return o[:, :t], kc

    @staticmethod
    def backward(ctx, do, dk_cache):
        q, k, v, w, beta, o, ws = ctx.saved_tensors
        t, tp = ctx.t, q.shape[1]
        if do.dtype != q.dtype:
            do = do.to(q.dtype)
        do = _ready(_pad_t(do, tp))
        lib = _lib.load(_LIB)
        name = _entry(True, False, q.dtype)
        B, T, HQ, K = q.shape
        H = k.shape[2]
        dq, dk, dv, dw = (torch.empty_like(x) for x in (q, k, v, w))
        db = torch.empty(B, T, H, dtype=q.dtype, device=q.device)
        bws = torch.empty(getattr(lib, name + "_workspace_bytes")(B, T, H, HQ, K), dtype=torch.uint8,
                          device=q.device)
        st3 = lambda x: _lib.strides3(x, (0, 2, 1))  # noqa: E731
        bst = lambda x: (ctypes.c_int64 * 3)(x.stride(0), x.stride(2), x.stride(1))  # noqa: E731
        rc = getattr(lib, name)(
            _lib.ptr(do), st3(do), _lib.ptr(q), st3(q), _lib.ptr(k), st3(k), _lib.ptr(v), st3(v),
            _lib.ptr(w), st3(w), _lib.ptr(beta), bst(beta), _lib.ptr(o), st3(o), _lib.ptr(ws),
            _lib.ptr(dq), st3(dq), _lib.ptr(dk), st3(dk), _lib.ptr(dv), st3(dv), _lib.ptr(dw), st3(dw),
            _lib.ptr(db), bst(db), _lib.ptr(bws), B, T, H, HQ, K, float(ctx.scale), _lib.stream_handle(q.device))
        _lib.check(lib, rc, name)
        return (dq[:, :t], dk[:, :t], dv[:, :t], dw[:, :t], db[:, :t], None, None, None, None)


def _check(q, k, v, w, beta, g):
    assert q.shape[-1] in [16, 32, 64, 128], "only support head_dim in [16, 32, 64, 128] for now. Stay tuned!"
    assert v.shape[-1] in [16, 32, 64, 128], "only support head_dim in [16, 32, 64, 128] for now. Stay tuned!"
    assert q.shape[-1] == k.shape[-1], 'q, k should have the same head_dim.'
    assert k.shape == w.shape, 'k, w should have the same shape.'
    assert beta.shape[:3] == k.shape[:3], 'beta should have the same number of heads as k'
    assert g is None, 'g is not supported'
    assert q.shape[-2] % k.shape[-2] == 0, 'the number of query heads should be divisible by the number of key heads'
    if q.dtype not in (torch.bfloat16, torch.float32):
        raise TypeError(f"lucid_amd: q must be bfloat16 or float32, got {q.dtype}")
    for name, x in (("q", q), ("k", k), ("v", v), ("w", w), ("beta", beta)):
        if not x.is_cuda:
            raise RuntimeError(f"lucid_amd: {name} must be a GPU tensor (no CPU path)")
        if x.dtype != q.dtype:
            raise TypeError(f"lucid_amd: {name} must have q's dtype {q.dtype}, got {x.dtype}")
    if q.dtype == torch.float32 and max(q.shape[-1], v.shape[-1]) > _KDS[0]:
        raise NotImplementedError("lucid_amd: fp32 LUCID-Path runs at head dims up to 64 (bf16 up to 128)")


_KDS = (64, 128)  # head dims of the kernels (q, k, w and v rows share one)


def _pad_d(x: torch.Tensor, kd: int) -> torch.Tensor:
    """Zero-pad the head axis (last) to the kernels' kd columns (differentiable)."""
    return x if x.shape[-1] == kd else F.pad(x, (0, kd - x.shape[-1]))


def _apply(fn, q, k, v, w, beta, g, scale, cu_seqlens, use_cache):
    kd, vd = k.shape[-1], v.shape[-1]
    kk = _KDS[0] if max(kd, vd) <= _KDS[0] else _KDS[1]
    if kd != kk or vd != kk:
        pd = lambda x: _pad_d(x, kk)  # noqa: E731
        o, kc = _apply(fn, pd(q), pd(k), pd(v), pd(w), beta, g, scale, cu_seqlens, use_cache)
        return o[..., :vd], (kc[..., :kd] if kc is not None else None)
    if q.shape[1] == 0 or q.numel() == 0:  # empty: empty results, as the reference's ops give
        o = q.new_zeros(*q.shape[:3], v.shape[-1]) + 0 * (q.sum() + k.sum() + v.sum() + w.sum() + beta.sum())
        return o, (k.new_empty(k.shape) if use_cache else None)
    if cu_seqlens is None:
        return fn.apply(q, k, v, w, beta, g, scale, None, use_cache)
    # packed sequences [1, sum T_i, ...] (the reference's varlen mode, parallel.py:189,214-216):
    # sequences are bucketed by their length rounded up to the 64-position chunk, and each
    # bucket runs as one batched call on zero-padded sequences (exact: padding only follows
    # the real positions, and every operator here is causal)
    if q.shape[0] != 1:
        raise ValueError("cu_seqlens requires batch size 1 (packed sequences)")
    bounds = [int(x) for x in cu_seqlens.tolist()]
    if bounds[0] != 0 or bounds[-1] != q.shape[1] or any(b1 < b0 for b0, b1 in zip(bounds[:-1], bounds[1:])):
        raise ValueError("cu_seqlens must rise from 0 to the packed length")
    spans = [(b0, b1) for b0, b1 in zip(bounds[:-1], bounds[1:]) if b1 > b0]
    buckets: dict[int, list[int]] = {}
    for i, (b0, b1) in enumerate(spans):
        buckets.setdefault((b1 - b0 + 63) // 64 * 64, []).append(i)
    outs: list = [None] * len(spans)
    caches: list = [None] * len(spans)
    for tp, members in buckets.items():
        def stack(x):
            return torch.cat([_pad_t(x[:, spans[i][0]:spans[i][1]], tp) for i in members], 0)
        o_b, kc_b = fn.apply(stack(q), stack(k), stack(v), stack(w), stack(beta), g, scale, None, use_cache)
        for r, i in enumerate(members):
            n = spans[i][1] - spans[i][0]
            outs[i] = o_b[r:r + 1, :n]
            if use_cache:
                caches[i] = kc_b[r:r + 1, :n]
    return torch.cat(outs, 1), (torch.cat(caches, 1) if use_cache else None)


@torch.compiler.disable
def parallel_path_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    w: torch.Tensor,
    beta: torch.Tensor,
    g: Optional[torch.Tensor] = None,
    scale: float = None,
    cu_seqlens: Optional[torch.Tensor] = None,
    use_cache: bool = False,
):
    """PaTH softmax attention: O = softmax(s A) V over the path logits A (j <= i).

    q [B,T,HQ,K], k/w [B,T,H,K], v [B,T,H,V], beta [B,T,H]; returns
    ``(o [B,T,HQ,V], k_cache [B,T,H,K] or None)``.  Gating (``g``) is not supported,
    as in the LUCID-Path entry point.
    """
    if scale is None:
        scale = k.shape[-1] ** -0.5
    _check(q, k, v, w, beta, g)
    return _apply(ParallelPathAttentionFunction, q, k, v, w, beta, g, scale, cu_seqlens, use_cache)


@torch.compiler.disable
def parallel_lucid_path_attention(
    k: torch.Tensor,
    v: torch.Tensor,
    w: torch.Tensor,
    beta: torch.Tensor,
    q: Optional[torch.Tensor] = None,
    g: Optional[torch.Tensor] = None,
    scale: float = None,
    cu_seqlens: Optional[torch.Tensor] = None,
    use_cache: bool = False,
):
    """LUCID Path attention: solves (I + L) O = V with L = stril(exp(A * scale - 1/scale)).

    Same arguments, defaults and asserts as the reference (parallel.py:180-241);
    returns ``(o [B,T,HQ,V], k_cache [B,T,H,K] or None)``.
    """
    if q is None:
        q = k
    if scale is None:
        scale = k.shape[-1] ** -0.5
    _check(q, k, v, w, beta, g)
    return _apply(ParallelLUCIDPathAttentionFunction, q, k, v, w, beta, g, scale, cu_seqlens, use_cache)


def lucid_path_layer_attention(q, k, v, w, beta, scale=None):
    """One LUCID-Path layer's attention: V' = (I + L)^-1 V with the key-key path
    preconditioner (``parallel_lucid_path_attention`` with q = k), then PaTH softmax
    attention of the queries over (k, V')."""
    vp, _ = parallel_lucid_path_attention(k, v, w, beta, q=None, scale=scale)  # [B, T, H, V]
    o, _ = parallel_path_attention(q, k, vp, w, beta, scale=scale)
    return o
