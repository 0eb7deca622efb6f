"""LUCID attention operators on the HIP kernels (MI355X / gfx950).

Python mirror of the reference operator seams in ``modeling_lucid.py``:

* :func:`get_v_prime`      -- ``LucidAttention.get_v_prime`` (:551-574): V' = P^-1 V,
  differentiable (its backward is Lucid_Tril_Solver.backward, :314-382, and k_norm's)
* :func:`eager_lucid_attention_forward` -- ``LucidAttention.eager_lucid_attention_forward``
  (:505-549): O = softmax(s Q K^T, causal) V' for a given V', differentiable
* :func:`lucid_attention`  -- both in one call on the fused kernel sequence (the path
  LucidAttention.forward takes, :461-496)
* :func:`causal_attention` -- the same attention kernels with V' = V (plain causal attention)

Layouts follow the reference: ``query [B, Hq, T, d]``, ``key/value [B, Hkv, T, d]``
(any strides with a contiguous last axis, e.g. the ``.view(...).transpose(1, 2)``
views LucidAttention builds), output ``[B, T, Hq, d]``.  Inputs must be bf16 or fp32
CUDA(HIP) tensors with d <= 128 (fp32 is computed on bf16 hi/lo pairs to ~1e-4 relative,
fp32 outputs); anything else raises (there is no CPU or eager fallback).  T that is not a multiple of 128 is zero-padded at the end, which is exact for
every real row because P and the attention mask are causal.  Head dims other than 64 and
128 (the reference model's is 68) run on rows zero-padded to the next of the two, which
leaves every dot product unchanged; the RMS of k_norm divides by the true d.
"""
from __future__ import annotations

import contextlib

import torch
import torch.nn.functional as F

from . import _lib

_T_ALIGN = 128
_MAX_D = 128  # head dims up to 128: rows are zero-padded to 64 or 128 columns


def _padded_dim(d: int) -> int:
    return 64 if d <= 64 else 128


def _pad_d(t: torch.Tensor, dp: int) -> torch.Tensor:
    """Zero-pad the head axis (last) to ``dp`` columns (differentiable; a no-op at dp)."""
    return t if t.shape[-1] == dp else F.pad(t, (0, dp - t.shape[-1]))


def _check_inputs(q, k, v, f32_ok=False):
    """Shapes, device and dtype of the operands; ``f32_ok``: fp32 operands are accepted, all of
    one dtype."""
    for name, t in (("query", q), ("key", k), ("value", v)):
        if t is None:
            continue
        if not t.is_cuda:
            raise RuntimeError(f"lucid_amd: {name} must be a GPU tensor (no CPU path)")
        if t.dtype != torch.bfloat16 and not (f32_ok and t.dtype == torch.float32):
            raise TypeError(f"lucid_amd: {name} must be bfloat16{' or float32' if f32_ok else ''}, got {t.dtype}")
        if t.dim() != 4:
            raise ValueError(f"lucid_amd: {name} must be 4-D [B, H, T, d]")
    if len({t.dtype for t in (q, k, v) if t is not None}) > 1:
        raise TypeError("lucid_amd: query, key and value must share one dtype")
    if v is not None and k.shape != v.shape:
        raise ValueError(f"lucid_amd: key {tuple(k.shape)} and value {tuple(v.shape)} must match")
    d = k.shape[-1]
    if not 1 <= d <= _MAX_D:
        raise ValueError(f"lucid_amd: head_dim {d} not supported (supported: 1 .. {_MAX_D})")
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


def _fwd(q, k, v, scale, eps, dn):
    lib = _lib.load()
    B, Hq, T, D = q.shape
    Hkv = k.shape[1]
    dev = q.device
    o = torch.empty(B, T, Hq, D, dtype=torch.bfloat16, device=dev)
    vprime = torch.empty(B, Hkv, T, D, dtype=torch.float32, device=dev)
    lse = torch.empty(B, Hq, T, dtype=torch.float32, device=dev)
    ws = torch.empty(lib.lucid_fwd_workspace_bytes(B, Hq, Hkv, T, dn), dtype=torch.uint8, device=dev)
    rc = lib.lucid_attn_fwd(
        _lib.ptr(q), _lib.strides3(q, (0, 1, 2)), _lib.ptr(k), _lib.strides3(k, (0, 1, 2)),
        _lib.ptr(v), _lib.strides3(v, (0, 1, 2)), _lib.ptr(o), _lib.strides3(o, (0, 2, 1)),
        _lib.ptr(vprime), _lib.ptr(lse), _lib.ptr(ws), B, Hq, Hkv, T, dn, float(scale), float(eps),
        _lib.stream_handle(dev))
    _lib.check(lib, rc, "lucid_attn_fwd")
    return o, vprime, lse, ws


def _fwd_f32(q, k, v, scale, eps, dn):
    lib = _lib.load()
    B, Hq, T, D = q.shape
    Hkv = k.shape[1]
    dev = q.device
    o = torch.empty(B, T, Hq, D, dtype=torch.float32, device=dev)
    vprime = torch.empty(B, Hkv, T, D, dtype=torch.float32, device=dev)
    lse = torch.empty(B, Hq, T, dtype=torch.float32, device=dev)
    ws = torch.empty(lib.lucid_fwd_f32_workspace_bytes(B, Hq, Hkv, T, dn), dtype=torch.uint8, device=dev)
    rc = lib.lucid_attn_fwd_f32(
        _lib.ptr(q), _lib.strides3(q, (0, 1, 2)), _lib.ptr(k), _lib.strides3(k, (0, 1, 2)),
        _lib.ptr(v), _lib.strides3(v, (0, 1, 2)), _lib.ptr(o), _lib.strides3(o, (0, 2, 1)),
        _lib.ptr(vprime), _lib.ptr(lse), _lib.ptr(ws), B, Hq, Hkv, T, dn, float(scale), float(eps),
        _lib.stream_handle(dev))
    _lib.check(lib, rc, "lucid_attn_fwd_f32")
    return o, vprime, lse, ws


def _grad_buf(B, H, T, D, dtype, dev, time_major):
    """A [B, H, T, D] gradient buffer; time_major: stored as [B, T, H, D] (the layout of the
    usual ``proj(x).view(B, T, H, D).transpose(1, 2)`` operands, whose view backward then
    needs no copy)."""
    if time_major:
        return torch.empty(B, T, H, D, dtype=dtype, device=dev).transpose(1, 2)
    return torch.empty(B, H, T, D, dtype=dtype, device=dev)


def _time_major(x: torch.Tensor) -> bool:
    return x.dim() == 4 and x.shape[1] > 1 and x.stride(1) < x.stride(2)


def _bwd_f32(do, q, k, o, lse, ws, scale, dn, layouts=(False, False, False)):
    lib = _lib.load()
    B, Hq, T, D = q.shape
    Hkv = k.shape[1]
    dev = q.device
    dq = _grad_buf(B, Hq, T, D, torch.float32, dev, layouts[0])
    dk = _grad_buf(B, Hkv, T, D, torch.float32, dev, layouts[1])
    dv = _grad_buf(B, Hkv, T, D, torch.float32, dev, layouts[2])
    bws = torch.empty(lib.lucid_bwd_f32_workspace_bytes(B, Hq, Hkv, T, dn), dtype=torch.uint8, device=dev)
    rc = lib.lucid_attn_bwd_f32(
        _lib.ptr(do), _lib.strides3(do, (0, 2, 1)), _lib.ptr(o), _lib.strides3(o, (0, 2, 1)),
        _lib.ptr(lse), _lib.ptr(ws), _lib.ptr(dq), _lib.strides3(dq, (0, 1, 2)),
        _lib.ptr(dk), _lib.strides3(dk, (0, 1, 2)), _lib.ptr(dv), _lib.strides3(dv, (0, 1, 2)),
        _lib.ptr(bws), B, Hq, Hkv, T, dn, float(scale), _lib.stream_handle(dev))
    _lib.check(lib, rc, "lucid_attn_bwd_f32")
    return dq, dk, dv


def _bwd(do, q, k, o, lse, ws, scale, eps, dn, layouts=(False, False, False)):
    lib = _lib.load()
    B, Hq, T, D = q.shape
    Hkv = k.shape[1]
    dev = q.device
    dq = _grad_buf(B, Hq, T, D, torch.bfloat16, dev, layouts[0])
    dk = _grad_buf(B, Hkv, T, D, torch.bfloat16, dev, layouts[1])
    dv = _grad_buf(B, Hkv, T, D, torch.bfloat16, dev, layouts[2])
    bws = torch.empty(lib.lucid_bwd_workspace_bytes(B, Hq, Hkv, T, dn), dtype=torch.uint8, device=dev)
    rc = lib.lucid_attn_bwd(
        _lib.ptr(do), _lib.strides3(do, (0, 2, 1)), _lib.ptr(q), _lib.strides3(q, (0, 1, 2)),
        _lib.ptr(k), _lib.strides3(k, (0, 1, 2)), _lib.ptr(o), _lib.strides3(o, (0, 2, 1)),
        _lib.ptr(lse), _lib.ptr(ws), _lib.ptr(dq), _lib.strides3(dq, (0, 1, 2)),
        _lib.ptr(dk), _lib.strides3(dk, (0, 1, 2)), _lib.ptr(dv), _lib.strides3(dv, (0, 1, 2)),
        _lib.ptr(bws), B, Hq, Hkv, T, dn, float(scale), float(eps), _lib.stream_handle(dev))
    _lib.check(lib, rc, "lucid_attn_bwd")
    return dq, dk, dv


class LucidAttentionFunction(torch.autograd.Function):
    """O = softmax(s Q K^T, causal) (P^-1 V) with HIP forward and backward kernels.

    Gradients follow ``Lucid_Tril_Solver.backward`` (modeling_lucid.py:314-382)
    for the preconditioner and the softmax-attention backward for SDPA.
    """

    @staticmethod
    def forward(ctx, q, k, v, scale, eps, dn):
        t = q.shape[2]
        ctx.empty = t == 0 or q.numel() == 0
        ctx.shapes = (q.shape, k.shape)
        if ctx.empty:  # the reference's torch ops return empty results (no kernel launch)
            B, Hq, _, D = q.shape
            return (q.new_empty(B, t, Hq, D),
                    torch.empty(B, k.shape[1], t, D, dtype=torch.float32, device=q.device))
        tp = _padded_len(t)
        qp, kp, vp_ = _prep(q, tp), _prep(k, tp), _prep(v, tp)
        ctx.f32 = q.dtype == torch.float32
        o, vprime, lse, ws = (_fwd_f32 if ctx.f32 else _fwd)(qp, kp, vp_, scale, eps, dn)
        ctx.save_for_backward(qp, kp, o, lse, ws)
        ctx.scale, ctx.eps, ctx.t, ctx.dn = scale, eps, t, dn
        # the gradients are written in the memory order of the operands they belong to
        ctx.layouts = (_time_major(q), _time_major(k), _time_major(v))
        ctx.mark_non_differentiable(vprime)
        # no zero-filled gradient for the V' output, which the backward ignores (a T x d fp32
        # fill per call otherwise)
        ctx.set_materialize_grads(False)
        return o[:, :t], vprime[:, :, :t]

    @staticmethod
    def backward(ctx, do, _dvprime):
        if do is None:  # O took no part in the loss (gradients are not materialised)
            return None, None, None, None, None, None
        if ctx.empty:
            return (do.new_zeros(ctx.shapes[0]), do.new_zeros(ctx.shapes[1]), do.new_zeros(ctx.shapes[1]),
                    None, None, None)
        qp, kp, o, lse, ws = ctx.saved_tensors
        t, tp = ctx.t, qp.shape[2]
        dt = torch.float32 if ctx.f32 else torch.bfloat16
        if do.dtype != dt:
            do = do.to(dt)
        if t != tp:
            do = F.pad(do, (0, 0, 0, 0, 0, tp - t))
        if do.stride(-1) != 1 or any(s % 8 for s in do.stride()) or do.data_ptr() % 16:
            do = do.contiguous()
        if ctx.f32:
            dq, dk, dv = _bwd_f32(do, qp, kp, o, lse, ws, ctx.scale, ctx.dn, ctx.layouts)
        else:
            dq, dk, dv = _bwd(do, qp, kp, o, lse, ws, ctx.scale, ctx.eps, ctx.dn, ctx.layouts)
        return dq[:, :, :t], dk[:, :, :t], dv[:, :, :t], None, None, None


_PRECISIONS = {"auto": 0, "fast": 1, "exact": 2}


def set_precision(mode: str = "auto") -> None:
    """Precision of the preconditioner chains for the forward calls that follow on this thread.

    The mode is per thread (other threads keep theirs); a backward uses the choice its
    forward recorded, whatever thread it runs on.  :func:`precision` sets it for a block.

    ``"auto"`` (default) measures each head's row mass ``max_i sum_{j<i} P_ij^2`` (sampled)
    and runs heads above 4 -- keys along a shared direction, where the chain products
    cancel heavily -- through kernels that carry V' and dV as bf16 hi/lo pairs and split
    every product into three bf16 terms (~fp32 accuracy), the other heads through the bf16
    kernels.  ``"fast"`` and ``"exact"`` force one kind for every head.
    """
    if mode not in _PRECISIONS:
        raise ValueError(f"lucid_amd: precision must be one of {sorted(_PRECISIONS)}, got {mode!r}")
    lib = _lib.load()
    _lib.check(lib, lib.lucid_set_precision(_PRECISIONS[mode]), "lucid_set_precision")


def get_precision() -> str:
    code = _lib.load().lucid_get_precision()
    return {v: k for k, v in _PRECISIONS.items()}[code]


def set_fused_forward(on: bool = True) -> None:
    """Forward kernel schedule for the calls that follow on this thread (per thread, like
    :func:`set_precision`; :func:`fused_forward` sets it for a block).

    On (default): at head dim <= 64 with one query head per kv head the preconditioner chain
    and the causal attention of each 128-row block run in one fused kernel that feeds every
    staged key tile to both; off: the chain kernel, then the attention kernel.  The results
    agree up to the rounding order of the attention's online softmax.
    """
    lib = _lib.load()
    _lib.check(lib, lib.lucid_set_fused_forward(1 if on else 0), "lucid_set_fused_forward")


def get_fused_forward() -> bool:
    return bool(_lib.load().lucid_get_fused_forward())


@contextlib.contextmanager
def precision(mode: str):
    """``with precision("exact"): ...`` -- :func:`set_precision` for the block, restored after."""
    old = get_precision()
    set_precision(mode)
    try:
        yield
    finally:
        set_precision(old)


@contextlib.contextmanager
def fused_forward(on: bool):
    """``with fused_forward(False): ...`` -- :func:`set_fused_forward` for the block, restored after."""
    old = get_fused_forward()
    set_fused_forward(on)
    try:
        yield
    finally:
        set_fused_forward(old)


def head_row_mass(ws: torch.Tensor, B: int, Hq: int, Hkv: int, T: int, D: int) -> torch.Tensor:
    """Per-head row mass recorded in a forward workspace (float [B*Hkv]); heads above 4 ran the
    exact chain kernels.  ``T`` is the padded length the forward ran at."""
    lib = _lib.load()
    off = lib.lucid_fwd_workspace_mass_offset(B, Hq, Hkv, T, D)
    return ws[off:off + 4 * B * Hkv].view(torch.float32).clone()


def lucid_attention(query, key, value, scaling=None, eps=1e-5, return_vprime=False):
    """LUCID attention: ``softmax(s Q K^T, causal) P^-1 V``; returns O ``[B, T, Hq, d]``.

    ``eps`` is the k_norm epsilon (``config.rms_norm_eps``, modeling_lucid.py:409).
    bf16 inputs give bf16 O; fp32 inputs give fp32 O and gradients.
    """
    _check_inputs(query, key, value, f32_ok=True)
    d = query.shape[-1]
    scale = d ** -0.5 if scaling is None else float(scaling)
    dp = _padded_dim(d)
    q, k, v = (_pad_d(t, dp) for t in (query, key, value))
    o, vprime = LucidAttentionFunction.apply(q, k, v, scale, eps, d)
    if dp != d:
        o, vprime = o[..., :d], vprime[..., :d]
    return (o, vprime) if return_vprime else o


def _check_causal_mask(mask, lq, lk):
    """The reference's only mask is the causal one (create_causal_mask, modeling_lucid.py:600-618:
    bool, True where key j <= query i of the last ``lq`` rows); its training path ignores the mask
    and runs is_causal=True (:520-530).  The kernels are causal by construction, so a mask is
    accepted only if it is that one; anything else raises instead of being ignored silently."""
    if mask is None:
        return
    if not torch.is_tensor(mask) or mask.dtype != torch.bool or mask.dim() < 2:
        raise NotImplementedError("lucid_amd: attention_mask must be None or the causal bool mask")
    m = mask[..., -lq:, :lk]
    if m.shape[-2:] != (lq, lk):
        raise ValueError(f"lucid_amd: attention_mask {tuple(mask.shape)} does not cover {lq} x {lk}")
    causal = torch.ones(lq, lk, dtype=torch.bool, device=mask.device).tril_(lk - lq)
    if not bool((m == causal).all()):
        raise NotImplementedError("lucid_amd: only the causal attention mask is supported")


class GetVPrimeFunction(torch.autograd.Function):
    """``V' = P(K^)^-1 V`` with its own backward (Lucid_Tril_Solver.backward,
    modeling_lucid.py:314-382, and the k_norm backward): C ``lucid_get_v_prime`` /
    ``lucid_precond_bwd``.  V' is returned in the dtype of ``value`` like the reference's
    ``solve_triangular``; the backward uses the forward's fp32 solve state."""

    @staticmethod
    def forward(ctx, key, value, scale, eps, dn, knorm=True):
        B, Hkv, T, D = key.shape
        ctx.shape, ctx.t, ctx.knorm = key.shape, T, knorm
        if T == 0 or key.numel() == 0:
            ctx.empty = True
            return value.new_empty(B, Hkv, T, D)
        ctx.empty = False
        lib = _lib.load()
        tp = _padded_len(T)
        k, v = _prep(key, tp), _prep(value, tp)
        ctx.f32 = key.dtype == torch.float32
        vprime = torch.empty(B, Hkv, tp, D, dtype=torch.float32, device=key.device)
        if ctx.f32:
            ws = torch.empty(lib.lucid_v_prime_f32_workspace_bytes(B, Hkv, tp, dn), dtype=torch.uint8,
                             device=key.device)
            name = "lucid_get_v_prime_f32" if knorm else "lucid_tril_solve_f32"
        else:
            ws = torch.empty(lib.lucid_fwd_workspace_bytes(B, Hkv, Hkv, tp, dn), dtype=torch.uint8, device=key.device)
            name = "lucid_get_v_prime" if knorm else "lucid_tril_solve"
        args = [_lib.ptr(k), _lib.strides3(k, (0, 1, 2)), _lib.ptr(v), _lib.strides3(v, (0, 1, 2)),
                _lib.ptr(vprime), _lib.ptr(ws), B, Hkv, tp, dn, scale]
        if knorm:  # k_norm's epsilon (the solver seam takes normalised keys)
            args.append(float(eps))
        rc = getattr(lib, name)(*args, _lib.stream_handle(key.device))
        _lib.check(lib, rc, name)
        ctx.save_for_backward(k, ws)
        ctx.scale, ctx.dn = scale, dn
        return vprime[:, :, :T].to(value.dtype)

    @staticmethod
    def backward(ctx, dvp):
        if ctx.empty:
            return dvp.new_zeros(ctx.shape), dvp.new_zeros(ctx.shape), None, None, None, None
        k, ws = ctx.saved_tensors
        lib = _lib.load()
        B, Hkv, tp, D = k.shape
        t, dn = ctx.t, ctx.dn
        bws = torch.empty(lib.lucid_precond_bwd_workspace_bytes(B, Hkv, tp, dn), dtype=torch.uint8, device=k.device)
        if ctx.f32:  # fp32 inputs: fp32 dV' in, fp32 dK and dV out
            dvp = _prep(dvp.float(), tp)
            dk = torch.empty(B, Hkv, tp, D, dtype=torch.float32, device=k.device)
            dv = torch.empty_like(dk)
            name = "lucid_precond_bwd_f32" if ctx.knorm else "lucid_tril_solve_bwd_f32"
            rc = getattr(lib, name)(_lib.ptr(dvp), _lib.strides3(dvp, (0, 1, 2)), _lib.ptr(ws), _lib.ptr(dk),
                                    _lib.strides3(dk, (0, 1, 2)), _lib.ptr(dv), _lib.strides3(dv, (0, 1, 2)),
                                    _lib.ptr(bws), B, Hkv, tp, dn, ctx.scale, _lib.stream_handle(k.device))
            _lib.check(lib, rc, name)
            return dk[:, :, :t], dv[:, :, :t], None, None, None, None
        f32 = dvp.dtype == torch.float32
        if not f32 and dvp.dtype != torch.bfloat16:
            dvp = dvp.to(torch.bfloat16)
        dvp = _prep(dvp, tp)
        dk = torch.empty(B, Hkv, tp, D, dtype=torch.bfloat16, device=k.device)
        dv = torch.empty_like(dk)
        name = "lucid_precond_bwd" if ctx.knorm else "lucid_tril_solve_bwd"
        rc = getattr(lib, name)(_lib.ptr(k), _lib.strides3(k, (0, 1, 2)), _lib.ptr(dvp), _lib.strides3(dvp, (0, 1, 2)),
                                int(f32), _lib.ptr(ws), _lib.ptr(dk), _lib.strides3(dk, (0, 1, 2)), _lib.ptr(dv),
                                _lib.strides3(dv, (0, 1, 2)), _lib.ptr(bws), B, Hkv, tp, dn, ctx.scale,
                                _lib.stream_handle(k.device))
        _lib.check(lib, rc, name)
        return dk[:, :, :t], dv[:, :, :t], None, None, None, None


class AttentionOnVPrimeFunction(torch.autograd.Function):
    """``O = softmax(s Q K^T, causal) V'`` for a given V' (eager_lucid_attention_forward,
    modeling_lucid.py:505-549), with dV' in the backward: C ``lucid_attn_vp_fwd`` /
    ``lucid_attn_vp_bwd``."""

    @staticmethod
    def forward(ctx, q, k, vp, scale, eps, dn):
        B, Hq, T, D = q.shape
        Hkv = k.shape[1]
        ctx.shapes, ctx.t, ctx.vdtype = (q.shape, k.shape, vp.shape), T, vp.dtype
        if T == 0 or q.numel() == 0:
            ctx.empty = True
            return q.new_empty(B, T, Hq, D)
        ctx.empty = False
        lib = _lib.load()
        tp = _padded_len(T)
        qp, kp = _prep(q, tp), _prep(k, tp)
        dev = q.device
        ctx.f32in = q.dtype == torch.float32
        if ctx.f32in:  # fp32 q and k: the fp32 kernels, V' in fp32
            vpp = _prep(vp.float(), tp)
            o = torch.empty(B, tp, Hq, D, dtype=torch.float32, device=dev)
            lse = torch.empty(B, Hq, tp, dtype=torch.float32, device=dev)
            ws = torch.empty(lib.lucid_attn_vp_fwd_f32_workspace_bytes(B, Hq, Hkv, tp, dn), dtype=torch.uint8,
                             device=dev)
            rc = lib.lucid_attn_vp_fwd_f32(_lib.ptr(qp), _lib.strides3(qp, (0, 1, 2)), _lib.ptr(kp),
                                           _lib.strides3(kp, (0, 1, 2)), _lib.ptr(vpp), _lib.strides3(vpp, (0, 1, 2)),
                                           _lib.ptr(o), _lib.strides3(o, (0, 2, 1)), _lib.ptr(lse), _lib.ptr(ws),
                                           B, Hq, Hkv, tp, dn, scale, float(eps), _lib.stream_handle(dev))
            _lib.check(lib, rc, "lucid_attn_vp_fwd_f32")
            ctx.save_for_backward(qp, kp, o, lse, ws)
            ctx.scale, ctx.dn = scale, dn
            return o[:, :T]
        f32 = vp.dtype == torch.float32
        vpp = _prep(vp if f32 else vp.to(torch.bfloat16), tp)
        o = torch.empty(B, tp, Hq, D, dtype=torch.bfloat16, device=dev)
        lse = torch.empty(B, Hq, tp, dtype=torch.float32, device=dev)
        ws = torch.empty(lib.lucid_attn_vp_fwd_workspace_bytes(B, Hq, Hkv, tp, dn), dtype=torch.uint8, device=dev)
        rc = lib.lucid_attn_vp_fwd(_lib.ptr(qp), _lib.strides3(qp, (0, 1, 2)), _lib.ptr(kp), _lib.strides3(kp, (0, 1, 2)),
                                   _lib.ptr(vpp), _lib.strides3(vpp, (0, 1, 2)), int(f32), _lib.ptr(o),
                                   _lib.strides3(o, (0, 2, 1)), _lib.ptr(lse), _lib.ptr(ws), B, Hq, Hkv, tp, dn, scale,
                                   float(eps), _lib.stream_handle(dev))
        _lib.check(lib, rc, "lucid_attn_vp_fwd")
        ctx.save_for_backward(qp, kp, o, lse, ws)
        ctx.scale, ctx.dn = scale, dn
        return o[:, :T]

    @staticmethod
    def backward(ctx, do):
        qs, ks, vs = ctx.shapes
        if ctx.empty:
            return (do.new_zeros(qs), do.new_zeros(ks), torch.zeros(vs, dtype=ctx.vdtype, device=do.device),
                    None, None, None)
        qp, kp, o, lse, ws = ctx.saved_tensors
        lib = _lib.load()
        B, Hq, tp, D = qp.shape
        Hkv, t, dn = kp.shape[1], ctx.t, ctx.dn
        dt = torch.float32 if ctx.f32in else torch.bfloat16
        if do.dtype != dt:
            do = do.to(dt)
        if t != tp:
            do = F.pad(do, (0, 0, 0, 0, 0, tp - t))
        if do.stride(-1) != 1 or any(s % 8 for s in do.stride()) or do.data_ptr() % 16:
            do = do.contiguous()
        dev = qp.device
        if ctx.f32in:
            dq = torch.empty(B, Hq, tp, D, dtype=torch.float32, device=dev)
            dk = torch.empty(B, Hkv, tp, D, dtype=torch.float32, device=dev)
            dvp = torch.empty(B, Hkv, tp, D, dtype=torch.float32, device=dev)
            bws = torch.empty(lib.lucid_attn_vp_bwd_f32_workspace_bytes(B, Hq, Hkv, tp, dn), dtype=torch.uint8,
                              device=dev)
            rc = lib.lucid_attn_vp_bwd_f32(_lib.ptr(do), _lib.strides3(do, (0, 2, 1)), _lib.ptr(o),
                                           _lib.strides3(o, (0, 2, 1)), _lib.ptr(lse), _lib.ptr(ws), _lib.ptr(dq),
                                           _lib.strides3(dq, (0, 1, 2)), _lib.ptr(dk), _lib.strides3(dk, (0, 1, 2)),
                                           _lib.ptr(dvp), _lib.strides3(dvp, (0, 1, 2)), _lib.ptr(bws),
                                           B, Hq, Hkv, tp, dn, ctx.scale, _lib.stream_handle(dev))
            _lib.check(lib, rc, "lucid_attn_vp_bwd_f32")
            return dq[:, :, :t], dk[:, :, :t], dvp[:, :, :t].to(ctx.vdtype), None, None, None
        f32 = ctx.vdtype == torch.float32
        dq = torch.empty(B, Hq, tp, D, dtype=torch.bfloat16, device=dev)
        dk = torch.empty(B, Hkv, tp, D, dtype=torch.bfloat16, device=dev)
        dvp = torch.empty(B, Hkv, tp, D, dtype=torch.float32 if f32 else torch.bfloat16, device=dev)
        bws = torch.empty(lib.lucid_attn_vp_bwd_workspace_bytes(B, Hq, Hkv, tp, dn), dtype=torch.uint8, device=dev)
        rc = lib.lucid_attn_vp_bwd(_lib.ptr(do), _lib.strides3(do, (0, 2, 1)), _lib.ptr(qp), _lib.strides3(qp, (0, 1, 2)),
                                   _lib.ptr(kp), _lib.strides3(kp, (0, 1, 2)), _lib.ptr(o), _lib.strides3(o, (0, 2, 1)),
                                   _lib.ptr(lse), _lib.ptr(ws), _lib.ptr(dq), _lib.strides3(dq, (0, 1, 2)), _lib.ptr(dk),
                                   _lib.strides3(dk, (0, 1, 2)), _lib.ptr(dvp), _lib.strides3(dvp, (0, 1, 2)), int(f32),
                                   _lib.ptr(bws), B, Hq, Hkv, tp, dn, ctx.scale, _lib.stream_handle(dev))
        _lib.check(lib, rc, "lucid_attn_vp_bwd")
        dvp = dvp[:, :, :t]
        if dvp.dtype != ctx.vdtype:
            dvp = dvp.to(ctx.vdtype)
        return dq[:, :, :t], dk[:, :, :t], dvp, None, None, None


def get_v_prime(key, value, scaling=None, attention_mask=None, eps=1e-5):
    """``V' = P^-1 V`` -- ``LucidAttention.get_v_prime(key, value, scaling, attention_mask)``
    (modeling_lucid.py:551-574), differentiable w.r.t. ``key`` and ``value``.

    ``key, value [B, Hkv, T, d]`` (bf16 or fp32, d <= 128); returns V' in ``value``'s dtype.
    ``eps`` is k_norm's epsilon (``config.rms_norm_eps``).  ``attention_mask``: None or the
    causal mask."""
    _check_inputs(None, key, value, f32_ok=True)
    _check_causal_mask(attention_mask, key.shape[2], key.shape[2])
    d = key.shape[-1]
    scale = d ** -0.5 if scaling is None else float(scaling)
    dp = _padded_dim(d)
    vprime = GetVPrimeFunction.apply(_pad_d(key, dp), _pad_d(value, dp), scale, eps, d)
    return vprime if dp == d else vprime[..., :d]


class Lucid_Tril_Solver:  # noqa: N801  (the reference's class name)
    """Drop-in for ``Lucid_Tril_Solver`` (modeling_lucid.py:284-382): ``Lucid_Tril_Solver.apply(key,
    value, scaling, BS=2**14)`` solves ``P V' = V`` for keys that are already normalised
    (``key`` is K^: the reference's get_v_prime applies k_norm before calling it, :562-565), with
    ``P_ij = exp(scaling K^_i . K^_j - 1/scaling)`` for j <= i.  Differentiable w.r.t. ``key``
    and ``value``; the gradient is the reference backward's ``(grad_k, grad_v, None, None)``:
    ``dV = P^-T dV'``, ``dK^ = -scaling (M K^ + M^T K^)``, ``M = tril((dV V'^T) * P)`` (no
    RMSNorm backward).  C ``lucid_tril_solve`` / ``lucid_tril_solve_bwd`` (``_f32`` for fp32).

    ``BS`` is the reference's block size; as there, ``T`` must exceed it and be a multiple of it
    (``AssertionError`` otherwise, :287-288).  The solve itself is the library's chained
    blockwise one, so the result does not depend on ``BS``; ``value`` is left unmodified (the
    reference subtracts from its rows in place, :296-299).  Layouts ``[B, Hkv, T, d]``, bf16
    or fp32 with d <= 128; V' comes back in ``value``'s dtype.
    """

    @staticmethod
    def apply(key, value, scaling, BS=2 ** 14):
        L = key.shape[-2]
        assert L > BS, f"Sequence length {L} must be greater than block size {BS}."
        assert L % BS == 0, f"Sequence length {L} must be divisible by block size {BS}."
        _check_inputs(None, key, value, f32_ok=True)
        d = key.shape[-1]
        dp = _padded_dim(d)
        vprime = GetVPrimeFunction.apply(_pad_d(key, dp), _pad_d(value, dp), float(scaling), 0.0, d, False)
        return vprime if dp == d else vprime[..., :d]


def eager_lucid_attention_forward(query, key, v_prime, scaling=None, attention_mask=None, eps=1e-5, **kwargs):
    """``LucidAttention.eager_lucid_attention_forward(query, key, v_prime, scaling, attention_mask)``
    (modeling_lucid.py:505-549): causal softmax attention of ``query [B, Hq, T, d]`` and
    ``key [B, Hkv, T, d]`` on a given ``v_prime [B, Hkv, T, d]`` (bf16 or fp32; GQA by index,
    no repeat_kv copy).  fp32 query and key run the fp32 kernels (fp32 O).  Returns
    ``(O [B, T, Hq, d], None)``, differentiable w.r.t. all three.
    ``attention_mask``: None or the causal mask.  ``eps`` (k_norm's) only serves the per-head
    precision choice (:func:`set_precision`)."""
    _check_inputs(query, key, None, f32_ok=True)
    if v_prime.shape != key.shape or not v_prime.is_cuda or v_prime.dtype not in (torch.bfloat16, torch.float32):
        raise ValueError("lucid_amd: v_prime must be a bf16 or fp32 GPU tensor shaped like key")
    _check_causal_mask(attention_mask, query.shape[2], key.shape[2])
    d = query.shape[-1]
    scale = d ** -0.5 if scaling is None else float(scaling)
    dp = _padded_dim(d)
    o = AttentionOnVPrimeFunction.apply(_pad_d(query, dp), _pad_d(key, dp), _pad_d(v_prime, dp), scale, eps, d)
    return (o if dp == d else o[..., :d]), None


def causal_attention(query, key, value, scaling=None):
    """Plain causal softmax attention on the same HIP kernels (V' = V): ``O [B, T, Hq, d]``.

    The build's own comparator for the cost of the preconditioner (no counterpart in the
    reference, which calls SDPA)."""
    return eager_lucid_attention_forward(query, key, value, scaling)[0]


def lucid_decode(query, key, value, key_cache, vprime_cache, cache_len, scaling=None, eps=1e-5):
    """A decoding step for L new tokens per sequence (``get_new_v_prime`` for ``L_k`` new
    tokens and the cached attention of LucidAttention.forward, modeling_lucid.py:475-496,
    576-598), in one call.

    ``query [B, Hq, L, d]``, ``key/value [B, Hkv, L, d]`` (bf16; keys with RoPE applied;
    the L tokens in sequence order); ``key_cache`` / ``vprime_cache`` are bf16 buffers
    ``[B, Hkv, T_cap, dp]`` whose first ``cache_len`` rows are valid, ``dp`` = 64 for
    d <= 64 and 128 above (columns beyond d zero: the head rows zero-padded).  Each token's
    V' row is the prefill row (exact diagonal, coupled to the cache and to the earlier new
    tokens: ``v'_t = (v_t - sum_{j<t} P_tj v'_j) / P_tt``) and each token attends to the
    cache and to the new tokens up to itself; the keys and V' rows are written at rows
    ``cache_len .. cache_len + L - 1`` of the caches in place.  Returns
    ``(O [B, L, Hq, d], V' fp32 [B, Hkv, L, d])``.
    """
    _check_inputs(None, key, value)
    for name, t in (("query", query), ("key_cache", key_cache), ("vprime_cache", vprime_cache)):
        if not t.is_cuda or t.dtype != torch.bfloat16 or t.dim() != 4:
            raise TypeError(f"lucid_amd: {name} must be a 4-D bfloat16 GPU tensor")
    for name, t in (("key_cache", key_cache), ("vprime_cache", vprime_cache)):  # written in place: no copies
        if t.stride(-1) != 1 or any(s % 8 for s in t.stride()[:3]) or t.data_ptr() % 16:
            raise ValueError(f"lucid_amd: {name} needs a contiguous last axis and 8-element aligned strides")
    B, Hkv, L, d = key.shape
    Hq = query.shape[1]
    D = _padded_dim(d)
    if query.shape[0] != B or query.shape[2] != L or query.shape[3] != d or Hq % Hkv:
        raise ValueError("lucid_amd: query [B, Hq, L, d] disagrees with key [B, Hkv, L, d]")
    if key_cache.shape[:2] != (B, Hkv) or vprime_cache.shape != key_cache.shape or key_cache.shape[3] != D:
        raise ValueError(f"lucid_amd: cache buffers must be [B, Hkv, T_cap, {D}] for head_dim {d}")
    lib = _lib.load()
    cap = key_cache.shape[2]
    if L == 0:
        return (query.new_empty(B, 0, Hq, d), torch.empty(B, Hkv, 0, d, dtype=torch.float32, device=query.device))
    q, k, v = (_prep(_pad_d(t, D), L) for t in (query, key, value))
    o = torch.empty(B, L, Hq, D, dtype=torch.bfloat16, device=q.device)
    vp_new = torch.empty(B, Hkv, L, D, dtype=torch.float32, device=q.device)
    ws = torch.empty(max(lib.lucid_decode_tokens_workspace_bytes(B, Hq, Hkv, L, cap, d), 256), dtype=torch.uint8,
                     device=q.device)
    scale = d ** -0.5 if scaling is None else float(scaling)
    rc = lib.lucid_decode_tokens(
        _lib.ptr(q), _lib.strides3(q, (0, 1, 2)), _lib.ptr(k), _lib.strides3(k, (0, 1, 2)),
        _lib.ptr(v), _lib.strides3(v, (0, 1, 2)), _lib.ptr(key_cache), _lib.strides3(key_cache, (0, 1, 2)),
        _lib.ptr(vprime_cache), _lib.strides3(vprime_cache, (0, 1, 2)), _lib.ptr(o), _lib.strides3(o, (0, 2, 1)),
        _lib.ptr(vp_new), _lib.ptr(ws), B, Hq, Hkv, L, int(cache_len), cap, d, scale, float(eps),
        _lib.stream_handle(q.device))
    _lib.check(lib, rc, "lucid_decode_tokens")
    return (o, vp_new) if D == d else (o[..., :d], vp_new[..., :d])
