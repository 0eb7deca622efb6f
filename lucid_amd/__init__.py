"""lucid_amd -- LUCID attention and LUCID-Path for AMD MI355X (gfx950) on hand-written HIP kernels.

Operator entry points (drop-ins for the reference seams):

* :func:`lucid_amd.lucid.lucid_attention` / :func:`lucid_amd.lucid.get_v_prime` /
  :func:`lucid_amd.lucid.eager_lucid_attention_forward` (modeling_lucid.py operator part)
* :func:`lucid_amd.lucid.lucid_decode` (one decoding step against a (K, V') cache)
* :func:`lucid_amd.lucid.set_precision` (bf16 or hi/lo-split chain products, chosen per head by default)
* :func:`lucid_amd.lucid.set_fused_forward` (one fused chain + attention kernel, or two kernels)
* :mod:`lucid_amd.modeling_lucid` (the reference model file's classes on these operators)
* :mod:`lucid_amd.model_ops` (fused RMSNorm, RoPE, SwiGLU gate and causal-LM loss of the decoder)
* :mod:`lucid_amd.optim` (AdamW on one HIP pass per step)
* :mod:`lucid_amd.lucid_path` (LUCID-Path and PaTH softmax attention)
"""
from .lucid import (LucidAttentionFunction, causal_attention, eager_lucid_attention_forward, get_fused_forward,
                    get_precision, get_v_prime, lucid_attention, lucid_decode, set_fused_forward, set_precision)

__all__ = [
    "LucidAttentionFunction",
    "causal_attention",
    "eager_lucid_attention_forward",
    "get_fused_forward",
    "get_precision",
    "get_v_prime",
    "lucid_attention",
    "lucid_decode",
    "set_fused_forward",
    "set_precision",
]
