"""Llama-architecture decoder with LUCID attention on the HIP kernels.

Mirror of the reference model file (``modeling_lucid.py``): the module tree and
parameter names follow it (``model.layers.N.self_attn.q_proj`` ...), so its state
dicts load unchanged, and ``LucidAttention.forward`` keeps the reference signature
(``modeling_lucid.py:421-503``).  The attention core -- K^ = RMSNorm(K), the
preconditioner solve V' = P^-1 V and causal softmax attention on V' -- runs in
``lucid_amd.lucid_attention`` (HIP); RMSNorm, RoPE, the SwiGLU gate and the loss on bf16
GPU activations run as one HIP kernel pass each way (``lucid_amd.model_ops``; the torch
expressions otherwise); embeddings and the projections / LM head are plain PyTorch (hipBLASLt
GEMMs).

Decoding with a cache (``get_new_v_prime``, ``modeling_lucid.py:576-598``) keeps
(K, V') per layer and runs the HIP decoding step ``lucid_decode``.  The new rows of V'
follow the prefill definition exactly:
v'_t = (v_t - sum_{j<t} P_tj v'_j) / P_tt with the non-unit diagonal
P_tt = exp(s |K^_t|^2 - 1/s), so a decoded token gets the same V' row as the same
token inside a prefill (the reference's decode path drops the division by P_tt).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch
import torch.nn as nn
import torch.nn.functional as F

from .lucid import _padded_dim, lucid_attention, lucid_decode
from .model_ops import (apply_rope, causal_lm_loss, causal_lm_loss_supported, qkv_rope, rms_norm,
                        rms_norm_supported, rope_supported, swiglu, swiglu_supported)


@dataclass
class LucidConfig:
    vocab_size: int = 32000
    hidden_size: int = 2048
    intermediate_size: int = 5632
    num_hidden_layers: int = 16
    num_attention_heads: int = 32
    num_key_value_heads: Optional[int] = None
    head_dim: Optional[int] = None
    rms_norm_eps: float = 1e-5
    rope_theta: float = 10000.0
    max_position_embeddings: int = 131072
    attention_bias: bool = False
    mlp_bias: bool = False
    use_rope: bool = True
    tie_word_embeddings: bool = False
    initializer_range: float = 0.02

    def __post_init__(self):
        if self.num_key_value_heads is None:
            self.num_key_value_heads = self.num_attention_heads
        if self.head_dim is None:
            self.head_dim = self.hidden_size // self.num_attention_heads


class LlamaRMSNorm(nn.Module):
    """modeling_lucid.py:58-75 (float32 statistics, weight applied in the input dtype)."""

    def __init__(self, hidden_size: int, eps: float = 1e-6):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(hidden_size))
        self.variance_epsilon = eps

    def forward(self, hidden_states: torch.Tensor) -> torch.Tensor:
        if rms_norm_supported(hidden_states, self.weight):
            return rms_norm(hidden_states, self.weight, self.variance_epsilon)  # one HIP pass each way
        input_dtype = hidden_states.dtype
        x = hidden_states.to(torch.float32)
        x = x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + self.variance_epsilon)
        return self.weight * x.to(input_dtype)


class LlamaRotaryEmbedding(nn.Module):
    """Default RoPE (modeling_lucid.py:78-110): cos/sin of position * theta^(-2i/d)."""

    def __init__(self, config: LucidConfig, device=None):
        super().__init__()
        d = config.head_dim
        inv_freq = 1.0 / (config.rope_theta ** (torch.arange(0, d, 2, dtype=torch.int64, device=device).float() / d))
        self.register_buffer("inv_freq", inv_freq, persistent=False)

    @torch.no_grad()
    def forward(self, x: torch.Tensor, position_ids: torch.Tensor):
        freqs = position_ids[:, :, None].float() * self.inv_freq[None, None, :].to(x.device)
        emb = torch.cat((freqs, freqs), dim=-1)
        return emb.cos().to(x.dtype), emb.sin().to(x.dtype)


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    x1, x2 = x[..., : x.shape[-1] // 2], x[..., x.shape[-1] // 2:]
    return torch.cat((-x2, x1), dim=-1)


def apply_rotary_pos_emb(q, k, cos, sin, unsqueeze_dim: int = 1):
    """modeling_lucid.py:118-145."""
    if unsqueeze_dim == 1 and rope_supported(q, cos) and rope_supported(k, cos):
        return apply_rope(q, cos, sin), apply_rope(k, cos, sin)  # one HIP pass each way
    cos, sin = cos.unsqueeze(unsqueeze_dim), sin.unsqueeze(unsqueeze_dim)
    return (q * cos) + (rotate_half(q) * sin), (k * cos) + (rotate_half(k) * sin)


class LlamaMLP(nn.Module):
    """SwiGLU feed-forward (modeling_lucid.py:155-167)."""

    def __init__(self, config: LucidConfig):
        super().__init__()
        self.gate_proj = nn.Linear(config.hidden_size, config.intermediate_size, bias=config.mlp_bias)
        self.up_proj = nn.Linear(config.hidden_size, config.intermediate_size, bias=config.mlp_bias)
        self.down_proj = nn.Linear(config.intermediate_size, config.hidden_size, bias=config.mlp_bias)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        g, u = self.gate_proj(x), self.up_proj(x)
        if swiglu_supported(g, u):
            return self.down_proj(swiglu(g, u))  # one HIP pass each way
        return self.down_proj(F.silu(g) * u)


class LucidCache:
    """Per-layer (K with RoPE applied, V') cache for decoding (the reference keeps the same
    pair in a DynamicCache, modeling_lucid.py:479-481).  Rows live in preallocated bf16
    buffers [B, Hkv, capacity, dp] that grow by doubling, so a decoding step appends in
    place instead of concatenating the whole cache (dp: the head dim d zero-padded to 64 or
    128, the row width of the decoding kernel); ``key_cache`` / ``value_cache`` give the
    valid rows [B, Hkv, T, d]."""

    def __init__(self, min_capacity: int = 256):
        self._k: list[torch.Tensor] = []
        self._v: list[torch.Tensor] = []
        self._len: list[int] = []
        self._d: list[int] = []
        self.min_capacity = min_capacity

    @property
    def key_cache(self) -> list[torch.Tensor]:
        return [k[:, :, :n, :d] for k, n, d in zip(self._k, self._len, self._d)]

    @property
    def value_cache(self) -> list[torch.Tensor]:
        return [v[:, :, :n, :d] for v, n, d in zip(self._v, self._len, self._d)]

    def get_seq_length(self, layer_idx: int = 0) -> int:
        return self._len[layer_idx] if layer_idx < len(self._len) else 0

    def reserve(self, layer_idx: int, like: torch.Tensor, extra: int) -> None:
        """Make room for ``extra`` more rows of layer ``layer_idx`` (``like``: [B, Hkv, *, d])."""
        n = self.get_seq_length(layer_idx)
        if layer_idx == len(self._k):
            cap = max(self.min_capacity, -(-extra // 256) * 256)
            d = like.shape[3]
            shape = (like.shape[0], like.shape[1], cap, _padded_dim(d))
            alloc = torch.empty if shape[3] == d else torch.zeros  # padded columns stay zero
            self._k.append(alloc(shape, dtype=torch.bfloat16, device=like.device))
            self._v.append(alloc(shape, dtype=torch.bfloat16, device=like.device))
            self._len.append(0)
            self._d.append(d)
            return
        cap = self._k[layer_idx].shape[2]
        if n + extra <= cap:
            return
        new_cap = max(2 * cap, -(-(n + extra) // 256) * 256)
        for bufs in (self._k, self._v):
            old = bufs[layer_idx]
            alloc = torch.empty if old.shape[3] == self._d[layer_idx] else torch.zeros
            grown = alloc(old.shape[0], old.shape[1], new_cap, old.shape[3], dtype=old.dtype, device=old.device)
            grown[:, :, :n] = old[:, :, :n]
            bufs[layer_idx] = grown

    def buffers(self, layer_idx: int):
        return self._k[layer_idx], self._v[layer_idx], self._len[layer_idx]

    def advance(self, layer_idx: int, n: int = 1) -> None:
        self._len[layer_idx] += n

    def update(self, key: torch.Tensor, v_prime: torch.Tensor, layer_idx: int):
        """Append rows (prefill); returns the valid (K, V') of the layer."""
        self.reserve(layer_idx, key, key.shape[2])
        k, v, n = self.buffers(layer_idx)
        t = key.shape[2]
        d = self._d[layer_idx]
        k[:, :, n:n + t, :d] = key
        v[:, :, n:n + t, :d] = v_prime
        self._len[layer_idx] = n + t
        return k[:, :, :n + t, :d], v[:, :, :n + t, :d]


_STACKED_QKV_MIN_NUMEL = 1 << 20  # activations at least this large take one stacked q/k/v GEMM


class LucidAttention(nn.Module):
    """LUCID attention module (modeling_lucid.py:385-503) on the HIP kernels."""

    def __init__(self, config: LucidConfig, layer_idx: int):
        super().__init__()
        self.config = config
        self.layer_idx = layer_idx
        self.head_dim = config.head_dim
        self.num_key_value_groups = config.num_attention_heads // config.num_key_value_heads
        self.scaling = self.head_dim ** -0.5
        self.is_causal = True
        self.use_rope = config.use_rope
        self.q_proj = nn.Linear(config.hidden_size, config.num_attention_heads * self.head_dim,
                                bias=config.attention_bias)
        self.k_proj = nn.Linear(config.hidden_size, config.num_key_value_heads * self.head_dim,
                                bias=config.attention_bias)
        self.v_proj = nn.Linear(config.hidden_size, config.num_key_value_heads * self.head_dim,
                                bias=config.attention_bias)
        # k_norm carries no parameters (modeling_lucid.py:409); it is applied inside the fused op
        self.o_proj = nn.Linear(config.num_attention_heads * self.head_dim, config.hidden_size,
                                bias=config.attention_bias)

    def forward(self, hidden_states: torch.Tensor, position_embeddings: tuple[torch.Tensor, torch.Tensor],
                attention_mask: Optional[torch.Tensor] = None, past_key_value: Optional[LucidCache] = None,
                cache_position: Optional[torch.Tensor] = None, **kwargs):
        input_shape = hidden_states.shape[:-1]
        hidden_shape = (*input_shape, -1, self.head_dim)
        if hidden_states.is_cuda and hidden_states.numel() >= _STACKED_QKV_MIN_NUMEL:
            # one GEMM over the stacked q / k / v weights (the parameters stay separate): on
            # long inputs its weight gradient runs at ~1.5x the rate of three narrow ones
            qkv = F.linear(hidden_states, torch.cat((self.q_proj.weight, self.k_proj.weight, self.v_proj.weight)),
                           None if self.q_proj.bias is None else
                           torch.cat((self.q_proj.bias, self.k_proj.bias, self.v_proj.bias)))
            nq, nk = self.q_proj.out_features, self.k_proj.out_features
            cos, sin = position_embeddings
            if self.use_rope and self.head_dim == 64 and rope_supported(qkv.view(*hidden_shape).transpose(1, 2), cos):
                # split + rotary embedding in one autograd step: the backward writes dq, dk and
                # dv into one gradient of qkv instead of concatenating them
                q, k, v = qkv_rope(qkv, cos, sin, nq, nk)
            else:
                q, k, v = (t.view(hidden_shape).transpose(1, 2) for t in qkv.split((nq, nk, nk), dim=-1))
                if self.use_rope:
                    q, k = apply_rotary_pos_emb(q, k, cos, sin)
        else:
            q = self.q_proj(hidden_states).view(hidden_shape).transpose(1, 2)
            k = self.k_proj(hidden_states).view(hidden_shape).transpose(1, 2)
            v = self.v_proj(hidden_states).view(hidden_shape).transpose(1, 2)
            cos, sin = position_embeddings
            if self.use_rope:
                q, k = apply_rotary_pos_emb(q, k, cos, sin)
        past = 0 if past_key_value is None else past_key_value.get_seq_length(self.layer_idx)
        if past == 0:
            # training / prefill: the fused HIP op (P never materialised, causal mask implicit)
            out, v_prime = lucid_attention(q, k, v, scaling=self.scaling, eps=self.config.rms_norm_eps,
                                           return_vprime=True)
            if past_key_value is not None:
                past_key_value.update(k, v_prime.to(k.dtype), self.layer_idx)
        else:
            out = self._decode(q, k, v, past_key_value)
        attn_output = out.reshape(*input_shape, -1).contiguous()
        return self.o_proj(attn_output), None

    def get_new_v_prime(self, key: torch.Tensor, value: torch.Tensor, past_key: torch.Tensor,
                        past_v_prime: torch.Tensor) -> torch.Tensor:
        """V' rows of new tokens given the cached keys and V' (modeling_lucid.py:576-598),
        with the exact non-unit diagonal; several new tokens are solved in order."""
        eps = self.config.rms_norm_eps
        s = self.scaling
        dt = torch.promote_types(key.dtype, torch.float32)
        key, past_key = key.to(dt), past_key.to(dt)
        kh = key * torch.rsqrt(key.pow(2).mean(-1, keepdim=True) + eps)
        pk = past_key * torch.rsqrt(past_key.pow(2).mean(-1, keepdim=True) + eps)
        pv = past_v_prime.to(dt)
        outs = []
        for t in range(key.shape[-2]):
            kt = kh[..., t:t + 1, :]
            keys = torch.cat([pk] + [kh[..., :t, :]], dim=-2)
            vps = torch.cat([pv] + outs, dim=-2) if outs else pv
            p = torch.exp(s * (kt @ keys.transpose(-1, -2)) - 1.0 / s)
            p_tt = torch.exp(s * (kt * kt).sum(-1, keepdim=True) - 1.0 / s)
            outs.append((value[..., t:t + 1, :].to(dt) - p @ vps) / p_tt)
        return torch.cat(outs, dim=-2)

    def _decode(self, q, k, v, cache: LucidCache) -> torch.Tensor:
        """The new tokens through one HIP decoding call (``lucid_decode``), which computes
        their V' rows exactly as ``get_new_v_prime`` (coupled to the cache and to each
        other) and appends (k_t, v'_t) to the cache in place; returns [B, Tn, Hq, d]."""
        n_new = q.shape[2]
        cache.reserve(self.layer_idx, k, n_new)
        kb, vb, n = cache.buffers(self.layer_idx)
        o, _ = lucid_decode(q, k, v, kb, vb, n, scaling=self.scaling, eps=self.config.rms_norm_eps)
        cache.advance(self.layer_idx, n_new)
        return o


class LlamaDecoderLayer(nn.Module):
    """modeling_lucid.py:621-684 (pre-norm residual blocks)."""

    def __init__(self, config: LucidConfig, layer_idx: int):
        super().__init__()
        self.self_attn = LucidAttention(config, layer_idx)
        self.mlp = LlamaMLP(config)
        self.input_layernorm = LlamaRMSNorm(config.hidden_size, eps=config.rms_norm_eps)
        self.post_attention_layernorm = LlamaRMSNorm(config.hidden_size, eps=config.rms_norm_eps)

    def forward(self, hidden_states, position_embeddings, past_key_value=None, **kwargs):
        residual = hidden_states
        h, _ = self.self_attn(self.input_layernorm(hidden_states), position_embeddings,
                              past_key_value=past_key_value)
        hidden_states = residual + h
        return hidden_states + self.mlp(self.post_attention_layernorm(hidden_states))


class LlamaModel(nn.Module):
    def __init__(self, config: LucidConfig):
        super().__init__()
        self.config = config
        self.embed_tokens = nn.Embedding(config.vocab_size, config.hidden_size)
        self.layers = nn.ModuleList([LlamaDecoderLayer(config, i) for i in range(config.num_hidden_layers)])
        self.norm = LlamaRMSNorm(config.hidden_size, eps=config.rms_norm_eps)
        self.rotary_emb = LlamaRotaryEmbedding(config)

    def forward(self, input_ids: torch.Tensor, past_key_values: Optional[LucidCache] = None) -> torch.Tensor:
        h = self.embed_tokens(input_ids)
        past = past_key_values.get_seq_length() if past_key_values is not None else 0
        pos = torch.arange(past, past + input_ids.shape[1], device=input_ids.device)[None].expand(input_ids.shape[0], -1)
        pe = self.rotary_emb(h, pos)
        for layer in self.layers:
            h = layer(h, pe, past_key_value=past_key_values)
        return self.norm(h)


class LlamaForCausalLM(nn.Module):
    """Causal LM head and shifted cross-entropy loss (modeling_lucid.py:847-967)."""

    def __init__(self, config: LucidConfig):
        super().__init__()
        self.config = config
        self.model = LlamaModel(config)
        self.lm_head = nn.Linear(config.hidden_size, config.vocab_size, bias=False)
        if config.tie_word_embeddings:
            self.lm_head.weight = self.model.embed_tokens.weight
        self.apply(self._init_weights)

    def _init_weights(self, module):
        """modeling_lucid.py:701-712: normal(0, initializer_range) weights, zero biases."""
        std = self.config.initializer_range
        if isinstance(module, nn.Linear):
            module.weight.data.normal_(mean=0.0, std=std)
            if module.bias is not None:
                module.bias.data.zero_()
        elif isinstance(module, nn.Embedding):
            module.weight.data.normal_(mean=0.0, std=std)
        elif isinstance(module, LlamaRMSNorm):
            module.weight.data.fill_(1.0)

    def forward(self, input_ids: torch.Tensor, labels: Optional[torch.Tensor] = None,
                past_key_values: Optional[LucidCache] = None):
        hidden = self.model(input_ids, past_key_values=past_key_values)
        logits = self.lm_head(hidden)
        loss = None
        if labels is not None and causal_lm_loss_supported(logits, labels):
            loss = causal_lm_loss(logits, labels)  # fused on the HIP kernels (no fp32 copy of the logits)
        elif labels is not None:
            loss = F.cross_entropy(logits[:, :-1].float().reshape(-1, logits.shape[-1]), labels[:, 1:].reshape(-1))
        return loss, logits


def count_parameters(model: nn.Module) -> int:
    return sum(p.numel() for p in model.parameters())


def c3_config() -> LucidConfig:
    """16 layers, hidden 2048, 32 heads x 64, SwiGLU 5632, vocab 32000."""
    return LucidConfig(vocab_size=32000, hidden_size=2048, intermediate_size=5632, num_hidden_layers=16,
                       num_attention_heads=32, head_dim=64, rope_theta=10000.0)


__all__ = ["LucidConfig", "LucidCache", "LucidAttention", "LlamaDecoderLayer", "LlamaModel", "LlamaForCausalLM",
           "LlamaRMSNorm", "LlamaMLP", "LlamaRotaryEmbedding", "apply_rotary_pos_emb", "c3_config",
           "count_parameters"]
