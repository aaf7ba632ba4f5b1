"""Qwen3 decoder restated in plain PyTorch (CPU), following ne/models/qwen3.py:13-203.

The module tree, parameter names and registration order match the reference
(qwen3.py:82-87, 123-125, 135-138, 157-162), so seeding torch and then drawing
every parameter from N(0, std^2) in ``parameters()`` order reproduces the
reference's random initialisation (nt/conftest.py:38-43 pattern) including the
RNG draws made by nn.Linear / nn.Embedding construction.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
from torch import nn
from torch.nn import functional

from oracle import attention as attn
from oracle.quant import QUANTIZED_PROJECTIONS, quantize_linear, int8_linear


@dataclass(frozen=True)
class Qwen3Config:
    vocab_size: int
    hidden_size: int
    intermediate_size: int
    num_hidden_layers: int
    num_attention_heads: int
    num_key_value_heads: int
    head_dim: int
    rms_norm_eps: float
    rope_theta: float
    tie_word_embeddings: bool


QWEN3_0_6B = Qwen3Config(151936, 1024, 3072, 28, 16, 8, 128, 1e-6, 1e6, True)


class RMSNorm(nn.Module):
    """qwen3.py:31-44."""

    def __init__(self, size: int, eps: float) -> None:
        super().__init__()
        self.weight = nn.Parameter(torch.ones(size))
        self.eps = eps

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        dtype = x.dtype
        x = x.float()
        variance = x.pow(2).mean(dim=-1, keepdim=True)
        x = x * torch.rsqrt(variance + self.eps)
        return self.weight * x.to(dtype)


def build_rotary_tables(positions, head_dim, rope_theta, dtype):
    """qwen3.py:47-57."""
    exps = torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim
    inv_freq = 1.0 / (rope_theta**exps)
    angles = positions.float()[..., None] * inv_freq
    angles = torch.cat((angles, angles), dim=-1).unsqueeze(1)
    return angles.cos().to(dtype), angles.sin().to(dtype)


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    """qwen3.py:60-62."""
    first, second = x.chunk(2, dim=-1)
    return torch.cat((-second, first), dim=-1)


def apply_rotary_embedding(x, cos, sin):
    """qwen3.py:65-68."""
    return x * cos + rotate_half(x) * sin


class Int8Linear(nn.Module):
    """int8_quantization.py:37-57."""

    def __init__(self, weight_int8: torch.Tensor, weight_scale: torch.Tensor) -> None:
        super().__init__()
        self.register_buffer("weight_int8", weight_int8)
        self.register_buffer("weight_scale", weight_scale)

    @classmethod
    def from_linear(cls, linear: nn.Linear) -> "Int8Linear":
        return cls(*quantize_linear(linear.weight))

    def forward(self, x):
        return int8_linear(x, self.weight_int8, self.weight_scale)


@dataclass
class CacheContext:
    """AttentionContext (attention_context.py:16-29) plus the pool it points at."""

    positions: torch.Tensor
    slot_mapping: torch.Tensor
    context_slots: torch.Tensor
    attention_mask: torch.Tensor
    key_caches: list
    value_caches: list
    key_scales: list | None = None
    value_scales: list | None = None


class Qwen3Attention(nn.Module):
    """qwen3.py:71-115."""

    def __init__(self, config: Qwen3Config, layer_index: int) -> None:
        super().__init__()
        self.layer_index = layer_index
        self.num_heads = config.num_attention_heads
        self.num_kv_heads = config.num_key_value_heads
        self.head_dim = config.head_dim
        q_size = self.num_heads * self.head_dim
        kv_size = self.num_kv_heads * self.head_dim
        self.q_proj = nn.Linear(config.hidden_size, q_size, bias=False)
        self.k_proj = nn.Linear(config.hidden_size, kv_size, bias=False)
        self.v_proj = nn.Linear(config.hidden_size, kv_size, bias=False)
        self.o_proj = nn.Linear(q_size, config.hidden_size, bias=False)
        self.q_norm = RMSNorm(self.head_dim, config.rms_norm_eps)
        self.k_norm = RMSNorm(self.head_dim, config.rms_norm_eps)

    def forward(self, x, cos, sin, context: CacheContext | None):
        b, s, _ = x.shape
        qs = (b, s, self.num_heads, self.head_dim)
        ks = (b, s, self.num_kv_heads, self.head_dim)
        q = self.q_norm(self.q_proj(x).view(qs)).transpose(1, 2)
        k = self.k_norm(self.k_proj(x).view(ks)).transpose(1, 2)
        v = self.v_proj(x).view(ks).transpose(1, 2)
        q = apply_rotary_embedding(q, cos, sin)
        k = apply_rotary_embedding(k, cos, sin)
        if context is None:
            rep = self.num_heads // self.num_kv_heads
            k = k.repeat_interleave(rep, dim=1)
            v = v.repeat_interleave(rep, dim=1)
            out = functional.scaled_dot_product_attention(q, k, v, is_causal=True)
        else:
            li = self.layer_index
            out = attn.run_cached_attention(
                q, k, v, context.positions, context.slot_mapping, context.context_slots,
                context.attention_mask, context.key_caches[li], context.value_caches[li],
                context.key_scales[li] if context.key_scales else None,
                context.value_scales[li] if context.value_scales else None,
            )
        return self.o_proj(out.transpose(1, 2).reshape(b, s, -1))


class Qwen3MLP(nn.Module):
    """qwen3.py:118-129."""

    def __init__(self, config: Qwen3Config) -> None:
        super().__init__()
        self.gate_proj = nn.Linear(config.hidden_size, config.intermediate_size, bias=False)
        self.up_proj = nn.Linear(config.hidden_size, config.intermediate_size, bias=False)
        self.down_proj = nn.Linear(config.intermediate_size, config.hidden_size, bias=False)

    def forward(self, x):
        return self.down_proj(functional.silu(self.gate_proj(x)) * self.up_proj(x))


class Qwen3DecoderLayer(nn.Module):
    """qwen3.py:132-150."""

    def __init__(self, config: Qwen3Config, layer_index: int) -> None:
        super().__init__()
        self.self_attn = Qwen3Attention(config, layer_index)
        self.mlp = Qwen3MLP(config)
        self.input_layernorm = RMSNorm(config.hidden_size, config.rms_norm_eps)
        self.post_attention_layernorm = RMSNorm(config.hidden_size, config.rms_norm_eps)

    def forward(self, x, cos, sin, context):
        x = x + self.self_attn(self.input_layernorm(x), cos, sin, context)
        return x + self.mlp(self.post_attention_layernorm(x))


class Qwen3Model(nn.Module):
    """qwen3.py:153-178."""

    def __init__(self, config: Qwen3Config) -> None:
        super().__init__()
        self.config = config
        self.embed_tokens = nn.Embedding(config.vocab_size, config.hidden_size)
        self.layers = nn.ModuleList(Qwen3DecoderLayer(config, i) for i in range(config.num_hidden_layers))
        self.norm = RMSNorm(config.hidden_size, config.rms_norm_eps)

    def forward(self, token_ids, context: CacheContext | None = None):
        x = self.embed_tokens(token_ids)
        if context is None:
            positions = torch.arange(token_ids.shape[1]).expand(token_ids.shape)
        else:
            positions = context.positions
        cos, sin = build_rotary_tables(positions, self.config.head_dim, self.config.rope_theta, x.dtype)
        for layer in self.layers:
            x = layer(x, cos, sin, context)
        return self.norm(x)


class Qwen3ForCausalLM(nn.Module):
    """qwen3.py:181-203."""

    def __init__(self, config: Qwen3Config) -> None:
        super().__init__()
        self.config = config
        self.model = Qwen3Model(config)
        if not config.tie_word_embeddings:
            self.lm_head = nn.Linear(config.hidden_size, config.vocab_size, bias=False)

    def forward(self, token_ids, context: CacheContext | None = None):
        return self.model(token_ids, context)

    def compute_logits(self, hidden):
        weight = self.model.embed_tokens.weight if self.config.tie_word_embeddings else self.lm_head.weight
        return functional.linear(hidden, weight)


def build_random_model(config: Qwen3Config, seed: int, std: float,
                       dtype: torch.dtype = torch.float32) -> Qwen3ForCausalLM:
    """nt/conftest.py:38-43 pattern: seed, build, draw every parameter N(0, std^2) in order."""
    torch.manual_seed(seed)
    model = Qwen3ForCausalLM(config)
    with torch.no_grad():
        for parameter in model.parameters():
            torch.nn.init.normal_(parameter, std=std)
    return model.to(dtype).eval()


def quantize_linear_layers(model: Qwen3ForCausalLM) -> int:
    """int8_quantization.py:60-73: the 7 projections per layer become Int8Linear."""
    replaced = 0
    for layer in model.model.layers:
        for parent in (layer.self_attn, layer.mlp):
            for name in QUANTIZED_PROJECTIONS:
                projection = getattr(parent, name, None)
                if isinstance(projection, nn.Linear):
                    setattr(parent, name, Int8Linear.from_linear(projection))
                    replaced += 1
    return replaced


class KVCachePool:
    """kv_cache_pool.py:34-69: per-layer ``[num_slots + 1, kv_heads, d]`` plus a scratch slot."""

    def __init__(self, config: Qwen3Config, num_slots: int, dtype: torch.dtype, is_int8: bool = False):
        shape = (num_slots + 1, config.num_key_value_heads, config.head_dim)
        scale_shape = (num_slots + 1, config.num_key_value_heads, 1)
        cache_dtype = torch.int8 if is_int8 else dtype
        n = config.num_hidden_layers
        self.num_slots = num_slots
        self.scratch_slot = num_slots
        self.key_caches = [torch.zeros(shape, dtype=cache_dtype) for _ in range(n)]
        self.value_caches = [torch.zeros(shape, dtype=cache_dtype) for _ in range(n)]
        self.key_scales = [torch.zeros(scale_shape, dtype=dtype) for _ in range(n)] if is_int8 else None
        self.value_scales = [torch.zeros(scale_shape, dtype=dtype) for _ in range(n)] if is_int8 else None
