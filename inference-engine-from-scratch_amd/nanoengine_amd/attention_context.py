"""Cached attention for one step in the reference's padded-batch form, on the HIP kernels.

Counterpart of ne/models/attention_context.py:16-109.  ``AttentionContext`` keeps the
reference's fields (``[b, q]`` positions and slot mapping, ``[b, c]`` context slots, the
``[b, 1, q, c]`` mask, the per-layer caches and scales) and adds what the paged kernel
reads instead of gathered slots and a dense mask: each sequence's block table, its
number of real query rows and its context length.  ``build_step_inputs``
(``nanoengine_amd.model_runner``) fills both.

``run_cached_attention`` writes the step's keys and values with ``ne_kv_write``
(quantising for an int8 pool, as ``write_to_cache`` does) and attends with
``ne_paged_verify_attention`` over the pool in place.  The real rows of a sequence are
its last ``query_lengths[i]`` positions, as ``build_step_inputs`` lays them out; padding
rows (slot mapping = the scratch slot) come back as zeros, where the reference returns
attention over the first key for them, a value no caller reads.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from nanoengine_amd import kernels


@dataclass(frozen=True)
class AttentionContext:
    """A padded batch of ``b`` sequences, ``q`` new tokens each, at most ``c`` context tokens."""

    positions: torch.Tensor  # [b, q] position of each new token, 0 for padding
    slot_mapping: torch.Tensor  # [b, q] slot of each new token's key / value; padding: scratch slot
    context_slots: torch.Tensor  # [b, c] slots of every token a query may attend to
    attention_mask: torch.Tensor  # [b, 1, q, c] True where a query may attend to a key
    key_caches: list[torch.Tensor]  # per layer [num_slots + 1, kv_heads, head_dim]
    value_caches: list[torch.Tensor]
    key_scales: list[torch.Tensor] | None = None  # int8 pool only: per layer [num_slots + 1, kv_heads, 1]
    value_scales: list[torch.Tensor] | None = None
    # read by the HIP kernels instead of context_slots / attention_mask
    block_tables: torch.Tensor | None = None  # [b, max_blocks] int32
    block_size: int = 16
    query_lengths: torch.Tensor | None = None  # [b] int32: real rows of each sequence (the first ones)
    context_lengths: torch.Tensor | None = None  # [b] int32: keys each sequence attends over
    max_context_length: int = 0


def build_attention_mask(positions: torch.Tensor, context_lengths: torch.Tensor,
                         context_length: int) -> torch.Tensor:
    """Causal and length mask: a query at position p sees keys 0..p of its own sequence
    (attention_context.py:32-39)."""
    key_positions = torch.arange(context_length, device=positions.device)
    is_causal = key_positions[None, None, :] <= positions[:, :, None]
    is_inside = key_positions[None, None, :] < context_lengths[:, None, None]
    return (is_causal & is_inside).unsqueeze(1)


def _scales_2d(scales: list[torch.Tensor] | None, layer_index: int) -> torch.Tensor | None:
    if not scales:
        return None
    s = scales[layer_index]
    return s.view(s.shape[0], -1)


def write_to_cache(cache: torch.Tensor, scales: torch.Tensor | None, target_slots: torch.Tensor,
                   vectors: torch.Tensor) -> None:
    """``vectors [n, kv_heads, d]`` into ``cache`` at ``target_slots``; an int8 cache also
    stores one scale per vector (attention_context.py:42-54), here ``[slots, kv_heads]``."""
    kernels.kv_write(vectors.contiguous(), target_slots.to(torch.int32).contiguous(), cache, scales)


def run_cached_attention(
    queries: torch.Tensor,
    keys: torch.Tensor,
    values: torch.Tensor,
    context: AttentionContext,
    layer_index: int,
) -> torch.Tensor:
    """Write this step's keys / values into the pool, then attend over each sequence's
    context (attention_context.py:66-109).  ``queries`` is ``[b, heads, q, d]`` bf16;
    ``keys`` and ``values`` are ``[b, kv_heads, q, d]``; returns ``[b, heads, q, d]``."""
    if context.block_tables is None or context.query_lengths is None or context.context_lengths is None:
        raise ValueError("the HIP attention reads block tables, query lengths and context lengths: "
                         "build the context with model_runner.build_step_inputs")
    b, heads, q, d = queries.shape
    kv_heads = keys.shape[1]
    key_scale = _scales_2d(context.key_scales, layer_index)
    value_scale = _scales_2d(context.value_scales, layer_index)
    key_cache = context.key_caches[layer_index]
    value_cache = context.value_caches[layer_index]
    target_slots = context.slot_mapping.reshape(-1)
    write_to_cache(key_cache, key_scale, target_slots, keys.transpose(1, 2).reshape(-1, kv_heads, d))
    write_to_cache(value_cache, value_scale, target_slots, values.transpose(1, 2).reshape(-1, kv_heads, d))

    rows = queries.transpose(1, 2).reshape(b * q, heads, d).contiguous()
    q_start = torch.arange(0, b * q, q, dtype=torch.int32, device=queries.device)
    out = torch.zeros_like(rows)
    kernels.paged_verify_attention(
        rows, key_cache, value_cache, key_scale, value_scale, context.block_tables, context.block_size,
        context.context_lengths, q_start, context.query_lengths, q,
        max(context.max_context_length, int(context.context_slots.shape[1])), out=out,
    )
    return out.view(b, q, heads, d).transpose(1, 2)
