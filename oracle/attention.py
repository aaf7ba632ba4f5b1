"""Cached GQA attention over a slot pool, restating ne/models/attention_context.py:42-109.

``paged_attention_reference`` is the kernel-level reference for the HIP paged verify
attention: for every sequence it gathers the context through the block table,
dequantises int8 entries exactly as ``read_from_cache`` does (int8 -> model dtype
times the stored scale), and runs masked softmax attention in fp32.
``textbook_attention_fp64`` restates the same maths with explicit loops in fp64
for tiny inputs; it pins the former.
"""

from __future__ import annotations

import math

import numpy as np
import torch

from oracle.quant import quantize_vectors


def write_to_cache(cache: torch.Tensor, scales: torch.Tensor | None, slots: torch.Tensor,
                   vectors: torch.Tensor) -> None:
    """attention_context.py:42-54."""
    if scales is None:
        cache.index_copy_(0, slots, vectors)
        return
    quantized, vector_scales = quantize_vectors(vectors)
    cache.index_copy_(0, slots, quantized)
    scales.index_copy_(0, slots, vector_scales)


def read_from_cache(cache: torch.Tensor, scales: torch.Tensor | None, slots: torch.Tensor,
                    dtype: torch.dtype) -> torch.Tensor:
    """attention_context.py:57-63: gather ``[b, c]`` slots into ``[b, c, kv_heads, d]``."""
    if scales is None:
        return cache[slots]
    return cache[slots].to(dtype) * scales[slots]


def run_cached_attention(queries, keys, values, positions, slot_mapping, context_slots, mask,
                         key_cache, value_cache, key_scale, value_scale) -> torch.Tensor:
    """attention_context.py:66-109 for one layer: write, gather, masked SDPA with GQA."""
    target = slot_mapping.reshape(-1)
    shape = (-1, keys.shape[1], keys.shape[3])
    write_to_cache(key_cache, key_scale, target, keys.transpose(1, 2).reshape(shape))
    write_to_cache(value_cache, value_scale, target, values.transpose(1, 2).reshape(shape))
    ctx_k = read_from_cache(key_cache, key_scale, context_slots, queries.dtype)
    ctx_v = read_from_cache(value_cache, value_scale, context_slots, queries.dtype)
    return torch.nn.functional.scaled_dot_product_attention(
        queries, ctx_k.transpose(1, 2), ctx_v.transpose(1, 2), attn_mask=mask, enable_gqa=True
    )


def gather_context(k_cache, v_cache, k_scale, v_scale, table, ctx, block_size, dtype):
    """K, V ``[ctx, kv_heads, d]`` of one sequence through its block table, dequantised."""
    positions = torch.arange(ctx)
    slots = table[positions // block_size].long() * block_size + positions % block_size
    k = read_from_cache(k_cache, None if k_scale is None else k_scale.reshape(-1, k_cache.shape[1], 1),
                        slots, dtype)
    v = read_from_cache(v_cache, None if v_scale is None else v_scale.reshape(-1, v_cache.shape[1], 1),
                        slots, dtype)
    return k, v


def paged_attention_reference(q, k_cache, v_cache, k_scale, v_scale, block_tables, block_size,
                              ctx_len, q_start, q_len, softmax_scale=None, model_dtype=torch.bfloat16):
    """Rows ``q_start[b] .. +q_len[b]`` of ``q [rows, Hq, d]`` attend over sequence b's context.

    The dequantised K/V are rounded to ``model_dtype`` as the reference does, then
    the softmax and both products run in fp32.  Rows of no sequence are zero.
    """
    q = q.float().cpu()
    rows, num_q_heads, d = q.shape
    num_kv_heads = k_cache.shape[1]
    group = num_q_heads // num_kv_heads
    scale = softmax_scale if softmax_scale is not None else 1.0 / math.sqrt(d)
    out = torch.zeros(rows, num_q_heads, d)
    for b in range(ctx_len.shape[0]):
        ctx, ql, qs = int(ctx_len[b]), int(q_len[b]), int(q_start[b])
        if ql == 0:
            continue
        k, v = gather_context(k_cache.cpu(), v_cache.cpu(),
                              None if k_scale is None else k_scale.cpu(),
                              None if v_scale is None else v_scale.cpu(),
                              block_tables[b].cpu(), ctx, block_size, model_dtype)
        k = k.float().repeat_interleave(group, dim=1)  # [ctx, Hq, d]
        v = v.float().repeat_interleave(group, dim=1)
        qb = q[qs : qs + ql]  # [ql, Hq, d]
        scores = torch.einsum("qhd,chd->hqc", qb, k) * scale
        pos = ctx - ql + torch.arange(ql)
        allowed = torch.arange(ctx)[None, :] <= pos[:, None]  # [ql, ctx]
        scores = scores.masked_fill(~allowed[None], float("-inf"))
        probs = torch.softmax(scores, dim=-1)
        out[qs : qs + ql] = torch.einsum("hqc,chd->qhd", probs, v)
    return out


def textbook_attention_fp64(q, keys, values, positions_q, scale):
    """Loops in fp64: q ``[n, Hq, d]``, keys/values ``[c, Hkv, d]``, query i sees keys <= positions_q[i]."""
    q = np.asarray(q, dtype=np.float64)
    keys = np.asarray(keys, dtype=np.float64)
    values = np.asarray(values, dtype=np.float64)
    n, hq, d = q.shape
    hkv = keys.shape[1]
    out = np.zeros((n, hq, d))
    for i in range(n):
        for h in range(hq):
            kh = h // (hq // hkv)
            visible = range(int(positions_q[i]) + 1)
            s = [scale * sum(q[i, h, t] * keys[j, kh, t] for t in range(d)) for j in visible]
            m = max(s)
            w = [math.exp(x - m) for x in s]
            z = sum(w)
            for t in range(d):
                out[i, h, t] = sum(w[idx] * values[j, kh, t] for idx, j in enumerate(visible)) / z
    return out
