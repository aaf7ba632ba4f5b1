"""Shared builders for the parity tests (synthetic, seeded inputs)."""

from __future__ import annotations

import numpy as np
import torch

from oracle.quant import quantize_vectors

HEAD_DIM = 128


def rel_err(got: torch.Tensor, ref: torch.Tensor) -> float:
    got = got.float().cpu()
    ref = ref.float().cpu()
    return float((got - ref).norm() / ref.norm().clamp(min=1e-30))


def make_pool(num_blocks: int, block_size: int, kv_heads: int, kv_dtype: str, scale_dtype=torch.bfloat16,
              seed: int = 0):
    """Slot pool ``[num_blocks*block_size + 1, kv_heads, 128]`` filled with N(0,1) (quantised for int8)."""
    g = torch.Generator().manual_seed(seed)
    slots = num_blocks * block_size + 1
    k = torch.randn(slots, kv_heads, HEAD_DIM, generator=g).to(torch.bfloat16)
    v = torch.randn(slots, kv_heads, HEAD_DIM, generator=g).to(torch.bfloat16)
    if kv_dtype == "bf16":
        return k, v, None, None
    # quantise exactly as the reference's int8 KV routine does, scales in scale_dtype
    kq, ks = quantize_vectors(k.to(scale_dtype))
    vq, vs = quantize_vectors(v.to(scale_dtype))
    return kq, vq, ks.reshape(slots, kv_heads), vs.reshape(slots, kv_heads)


def make_batch(ctx_lens: list[int], q_lens: list[int], num_blocks: int, block_size: int, seed: int = 1,
               padded_q: int | None = None):
    """Block tables from a seeded permutation of the pool; packed (or padded) query rows."""
    g = torch.Generator().manual_seed(seed)
    perm = torch.randperm(num_blocks, generator=g).tolist()
    max_blocks = max((c + block_size - 1) // block_size for c in ctx_lens)
    tables = torch.zeros(len(ctx_lens), max(max_blocks, 1), dtype=torch.int32)
    cursor = 0
    for b, c in enumerate(ctx_lens):
        n = (c + block_size - 1) // block_size
        tables[b, :n] = torch.tensor(perm[cursor : cursor + n], dtype=torch.int32)
        cursor += n
    assert cursor <= num_blocks, "pool too small for these contexts"
    if padded_q is None:
        starts = np.concatenate([[0], np.cumsum(q_lens)[:-1]]).astype(np.int32)
        rows = int(sum(q_lens))
    else:
        starts = (np.arange(len(q_lens)) * padded_q).astype(np.int32)
        rows = padded_q * len(q_lens)
    return tables, torch.tensor(ctx_lens, dtype=torch.int32), torch.tensor(starts), torch.tensor(
        q_lens, dtype=torch.int32), rows


def real_rows(q_start, q_len) -> torch.Tensor:
    idx = [int(s) + i for s, n in zip(q_start.tolist(), q_len.tolist()) for i in range(n)]
    return torch.tensor(idx, dtype=torch.long)
