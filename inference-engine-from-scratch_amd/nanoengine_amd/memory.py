"""KV memory: the slot pool and the paged allocator.

Host-side counterparts of ne/engine/memory/kv_cache_pool.py:11-69,
block_allocator.py:8-33, paged_allocator.py:16-79 and slot_allocator.py:10-38.
The pool keeps the reference layout so the kernels read it in place: per layer
``[num_slots + 1, kv_heads, head_dim]`` (int8 or model dtype) plus, for an int8
cache, scales ``[num_slots + 1, kv_heads, 1]`` in the model dtype; the last slot
is the scratch slot that padded rows write to.
"""

from __future__ import annotations

import math
from collections import deque

import numpy as np
import torch

BYTES_PER_MEGABYTE = 1024 * 1024


class OutOfKVMemoryError(Exception):
    """No free block is left in the KV cache pool (slot_allocator.py:10-11)."""


def count_kv_bytes_per_token(num_layers: int, num_kv_heads: int, head_dim: int, dtype: torch.dtype,
                             is_int8_cache: bool = False) -> int:
    """kv_cache_pool.py:11-24: 2 (K, V) x layers x KV heads x bytes per head vector."""
    element_size = torch.empty((), dtype=dtype).element_size()
    per_head = head_dim + element_size if is_int8_cache else head_dim * element_size
    return 2 * num_layers * num_kv_heads * per_head


class KVCachePool:
    """Per-layer key/value caches with the reference's shapes (kv_cache_pool.py:34-69)."""

    def __init__(self, num_layers: int, num_kv_heads: int, head_dim: int, num_slots: int,
                 device: torch.device, dtype: torch.dtype, is_int8_cache: bool = False,
                 block_size: int = 16) -> None:
        shape = (num_slots + 1, num_kv_heads, head_dim)
        scale_shape = (num_slots + 1, num_kv_heads, 1)
        cache_dtype = torch.int8 if is_int8_cache else dtype
        self.num_slots = num_slots
        self.scratch_slot = num_slots
        self.block_size = block_size
        self.is_int8_cache = is_int8_cache
        self.key_caches = [torch.zeros(shape, device=device, dtype=cache_dtype) for _ in range(num_layers)]
        self.value_caches = [torch.zeros(shape, device=device, dtype=cache_dtype) for _ in range(num_layers)]
        self.key_scales: list[torch.Tensor] | None = None
        self.value_scales: list[torch.Tensor] | None = None
        if is_int8_cache:
            self.key_scales = [torch.zeros(scale_shape, device=device, dtype=dtype) for _ in range(num_layers)]
            self.value_scales = [torch.zeros(scale_shape, device=device, dtype=dtype) for _ in range(num_layers)]

    def key_scale_2d(self, layer: int) -> torch.Tensor | None:
        return None if self.key_scales is None else self.key_scales[layer].view(self.num_slots + 1, -1)

    def value_scale_2d(self, layer: int) -> torch.Tensor | None:
        return None if self.value_scales is None else self.value_scales[layer].view(self.num_slots + 1, -1)


class BlockAllocator:
    """FIFO free list (block_allocator.py:8-33): allocate from the head, free to the tail."""

    def __init__(self, num_blocks: int) -> None:
        self.num_blocks = num_blocks
        self._free: deque[int] = deque(range(num_blocks))
        self._used: set[int] = set()

    @property
    def num_free_blocks(self) -> int:
        return len(self._free)

    @property
    def num_used_blocks(self) -> int:
        return len(self._used)

    def allocate(self) -> int:
        if not self._free:
            raise OutOfKVMemoryError("no free KV blocks")
        block = self._free.popleft()
        self._used.add(block)
        return block

    def free(self, block: int) -> None:
        if block not in self._used:
            raise ValueError(f"block {block} is not allocated")
        self._used.remove(block)
        self._free.append(block)


class PagedSlotAllocator:
    """Block tables per request (paged_allocator.py:21-79).

    Rollback of rejected guesses frees nothing: blocks reserved for them stay in
    the table and are overwritten later, as in the reference.
    """

    def __init__(self, num_blocks: int, block_size: int, device: torch.device) -> None:
        self.block_size = block_size
        self._blocks = BlockAllocator(num_blocks)
        self._tables: dict[str, list[int]] = {}
        self._device = device

    @property
    def num_total_slots(self) -> int:
        return self._blocks.num_blocks * self.block_size

    @property
    def num_reserved_slots(self) -> int:
        return self._blocks.num_used_blocks * self.block_size

    @property
    def num_free_blocks(self) -> int:
        return self._blocks.num_free_blocks

    @property
    def num_prefix_hit_tokens(self) -> int:
        return 0

    def block_table(self, request_id: str) -> list[int]:
        return list(self._tables.get(request_id, []))

    def count_missing_blocks(self, request_id: str, num_tokens: int) -> int:
        owned = len(self._tables.get(request_id, []))
        return max(0, math.ceil(num_tokens / self.block_size) - owned)

    def can_reserve(self, request_id: str, num_tokens: int) -> bool:
        return self.count_missing_blocks(request_id, num_tokens) <= self._blocks.num_free_blocks

    def reserve(self, request_id: str, num_tokens: int) -> list[int]:
        """Grow the table to hold ``num_tokens``; returns the newly added blocks."""
        if not self.can_reserve(request_id, num_tokens):
            raise OutOfKVMemoryError(f"no blocks for {num_tokens} tokens of {request_id}")
        table = self._tables.setdefault(request_id, [])
        added = [self._blocks.allocate() for _ in range(self.count_missing_blocks(request_id, num_tokens))]
        table.extend(added)
        return added

    def free(self, request_id: str) -> None:
        for block in self._tables.pop(request_id, []):
            self._blocks.free(block)

    def on_tokens_cached(self, request_id: str) -> None:
        """Called after a step wrote more of a sequence into the cache (no-op without a prefix cache)."""

    def slots_for(self, request_id: str, positions: np.ndarray) -> np.ndarray:
        table = np.asarray(self._tables[request_id], dtype=np.int64)
        return table[positions // self.block_size] * self.block_size + positions % self.block_size

    def build_context_slots(self, request_ids: list[str], context_length: int) -> torch.Tensor:
        """paged_allocator.py:69-79 (kept for API parity; the kernels read block tables)."""
        per_row = math.ceil(context_length / self.block_size)
        rows = [(self._tables[r][:per_row] + [0] * per_row)[:per_row] for r in request_ids]
        tables = torch.tensor(rows, dtype=torch.int64)
        positions = torch.arange(context_length)
        slots = tables[:, positions // self.block_size] * self.block_size + positions % self.block_size
        return slots.to(self._device)


def slots_for_budget(num_layers: int, num_kv_heads: int, head_dim: int, dtype: torch.dtype,
                     memory_megabytes: int, is_int8_cache: bool = False) -> int:
    """kv_cache_pool.py:27-31."""
    per_token = count_kv_bytes_per_token(num_layers, num_kv_heads, head_dim, dtype, is_int8_cache)
    return memory_megabytes * BYTES_PER_MEGABYTE // per_token
