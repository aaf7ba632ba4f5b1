"""KV memory managers and step packing, restating
ne/engine/memory/block_allocator.py:8-33, paged_allocator.py:16-79,
contiguous_allocator.py:13-62, kv_cache_pool.py:11-69 and
ne/engine/generation/batch_builder.py:22-65 (+ ne/models/attention_context.py:32-39).

Sequences are identified by a request-id string, as in the reference.
"""

from __future__ import annotations

import math
from collections import deque
from dataclasses import dataclass

import torch


class OutOfKVMemoryError(Exception):
    """slot_allocator.py:10-11."""


class BlockAllocator:
    """block_allocator.py:8-33: FIFO free list; freed blocks go to the tail."""

    def __init__(self, num_blocks: int) -> None:
        self.num_blocks = num_blocks
        self._free = deque(range(num_blocks))
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
    """paged_allocator.py:21-79."""

    def __init__(self, num_blocks: int, block_size: int) -> None:
        self.block_size = block_size
        self._blocks = BlockAllocator(num_blocks)
        self._tables: dict[str, list[int]] = {}

    @property
    def num_free_blocks(self) -> int:
        return self._blocks.num_free_blocks

    @property
    def num_reserved_slots(self) -> int:
        return self._blocks.num_used_blocks * self.block_size

    def block_table(self, request_id: str) -> list[int]:
        return list(self._tables.get(request_id, []))

    def count_missing_blocks(self, request_id: str, num_tokens: int) -> int:
        owned = len(self._tables.get(request_id, []))
        return max(0, math.ceil(num_tokens / self.block_size) - owned)

    def can_reserve(self, request_id: str, num_tokens: int) -> bool:
        return self.count_missing_blocks(request_id, num_tokens) <= self._blocks.num_free_blocks

    def reserve(self, request_id: str, num_tokens: int) -> None:
        if not self.can_reserve(request_id, num_tokens):
            raise OutOfKVMemoryError(f"no blocks for {num_tokens} tokens of {request_id}")
        table = self._tables.setdefault(request_id, [])
        for _ in range(self.count_missing_blocks(request_id, num_tokens)):
            table.append(self._blocks.allocate())

    def free(self, request_id: str) -> None:
        for block in self._tables.pop(request_id, []):
            self._blocks.free(block)

    def build_context_slots(self, request_ids: list[str], context_length: int) -> torch.Tensor:
        """paged_allocator.py:69-79: slot(p) = table[p // bs] * bs + p % bs, pad block 0."""
        per_row = math.ceil(context_length / self.block_size)
        rows = []
        for rid in request_ids:
            table = self._tables[rid][:per_row]
            rows.append(table + [0] * (per_row - len(table)))
        tables = torch.tensor(rows, dtype=torch.int64)
        positions = torch.arange(context_length)
        return tables[:, positions // self.block_size] * self.block_size + positions % self.block_size


class ContiguousSlotAllocator:
    """contiguous_allocator.py:13-62: one ``region_length`` slot range per sequence."""

    def __init__(self, num_regions: int, region_length: int) -> None:
        self.num_regions = num_regions
        self.region_length = region_length
        self._free_regions = list(range(num_regions - 1, -1, -1))
        self._region: dict[str, int] = {}

    @property
    def num_reserved_slots(self) -> int:
        """contiguous_allocator.py:25-27: a whole region per sequence holding one."""
        return len(self._region) * self.region_length

    def can_reserve(self, request_id: str, num_tokens: int) -> bool:
        if num_tokens > self.region_length:
            return False
        return request_id in self._region or bool(self._free_regions)

    def reserve(self, request_id: str, num_tokens: int) -> None:
        if not self.can_reserve(request_id, num_tokens):
            raise OutOfKVMemoryError(f"no region for {num_tokens} tokens of {request_id}")
        if request_id not in self._region:
            self._region[request_id] = self._free_regions.pop()

    def free(self, request_id: str) -> None:
        region = self._region.pop(request_id, None)
        if region is not None:
            self._free_regions.append(region)

    def build_context_slots(self, request_ids: list[str], context_length: int) -> torch.Tensor:
        starts = torch.tensor([self._region[r] * self.region_length for r in request_ids])
        return starts[:, None] + torch.arange(context_length)[None, :]


def count_kv_bytes_per_token(num_layers: int, num_kv_heads: int, head_dim: int,
                             element_size: int, is_int8: bool) -> int:
    """kv_cache_pool.py:11-24."""
    per_head = head_dim + element_size if is_int8 else head_dim * element_size
    return 2 * num_layers * num_kv_heads * per_head


@dataclass(frozen=True)
class StepInputs:
    token_ids: torch.Tensor  # [b, q]
    positions: torch.Tensor  # [b, q]
    slot_mapping: torch.Tensor  # [b, q], pads -> scratch slot
    context_slots: torch.Tensor  # [b, c]
    attention_mask: torch.Tensor  # [b, 1, q, c]
    last_token_indices: torch.Tensor  # [b]


def build_attention_mask(positions: torch.Tensor, context_lengths: torch.Tensor,
                         context_length: int) -> torch.Tensor:
    """attention_context.py:32-39."""
    key_positions = torch.arange(context_length)
    is_causal = key_positions[None, None, :] <= positions[:, :, None]
    is_inside = key_positions[None, None, :] < context_lengths[:, None, None]
    return (is_causal & is_inside).unsqueeze(1)


def build_step_inputs(
    token_ids: list[list[int]],
    num_cached: list[int],
    token_counts: list[int],
    context_slots_fn,
    scratch_slot: int,
) -> StepInputs:
    """batch_builder.py:22-65 for sequences given as token lists and cached counts.

    ``context_slots_fn(context_length) -> [b, context_length]`` supplies the
    allocator's ``build_context_slots`` for these sequences.
    """
    ends = [c + n for c, n in zip(num_cached, token_counts, strict=True)]
    q = max(token_counts)
    c = max(ends)
    token_rows, position_rows = [], []
    for toks, start, end in zip(token_ids, num_cached, ends, strict=True):
        pad = [0] * (q - (end - start))
        token_rows.append(toks[start:end] + pad)
        position_rows.append(list(range(start, end)) + pad)
    tokens = torch.tensor(token_rows, dtype=torch.int64)
    positions = torch.tensor(position_rows, dtype=torch.int64)
    counts = torch.tensor(token_counts)
    is_real = torch.arange(q)[None, :] < counts[:, None]
    context_slots = context_slots_fn(c)
    slot_mapping = context_slots.gather(1, positions).masked_fill(~is_real, scratch_slot)
    mask = build_attention_mask(positions, torch.tensor(ends), c)
    return StepInputs(tokens, positions, slot_mapping, context_slots, mask, counts - 1)
