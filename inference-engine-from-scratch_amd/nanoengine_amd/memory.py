"""KV memory: the slot pool, the paged allocator and the prefix cache.

Host-side counterparts of ne/engine/memory/kv_cache_pool.py:11-69,
block_allocator.py:8-33, paged_allocator.py:16-79, slot_allocator.py:10-38 and
prefix_cache.py:21-158.
The pool keeps the reference layout so the kernels read it in place: per layer
``[num_slots + 1, kv_heads, head_dim]`` (int8 or model dtype) plus, for an int8
cache, scales ``[num_slots + 1, kv_heads, 1]`` in the model dtype; the last slot
is the scratch slot that padded rows write to.
"""

from __future__ import annotations

import itertools
import math
from collections import OrderedDict, deque

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

    def allocate_many(self, count: int) -> list[int]:
        """``count`` blocks from the head, as ``count`` calls of ``allocate``."""
        if count > len(self._free):
            raise OutOfKVMemoryError("no free KV blocks")
        blocks = [self._free.popleft() for _ in range(count)]
        self._used.update(blocks)
        return blocks

    def free(self, block: int) -> None:
        if block not in self._used:
            raise ValueError(f"block {block} is not allocated")
        self._used.remove(block)
        self._free.append(block)


def _request_id(sequence) -> str:
    """The allocators take a ``Sequence`` (as the reference's do) or its request id."""
    return sequence if isinstance(sequence, str) else sequence.request_id


class PagedSlotAllocator:
    """Block tables per request (paged_allocator.py:21-79).

    Rollback of rejected guesses frees nothing: blocks reserved for them stay in
    the table and are overwritten later, as in the reference.  Every method takes
    a ``Sequence`` or its request id.
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

    def block_table(self, sequence) -> list[int]:
        return list(self._tables.get(_request_id(sequence), []))

    def num_blocks_of(self, sequence) -> int:
        return len(self._tables.get(_request_id(sequence), ()))

    def count_missing_blocks(self, sequence, num_tokens: int) -> int:
        owned = len(self._tables.get(_request_id(sequence), []))
        return max(0, math.ceil(num_tokens / self.block_size) - owned)

    def can_reserve(self, sequence, num_tokens: int) -> bool:
        return self.count_missing_blocks(sequence, num_tokens) <= self._blocks.num_free_blocks

    def reserve(self, sequence, num_tokens: int) -> list[int]:
        """Grow the table to hold ``num_tokens``; returns the newly allocated blocks."""
        rid = _request_id(sequence)
        table = self._tables.get(rid)
        missing = -(-num_tokens // self.block_size) - (0 if table is None else len(table))
        if missing > self._blocks.num_free_blocks:
            raise OutOfKVMemoryError(f"no blocks for {num_tokens} tokens of {rid}")
        if table is None:
            table = self._tables[rid] = []
        if missing <= 0:
            return []
        added = [self._blocks.allocate() for _ in range(missing)]
        table.extend(added)
        return added

    def peek_free(self, count: int) -> list[int] | None:
        """The next ``count`` blocks ``reserve`` would hand out (the head of the FIFO free
        list), or None when fewer are free."""
        free = self._blocks._free
        if count > len(free):
            return None
        return list(itertools.islice(free, count))

    def take_free(self, sequences: list, counts: list[int], blocks: list[int]) -> None:
        """Record what ``peek_free`` showed as reserved: sequence i grows by the next
        counts[i] blocks, in order -- the state ``reserve`` would leave for each of them
        in turn."""
        taken = self._blocks.allocate_many(len(blocks))
        if taken != blocks:
            raise RuntimeError("the free list changed between peek_free and take_free")
        at = 0
        for sequence, count in zip(sequences, counts):
            self._tables.setdefault(_request_id(sequence), []).extend(blocks[at : at + count])
            at += count

    def free(self, sequence) -> None:
        for block in self._tables.pop(_request_id(sequence), []):
            self._blocks.free(block)

    def on_tokens_cached(self, sequence) -> None:
        """Called after a step wrote more of a sequence into the cache (no-op without a prefix cache)."""

    def first_writable_position(self, sequence) -> int:
        """Positions below this one sit in blocks other requests may read (none here)."""
        return 0

    def slots_for(self, sequence, positions: np.ndarray) -> np.ndarray:
        table = np.asarray(self._tables[_request_id(sequence)], dtype=np.int64)
        return table[positions // self.block_size] * self.block_size + positions % self.block_size

    def build_context_slots(self, sequences: list, context_length: int) -> torch.Tensor:
        """paged_allocator.py:69-79 (kept for API parity; the kernels read block tables)."""
        per_row = math.ceil(context_length / self.block_size)
        request_ids = [_request_id(x) for x in sequences]
        rows = [(self._tables[r][:per_row] + [0] * per_row)[:per_row] for r in request_ids]
        tables = torch.tensor(rows, dtype=torch.int64)
        positions = torch.arange(context_length)
        slots = tables[:, positions // self.block_size] * self.block_size + positions % self.block_size
        return slots.to(self._device)


ROOT_PARENT_HASH = 0


def build_block_keys(token_ids, block_size: int, num_blocks: int, first: int = 0,
                     parent: int = ROOT_PARENT_HASH) -> list[tuple[int, tuple[int, ...]]]:
    """Keys of full blocks ``first`` .. ``num_blocks``-1 (prefix_cache.py:25-34).

    A key is (hash of the previous block's key, this block's tokens), so equal keys
    mean equal whole prefixes, not only equal 16-token windows.  ``parent`` is the
    hash of block ``first``-1's key (the root value for ``first`` 0), so a caller
    that remembers it extends a chain without rehashing the blocks before.  Python's
    hash of a tuple of ints is deterministic, so keys agree across processes and
    with the reference's."""
    keys = []
    for start in range(first * block_size, num_blocks * block_size, block_size):
        key = (parent, tuple(token_ids[start:start + block_size]))
        keys.append(key)
        parent = hash(key)
    return keys


class CachingBlockPool:
    """Reference-counted blocks whose content outlives their last owner (prefix_cache.py:37-97).

    A block with no owner is either empty (never registered) or cached (registered
    under a key, still holding that prefix's keys/values).  ``allocate`` takes an
    empty block first, then evicts the least recently freed cached block; ``share``
    takes one more reference to a cached block, reviving it if it was free."""

    def __init__(self, num_blocks: int) -> None:
        self.num_blocks = num_blocks
        self._refs = np.zeros(num_blocks, dtype=np.int64)
        self._empty: deque[int] = deque(range(num_blocks))
        self._cached_free: OrderedDict[int, None] = OrderedDict()  # least recently freed first
        self._block_of: dict = {}
        self._key_of: dict[int, tuple] = {}

    @property
    def num_free_blocks(self) -> int:
        return len(self._empty) + len(self._cached_free)

    @property
    def num_used_blocks(self) -> int:
        return self.num_blocks - self.num_free_blocks

    def reference_count(self, block: int) -> int:
        return int(self._refs[block])

    def is_free(self, block: int) -> bool:
        return self._refs[block] == 0

    def is_registered(self, block: int) -> bool:
        return block in self._key_of

    def allocate(self) -> int:
        if self._empty:
            block = self._empty.popleft()
        elif self._cached_free:
            block = next(iter(self._cached_free))
            del self._cached_free[block]
            del self._block_of[self._key_of.pop(block)]
        else:
            raise OutOfKVMemoryError("no free KV blocks")
        self._refs[block] = 1
        return block

    def free(self, block: int) -> None:
        if self._refs[block] <= 0:
            raise ValueError(f"block {block} is not allocated")
        self._refs[block] -= 1
        if self._refs[block] == 0:
            if block in self._key_of:
                self._cached_free[block] = None
            else:
                self._empty.append(block)

    def find(self, key) -> int | None:
        return self._block_of.get(key)

    def share(self, block: int) -> None:
        if self._refs[block] == 0:
            self._cached_free.pop(block)
        self._refs[block] += 1

    def register(self, block: int, key) -> None:
        """Record that ``block`` holds ``key``'s prefix; an existing key or block keeps its entry."""
        if key not in self._block_of and block not in self._key_of:
            self._block_of[key] = block
            self._key_of[block] = key


class PrefixCachingSlotAllocator(PagedSlotAllocator):
    """Paged allocator that shares full prompt blocks between requests (prefix_cache.py:100-158).

    Speculation-safe by its call sites, not by extra state: a block is registered only
    from ``on_tokens_cached(sequence)``, which keys blocks by ``sequence.token_ids`` and
    counts ``sequence.num_cached_tokens``.  The verify runner calls it after acceptance,
    when ``token_ids`` holds verified tokens only and ``num_cached_tokens`` counts the
    positions whose keys/values belong to them (the reference calls it from
    score_tokens while the guesses are still appended, model_runner.py:60-61, which
    would register blocks keyed by rejected guesses).  Registered blocks end below
    ``num_cached_tokens`` and a step only writes at ``num_cached_tokens`` and later, so
    no step - a rejected guess included - ever writes into a block another request
    can read.  ``first_writable_position`` exposes that bound for the runner to check.
    """

    def __init__(self, num_blocks: int, block_size: int, device: torch.device) -> None:
        super().__init__(num_blocks, block_size, device)
        self._blocks = CachingBlockPool(num_blocks)
        self._num_registered: dict[str, int] = {}
        # hash of the last registered block's key per request: verified tokens never
        # change, so registration extends the chain instead of rehashing a long history
        self._chain: dict[str, int] = {}
        self._hit_tokens = 0

    @property
    def num_prefix_hit_tokens(self) -> int:
        return self._hit_tokens

    @property
    def pool(self) -> CachingBlockPool:
        return self._blocks

    def find_cached_blocks(self, sequence) -> list[int]:
        """Cached blocks that match the start of ``sequence``; the last token is always
        left to compute, since its logits are needed (prefix_cache.py:111-120)."""
        return self._find_cached(sequence)[0]

    def _find_cached(self, sequence) -> tuple[list[int], int]:
        usable = (sequence.num_tokens - 1) // self.block_size
        found, parent = [], ROOT_PARENT_HASH
        for key in build_block_keys(sequence.token_ids, self.block_size, usable):
            block = self._blocks.find(key)
            if block is None:
                break
            found.append(block)
            parent = hash(key)
        return found, parent

    def can_reserve(self, sequence, num_tokens: int) -> bool:
        rid = _request_id(sequence)
        if rid in self._tables or isinstance(sequence, str):
            return super().can_reserve(rid, num_tokens)
        cached = self.find_cached_blocks(sequence)
        revived = sum(1 for b in cached if self._blocks.is_free(b))
        return math.ceil(num_tokens / self.block_size) - len(cached) <= self._blocks.num_free_blocks - revived

    def reserve(self, sequence, num_tokens: int) -> list[int]:
        """A new sequence first takes its cached prefix (setting ``num_cached_tokens``),
        then gets fresh blocks for the rest (prefix_cache.py:130-142).  Returns the
        freshly allocated blocks; shared ones are in ``block_table``."""
        rid = _request_id(sequence)
        if rid not in self._tables and not isinstance(sequence, str):
            if not self.can_reserve(sequence, num_tokens):
                raise OutOfKVMemoryError(f"no blocks for {rid}")
            cached, parent = self._find_cached(sequence)
            for block in cached:
                self._blocks.share(block)
            self._tables[rid] = list(cached)
            self._num_registered[rid] = len(cached)
            self._chain[rid] = parent
            sequence.num_cached_tokens = len(cached) * self.block_size
            self._hit_tokens += sequence.num_cached_tokens
        return super().reserve(rid, num_tokens)

    def on_tokens_cached(self, sequence) -> None:
        """Register the blocks that became full since the last call (prefix_cache.py:144-154)."""
        rid = sequence.request_id
        table = self._tables.get(rid, [])
        done = self._num_registered.get(rid, 0)
        full = min(sequence.num_cached_tokens // self.block_size, len(table), sequence.num_tokens // self.block_size)
        if full <= done:
            return
        keys = build_block_keys(sequence.token_ids, self.block_size, full, done,
                                self._chain.get(rid, ROOT_PARENT_HASH))
        for i, key in enumerate(keys, start=done):
            self._blocks.register(table[i], key)
        self._num_registered[rid] = full
        self._chain[rid] = hash(keys[-1])

    def first_writable_position(self, sequence) -> int:
        return self._num_registered.get(_request_id(sequence), 0) * self.block_size

    def free(self, sequence) -> None:
        super().free(sequence)
        self._num_registered.pop(_request_id(sequence), None)
        self._chain.pop(_request_id(sequence), None)


def slots_for_budget(num_layers: int, num_kv_heads: int, head_dim: int, dtype: torch.dtype,
                     memory_megabytes: int, is_int8_cache: bool = False) -> int:
    """kv_cache_pool.py:27-31."""
    per_token = count_kv_bytes_per_token(num_layers, num_kv_heads, head_dim, dtype, is_int8_cache)
    return memory_megabytes * BYTES_PER_MEGABYTE // per_token
