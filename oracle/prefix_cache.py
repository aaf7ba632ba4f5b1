"""Prefix caching, restating ne/engine/memory/prefix_cache.py:21-158.

Test infrastructure only: the tests compare the product allocator
(nanoengine_amd.memory) against this restatement on the same operation
sequences.  Sequences are any object with ``request_id``, ``token_ids`` and
``num_cached_tokens`` (oracle.verify.Sequence qualifies).

Pinned by tests/test_prefix_cache.py against the reference's own known-answer
cases (nt/engine/test_prefix_and_chunked_prefill.py:47-138): key chaining,
empty-first-then-LRU eviction, sharing of a cached prefix, recomputation of an
exact repeat's last token, revival of freed cached blocks, and the refcount
conservation property.
"""

from __future__ import annotations

import math
from collections import OrderedDict, deque

from oracle.paging import OutOfKVMemoryError

ROOT_PARENT_HASH = 0  # prefix_cache.py:22


def build_block_keys(token_ids, block_size, num_blocks):
    """prefix_cache.py:25-34: key i = (hash of key i-1, tokens of block i)."""
    keys = []
    parent = ROOT_PARENT_HASH
    for i in range(num_blocks):
        key = (parent, tuple(token_ids[i * block_size:(i + 1) * block_size]))
        keys.append(key)
        parent = hash(key)
    return keys


class CachingBlockPool:
    """prefix_cache.py:37-97: refcounts, an empty FIFO and an LRU of cached free blocks."""

    def __init__(self, num_blocks):
        self.num_blocks = num_blocks
        self.refs = [0] * num_blocks
        self.empty = deque(range(num_blocks))
        self.lru = OrderedDict()
        self.by_key = {}
        self.key_of = {}

    @property
    def num_free_blocks(self):
        return len(self.empty) + len(self.lru)

    @property
    def num_used_blocks(self):
        return self.num_blocks - self.num_free_blocks

    def is_free(self, block):
        return self.refs[block] == 0

    def allocate(self):
        """:60-70."""
        if self.empty:
            block = self.empty.popleft()
        elif self.lru:
            block, _ = self.lru.popitem(last=False)
            del self.by_key[self.key_of.pop(block)]
        else:
            raise OutOfKVMemoryError("no free KV blocks")
        self.refs[block] = 1
        return block

    def free(self, block):
        """:72-81."""
        if self.refs[block] <= 0:
            raise ValueError(f"block {block} is not allocated")
        self.refs[block] -= 1
        if self.refs[block]:
            return
        if block in self.key_of:
            self.lru[block] = None
        else:
            self.empty.append(block)

    def find(self, key):
        return self.by_key.get(key)

    def share(self, block):
        """:86-90."""
        if self.refs[block] == 0:
            del self.lru[block]
        self.refs[block] += 1

    def register(self, block, key):
        """:92-97: the first block registered under a key keeps it."""
        if key in self.by_key or block in self.key_of:
            return
        self.by_key[key] = block
        self.key_of[block] = key


class PrefixCachingSlotAllocator:
    """prefix_cache.py:100-158 over paged_allocator.py:21-67 (tables grow by whole blocks)."""

    def __init__(self, num_blocks, block_size):
        self.block_size = block_size
        self.blocks = CachingBlockPool(num_blocks)
        self.tables = {}
        self.registered = {}
        self.num_prefix_hit_tokens = 0

    @property
    def num_free_blocks(self):
        return self.blocks.num_free_blocks

    def block_table(self, sequence):
        return list(self.tables.get(sequence.request_id, []))

    def _missing(self, sequence, num_tokens):
        owned = len(self.tables.get(sequence.request_id, []))
        return max(0, math.ceil(num_tokens / self.block_size) - owned)

    def find_cached_blocks(self, sequence):
        """:111-120: cached full blocks from the start, always leaving one token to compute."""
        full = (len(sequence.token_ids) - 1) // self.block_size
        found = []
        for key in build_block_keys(sequence.token_ids, self.block_size, full):
            block = self.blocks.find(key)
            if block is None:
                break
            found.append(block)
        return found

    def can_reserve(self, sequence, num_tokens):
        """:122-128: revived cached blocks leave the free count when they are taken."""
        if sequence.request_id in self.tables:
            return self._missing(sequence, num_tokens) <= self.blocks.num_free_blocks
        cached = self.find_cached_blocks(sequence)
        revived = sum(1 for b in cached if self.blocks.is_free(b))
        missing = math.ceil(num_tokens / self.block_size) - len(cached)
        return missing <= self.blocks.num_free_blocks - revived

    def reserve(self, sequence, num_tokens):
        """:130-142."""
        rid = sequence.request_id
        if rid not in self.tables:
            if not self.can_reserve(sequence, num_tokens):
                raise OutOfKVMemoryError(f"no blocks for {rid}")
            cached = self.find_cached_blocks(sequence)
            for block in cached:
                self.blocks.share(block)
            self.tables[rid] = cached
            self.registered[rid] = len(cached)
            sequence.num_cached_tokens = len(cached) * self.block_size
            self.num_prefix_hit_tokens += sequence.num_cached_tokens
        if self._missing(sequence, num_tokens) > self.blocks.num_free_blocks:
            raise OutOfKVMemoryError(f"no blocks for {num_tokens} tokens of {rid}")
        table = self.tables[rid]
        for _ in range(self._missing(sequence, num_tokens)):
            table.append(self.blocks.allocate())

    def on_tokens_cached(self, sequence):
        """:144-154: register the blocks that became full since the last call."""
        table = self.tables.get(sequence.request_id, [])
        done = self.registered.get(sequence.request_id, 0)
        full = min(sequence.num_cached_tokens // self.block_size, len(table))
        if full <= done:
            return
        keys = build_block_keys(sequence.token_ids, self.block_size, full)
        for i in range(done, full):
            self.blocks.register(table[i], keys[i])
        self.registered[sequence.request_id] = full

    def free(self, sequence):
        """:156-158 (+ paged_allocator.py:57-60)."""
        for block in self.tables.pop(sequence.request_id, []):
            self.blocks.free(block)
        self.registered.pop(sequence.request_id, None)
