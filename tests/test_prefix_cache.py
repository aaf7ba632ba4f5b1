"""Prefix caching with speculation (CPU only; no kernel is launched).

* The oracle's restatement of ne/engine/memory/prefix_cache.py and the product's
  allocator both pass the reference's own known-answer cases
  (nt/engine/test_prefix_and_chunked_prefill.py:47-138, restated here with the same
  inputs and expected values) and the refcount-conservation property.
* The product allocator equals the oracle on random operation sequences: block
  tables, free counts, hit tokens and cached counts after every operation.
* Speculation safety, simulated with the runner's host protocol and random
  acceptance: every registered block's key is the key of the verified tokens, and no
  verify step ever writes a position inside a registered or shared block.  The
  reference's own protocol (registering while the guesses are appended,
  model_runner.py:60-61) is shown to break the first property on the oracle, which
  is why the product registers after acceptance.
"""

from __future__ import annotations

import random
from dataclasses import dataclass

import pytest
import torch
from hypothesis import given, settings
from hypothesis import strategies as st

from nanoengine_amd import memory as pm
from oracle import prefix_cache as op
from oracle.paging import OutOfKVMemoryError as OracleOOM

CPU = torch.device("cpu")
BLOCK = 4
SHARED = [5, 6, 7, 8, 9, 10, 11, 12]


@dataclass(eq=False)
class Seq:
    """The fields the allocators read (sequence_state.py:12-57)."""

    request_id: str
    token_ids: list
    num_cached_tokens: int = 0

    @property
    def num_tokens(self):
        return len(self.token_ids)

    @property
    def num_uncached_tokens(self):
        return len(self.token_ids) - self.num_cached_tokens


class Impl:
    """One allocator implementation behind a common constructor."""

    def __init__(self, name):
        self.name = name

    def pool(self, n):
        return op.CachingBlockPool(n) if self.name == "oracle" else pm.CachingBlockPool(n)

    def allocator(self, n, bs=BLOCK):
        if self.name == "oracle":
            return op.PrefixCachingSlotAllocator(n, bs)
        return pm.PrefixCachingSlotAllocator(n, bs, CPU)

    @property
    def oom(self):
        return OracleOOM if self.name == "oracle" else pm.OutOfKVMemoryError

    def keys(self, *a):
        return (op if self.name == "oracle" else pm).build_block_keys(*a)


IMPLS = [Impl("oracle"), Impl("product")]


def cache_everything(alloc, seq):
    """What a prefill does to the allocator (test_prefix_and_chunked_prefill.py:40-44)."""
    alloc.reserve(seq, seq.num_tokens)
    seq.num_cached_tokens = seq.num_tokens
    alloc.on_tokens_cached(seq)


# ----------------------------------------------------------- reference known answers
@pytest.mark.parametrize("impl", IMPLS, ids=lambda i: i.name)
def test_block_keys_include_the_whole_prefix(impl):
    """test_prefix_and_chunked_prefill.py:47-52."""
    first = impl.keys([1, 2, 3, 4, 9, 9, 9, 9], BLOCK, 2)
    second = impl.keys([0, 2, 3, 4, 9, 9, 9, 9], BLOCK, 2)
    assert first[1][1] == second[1][1] == (9, 9, 9, 9)
    assert first[1] != second[1]
    # closed form of the chain: the root parent is 0 and each parent is hash(previous key)
    assert first[0] == (0, (1, 2, 3, 4)) and first[1][0] == hash((0, (1, 2, 3, 4)))
    assert impl.keys([1, 2, 3], BLOCK, 0) == []


def test_extending_a_key_chain_equals_rebuilding_it():
    toks = list(range(100, 161))
    full = op.build_block_keys(toks, BLOCK, 15)
    for first in (0, 1, 7, 14, 15):
        parent = hash(full[first - 1]) if first else 0
        assert pm.build_block_keys(toks, BLOCK, 15, first, parent) == full[first:]


@pytest.mark.parametrize("impl", IMPLS, ids=lambda i: i.name)
def test_pool_reuses_empty_blocks_first_then_evicts_the_oldest_cached(impl):
    """test_prefix_and_chunked_prefill.py:55-76."""
    pool = impl.pool(2)
    old, new = pool.allocate(), pool.allocate()
    pool.register(old, (0, (1,)))
    pool.register(new, (0, (2,)))
    pool.free(old)
    pool.free(new)
    reused = pool.allocate()
    assert reused == old
    assert pool.find((0, (1,))) is None and pool.find((0, (2,))) == new
    pool.share(new)
    assert pool.num_free_blocks == 0
    with pytest.raises(impl.oom):
        pool.allocate()
    pool.free(new)
    pool.free(reused)
    with pytest.raises(ValueError, match="not allocated"):
        pool.free(reused)


@pytest.mark.parametrize("impl", IMPLS, ids=lambda i: i.name)
def test_first_registration_of_a_key_wins(impl):
    pool = impl.pool(3)
    a, b = pool.allocate(), pool.allocate()
    pool.register(a, (0, (1,)))
    pool.register(b, (0, (1,)))  # same key: a keeps it
    pool.register(a, (0, (2,)))  # a block keeps its first key
    assert pool.find((0, (1,))) == a and pool.find((0, (2,))) is None
    pool.free(b)
    assert pool.allocate() == 2  # b went back to the empty list's tail, after block 2
    assert pool.allocate() == b


@pytest.mark.parametrize("impl", IMPLS, ids=lambda i: i.name)
def test_second_request_shares_the_cached_prefix_blocks(impl):
    """test_prefix_and_chunked_prefill.py:79-92."""
    alloc = impl.allocator(8)
    first = Seq("first", [*SHARED, 1, 2])
    cache_everything(alloc, first)
    second = Seq("second", [*SHARED, 3])
    alloc.reserve(second, second.num_tokens)
    assert second.num_cached_tokens == 8
    assert alloc.block_table(second)[:2] == alloc.block_table(first)[:2]
    assert alloc.num_prefix_hit_tokens == 8
    alloc.free(first)
    alloc.free(second)
    assert alloc.num_free_blocks == 8


@pytest.mark.parametrize("impl", IMPLS, ids=lambda i: i.name)
def test_an_exact_repeat_still_recomputes_its_last_token(impl):
    """test_prefix_and_chunked_prefill.py:95-103."""
    alloc = impl.allocator(8)
    cache_everything(alloc, Seq("first", list(SHARED)))
    repeat = Seq("repeat", list(SHARED))
    alloc.reserve(repeat, repeat.num_tokens)
    assert repeat.num_cached_tokens == 4
    assert repeat.num_uncached_tokens == 4


@pytest.mark.parametrize("impl", IMPLS, ids=lambda i: i.name)
def test_freed_cached_blocks_are_revived_and_counted_as_used(impl):
    """test_prefix_and_chunked_prefill.py:106-117."""
    alloc = impl.allocator(3)
    first = Seq("first", [*SHARED, 1])
    cache_everything(alloc, first)
    alloc.free(first)
    second = Seq("second", [*SHARED, 2])
    assert alloc.can_reserve(second, second.num_tokens)
    assert not alloc.can_reserve(Seq("other", list(range(30, 43))), 13)
    alloc.reserve(second, second.num_tokens)
    assert second.num_cached_tokens == 8 and alloc.num_free_blocks == 0


@pytest.mark.parametrize("impl", IMPLS, ids=lambda i: i.name)
@settings(max_examples=50, deadline=None)
@given(st.lists(st.tuples(st.integers(0, 3), st.integers(1, 3)), max_size=30))
def test_reference_counts_never_lose_or_double_count_a_block(impl, operations):
    """test_prefix_and_chunked_prefill.py:120-138."""
    alloc = impl.allocator(12)
    live = {}
    for index, (slot, prefix_blocks) in enumerate(operations):
        if slot in live:
            alloc.free(live.pop(slot))
            continue
        seq = Seq(f"s{index}", SHARED[: prefix_blocks * 2] + [index, 1])
        if alloc.can_reserve(seq, seq.num_tokens):
            cache_everything(alloc, seq)
            live[slot] = seq
        owned = {b for s in live.values() for b in alloc.block_table(s)}
        assert len(owned) + alloc.num_free_blocks == 12
    for seq in live.values():
        alloc.free(seq)
    assert alloc.num_free_blocks == 12


# ------------------------------------------------------------- product vs oracle
def _snapshot(alloc, live):
    tables = {rid: alloc.block_table(s) for rid, s in live.items()}
    return tables, alloc.num_free_blocks, alloc.num_prefix_hit_tokens


@pytest.mark.parametrize("seed", range(8))
def test_product_allocator_equals_the_oracle_on_random_operations(seed):
    rng = random.Random(seed)
    ours, ref = pm.PrefixCachingSlotAllocator(24, BLOCK, CPU), op.PrefixCachingSlotAllocator(24, BLOCK)
    prefixes = [[rng.randrange(50) for _ in range(rng.choice([4, 8, 12]))] for _ in range(3)]
    live_o, live_r = {}, {}
    for step in range(300):
        action = rng.random()
        if action < 0.35 or not live_o:  # admit a request that may share a prefix
            rid = f"r{step}"
            prompt = rng.choice(prefixes)[: rng.randrange(0, 13)] + [rng.randrange(50) for _ in range(rng.randrange(1, 7))]
            so, sr = Seq(rid, list(prompt)), Seq(rid, list(prompt))
            ok = ours.can_reserve(so, so.num_tokens)
            assert ok == ref.can_reserve(sr, sr.num_tokens)
            if ok:
                ours.reserve(so, so.num_tokens)
                ref.reserve(sr, sr.num_tokens)
                assert so.num_cached_tokens == sr.num_cached_tokens
                cache_everything(ours, so)
                cache_everything(ref, sr)
                live_o[rid], live_r[rid] = so, sr
        elif action < 0.75:  # grow by a few verified tokens and report them cached
            rid = rng.choice(sorted(live_o))
            so, sr = live_o[rid], live_r[rid]
            extra = [rng.randrange(50) for _ in range(rng.randrange(1, 6))]
            n = so.num_tokens + len(extra)
            ok = ours.can_reserve(so, n)
            assert ok == ref.can_reserve(sr, n)
            if ok:
                ours.reserve(so, n)
                ref.reserve(sr, n)
                for s in (so, sr):
                    s.token_ids += extra
                    s.num_cached_tokens = s.num_tokens
                ours.on_tokens_cached(so)
                ref.on_tokens_cached(sr)
        else:
            rid = rng.choice(sorted(live_o))
            ours.free(live_o.pop(rid))
            ref.free(live_r.pop(rid))
        assert _snapshot(ours, live_o) == _snapshot(ref, live_r), f"step {step}"


# ------------------------------------------------------------- speculation safety
def _speculate(alloc, seq, rng, k, protocol):
    """One verify step of a sequence on the host: reserve L + g, write positions
    L-1 .. L-1+g, keep a random prefix of the guesses plus one token.

    protocol "product": the runner's order (register after acceptance with
    num_cached = L + kept).  protocol "reference": speculative_generator.py:70-85 with
    score_tokens' registration (model_runner.py:58-61) while the guesses are appended.
    Returns the written positions."""
    L = seq.num_tokens
    g = rng.randrange(0, k + 1)
    guesses = [rng.randrange(50) for _ in range(g)]
    alloc.reserve(seq, L + g)
    written = list(range(L - 1, L + g))
    kept = rng.randrange(0, g + 1)
    bonus = rng.randrange(50)
    if protocol == "reference":
        seq.token_ids += guesses
        seq.num_cached_tokens += 1 + g
        alloc.on_tokens_cached(seq)
        del seq.token_ids[L:]
        seq.token_ids += guesses[:kept] + [bonus]
        seq.num_cached_tokens = L + kept
    else:
        seq.token_ids += guesses[:kept] + [bonus]
        seq.num_cached_tokens = L + kept
        alloc.on_tokens_cached(seq)
    return written


def _registered_keys_match_tokens(alloc, seqs):
    """Every registered block in a live table holds the key of that table's verified tokens."""
    pool = alloc.blocks if isinstance(alloc, op.PrefixCachingSlotAllocator) else alloc.pool
    key_of = pool.key_of if isinstance(alloc, op.PrefixCachingSlotAllocator) else pool._key_of
    for seq in seqs:
        table = alloc.block_table(seq)
        want = op.build_block_keys(seq.token_ids, BLOCK, min(len(table), seq.num_cached_tokens // BLOCK))
        for i, key in enumerate(want):
            got = key_of.get(table[i])
            if got is not None and got != key:
                return False
    return True


@pytest.mark.parametrize("seed", range(6))
def test_verified_only_registration_never_exposes_a_guess_or_writes_a_shared_block(seed):
    rng = random.Random(seed)
    alloc = pm.PrefixCachingSlotAllocator(512, BLOCK, CPU)
    prefix = [rng.randrange(50) for _ in range(9)]
    live = []
    for i in range(4):
        seq = Seq(f"s{i}", prefix + [rng.randrange(50) for _ in range(rng.randrange(1, 6))])
        alloc.reserve(seq, seq.num_tokens)
        if i:
            assert seq.num_cached_tokens == 8  # two full blocks of the shared 9-token prefix
        assert seq.num_cached_tokens >= alloc.first_writable_position(seq)
        seq.num_cached_tokens = seq.num_tokens
        alloc.on_tokens_cached(seq)
        seq.token_ids.append(rng.randrange(50))  # the prefill's sampled token, not yet cached
        live.append(seq)
    for _ in range(40):
        for seq in live:
            bound = alloc.first_writable_position(seq)
            # state at write time: the step's own kept tokens may register blocks after it
            before = {b: (alloc.pool.reference_count(b), alloc.pool.is_registered(b))
                      for b in alloc.block_table(seq)}
            written = _speculate(alloc, seq, rng, 4, "product")
            table = alloc.block_table(seq)
            for pos in written:
                block = table[pos // BLOCK]
                assert pos >= bound
                assert before.get(block, (1, False)) == (1, False), \
                    f"{seq.request_id} wrote position {pos} into a shared or registered block"
        assert _registered_keys_match_tokens(alloc, live)
    # a later request with one sequence's verified history reuses its blocks
    donor = live[0]
    probe = Seq("probe", list(donor.token_ids))
    alloc.reserve(probe, probe.num_tokens)
    full = min(donor.num_cached_tokens, probe.num_tokens - 1) // BLOCK
    assert alloc.block_table(probe)[:full] == alloc.block_table(donor)[:full]


def test_the_reference_protocol_would_register_a_rejected_guess():
    """Why the runner registers after acceptance: registering while guesses are
    appended (model_runner.py:60-61) leaves a block keyed by tokens the sequence
    never kept, whose slots are later overwritten."""
    for seed in range(50):
        rng = random.Random(seed)
        alloc = op.PrefixCachingSlotAllocator(64, BLOCK)
        seq = Seq("s", [rng.randrange(50) for _ in range(5)])
        cache_everything(alloc, seq)
        seq.token_ids.append(rng.randrange(50))
        for _ in range(10):
            _speculate(alloc, seq, rng, 4, "reference")
        if not _registered_keys_match_tokens(alloc, [seq]):
            return
    pytest.fail("no seed exposed the reference protocol's stale registration")


def test_runner_refuses_a_write_below_the_shared_bound():
    alloc = pm.PrefixCachingSlotAllocator(8, BLOCK, CPU)
    seq = Seq("s", list(SHARED) + [1])
    cache_everything(alloc, seq)
    assert alloc.first_writable_position(seq) == 8
    assert pm.PagedSlotAllocator(8, BLOCK, CPU).first_writable_position(seq) == 0
    alloc.free(seq)
    assert alloc.first_writable_position(seq) == 0
