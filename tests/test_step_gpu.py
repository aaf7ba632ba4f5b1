"""A4: device packing of a batched verify step, bit-exact against the oracle.

ne_prepare_verify_step replaces build_step_inputs (ne/engine/generation/batch_builder.py:22-65)
and the paged slot arithmetic (ne/engine/memory/paged_allocator.py:69-79) for a verify step.
oracle.paging.build_step_inputs restates those for sequences whose token list is the
history plus this step's guesses and whose cached count is history_len - 1.  Every real
row's token, position and slot, the pads (token 0, position 0, the scratch slot), and the
per-sequence q_start / q_len / ctx_len must be identical.  Block tables come from the
oracle's paged allocator (FIFO free list), reserved for L + g tokens per sequence, so
positions cross block boundaries; draft counts are ragged (0..k) and some slots inactive.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import paging as opg
from nanoengine_amd import kernels

pytestmark = pytest.mark.gpu


def _case(rng, num_seqs, k, block_size, num_blocks, inactive_every):
    alloc = opg.PagedSlotAllocator(num_blocks, block_size)
    histories, drafts, active = [], [], []
    for b in range(num_seqs):
        is_active = inactive_every == 0 or b % inactive_every != inactive_every - 1
        # lengths that put the step's rows on both sides of a block boundary
        L = int(rng.integers(1, 6 * block_size)) if b % 3 else block_size * int(rng.integers(1, 5)) - int(
            rng.integers(0, 2))
        L = max(L, 1)
        g = int(rng.integers(0, k + 1))
        histories.append(rng.integers(0, 151936, size=L).tolist() if is_active else [])
        drafts.append(rng.integers(0, 151936, size=g).tolist() if is_active else [])
        active.append(is_active)
        if is_active:
            alloc.reserve(f"s{b}", L + g)
    return alloc, histories, drafts, active


@pytest.mark.parametrize("num_seqs,k,block_size,inactive_every",
                         [(64, 4, 16, 0), (37, 4, 16, 5), (32, 8, 16, 0), (9, 4, 32, 3), (1, 15, 16, 0)])
def test_prepare_verify_step_matches_build_step_inputs(device, num_seqs, k, block_size, inactive_every):
    rng = np.random.default_rng(1000 * num_seqs + k)
    num_blocks = num_seqs * 8
    alloc, histories, drafts, active = _case(rng, num_seqs, k, block_size, num_blocks, inactive_every)
    R = k + 1
    cap = max(max(len(h) for h in histories) + R, 1)
    max_blocks = -(-cap // block_size)
    hist = torch.zeros(num_seqs, cap, dtype=torch.int32)
    hlen = torch.zeros(num_seqs, dtype=torch.int32)
    dr = torch.zeros(num_seqs, k, dtype=torch.int32)
    nd = torch.zeros(num_seqs, dtype=torch.int32)
    tables = torch.zeros(num_seqs, max_blocks, dtype=torch.int32)
    for b in range(num_seqs):
        hist[b, : len(histories[b])] = torch.tensor(histories[b], dtype=torch.int32)
        hlen[b] = len(histories[b])
        dr[b, : len(drafts[b])] = torch.tensor(drafts[b], dtype=torch.int32)
        nd[b] = len(drafts[b]) if active[b] else int(rng.integers(0, k + 1))  # ignored when inactive
        table = alloc.block_table(f"s{b}")
        tables[b, : len(table)] = torch.tensor(table, dtype=torch.int32)
    scratch = num_blocks * block_size
    rows = num_seqs * R
    dev = device
    out = {name: torch.full((n,), -7, dtype=torch.int32, device=dev) for name, n in
           (("tokens", rows), ("positions", rows), ("slot_mapping", rows), ("q_start", num_seqs),
            ("q_len", num_seqs), ("ctx_len", num_seqs))}
    kernels.prepare_verify_step(hist.to(dev), hlen.to(dev), dr.to(dev), nd.to(dev), tables.to(dev), block_size,
                                scratch, out["tokens"], out["positions"], out["slot_mapping"], out["q_start"],
                                out["q_len"], out["ctx_len"])
    torch.cuda.synchronize()
    got = {name: t.cpu() for name, t in out.items()}

    act = [b for b in range(num_seqs) if active[b]]
    ref = opg.build_step_inputs(
        [histories[b] + drafts[b] for b in act], [len(histories[b]) - 1 for b in act],
        [len(drafts[b]) + 1 for b in act],
        lambda c: alloc.build_context_slots([f"s{b}" for b in act], c), scratch)
    qmax = ref.token_ids.shape[1]
    for j, b in enumerate(act):
        n = len(drafts[b]) + 1
        rows_b = slice(b * R, b * R + n)
        assert got["tokens"][rows_b].tolist() == ref.token_ids[j, :n].tolist(), f"seq {b} tokens"
        assert got["positions"][rows_b].tolist() == ref.positions[j, :n].tolist(), f"seq {b} positions"
        assert got["slot_mapping"][rows_b].tolist() == ref.slot_mapping[j, :n].tolist(), f"seq {b} slots"
        # the oracle pads to the longest sequence, the kernel to k + 1: both pad alike
        pad_ref = min(qmax, R) - n
        pads = slice(b * R + n, b * R + n + pad_ref)
        assert got["tokens"][pads].tolist() == ref.token_ids[j, n : n + pad_ref].tolist()
        assert got["positions"][pads].tolist() == ref.positions[j, n : n + pad_ref].tolist()
        assert got["slot_mapping"][pads].tolist() == ref.slot_mapping[j, n : n + pad_ref].tolist()
        assert int(got["q_start"][b]) == b * R
        assert int(got["q_len"][b]) == n
        assert int(got["ctx_len"][b]) == len(histories[b]) - 1 + n  # the oracle's context end
    for b in range(num_seqs):
        first_pad = b * R + (len(drafts[b]) + 1 if active[b] else 0)
        assert got["tokens"][first_pad : (b + 1) * R].eq(0).all()
        assert got["positions"][first_pad : (b + 1) * R].eq(0).all()
        assert got["slot_mapping"][first_pad : (b + 1) * R].eq(scratch).all()
        if not active[b]:
            assert int(got["q_len"][b]) == 0 and int(got["ctx_len"][b]) == 0


def test_prepare_verify_step_clamps_an_out_of_range_draft_count(device):
    """A draft count above max_drafts packs max_drafts guesses (never a row of the next
    sequence or a table entry past the reservation)."""
    k, bs = 4, 16
    hist = torch.arange(40, dtype=torch.int32).reshape(2, 20)
    hlen = torch.tensor([20, 20], dtype=torch.int32)
    dr = torch.arange(100, 108, dtype=torch.int32).reshape(2, 4)
    nd = torch.tensor([9, -3], dtype=torch.int32)
    tables = torch.tensor([[3, 5], [7, 1]], dtype=torch.int32)
    rows = 2 * (k + 1)
    outs = [torch.zeros(rows, dtype=torch.int32, device=device) for _ in range(3)] + [
        torch.zeros(2, dtype=torch.int32, device=device) for _ in range(3)]
    kernels.prepare_verify_step(hist.to(device), hlen.to(device), dr.to(device), nd.to(device), tables.to(device),
                                bs, 999, *outs)
    torch.cuda.synchronize()
    tokens, positions, slots, qs, ql, cl = (t.cpu().tolist() for t in outs)
    assert tokens[:5] == [19, 100, 101, 102, 103] and positions[:5] == [19, 20, 21, 22, 23]
    assert slots[:5] == [5 * 16 + 3, 5 * 16 + 4, 5 * 16 + 5, 5 * 16 + 6, 5 * 16 + 7]
    assert tokens[5:] == [39, 0, 0, 0, 0] and slots[5:] == [1 * 16 + 3, 999, 999, 999, 999]
    assert ql == [5, 1] and cl == [24, 20] and qs == [0, 5]


@pytest.mark.parametrize("k", [1, 4, 15])
def test_advance_step_counts_follow_num_guesses(k):
    """ne_advance_step_counts (the n-gram path's next-step counters) against the
    reference's rule num_guesses = max(0, min(k, max_new - generated - 1))
    (speculative_generator.py:71-72, interface.num_guesses): generated advances by the
    emitted tokens and the sampling step by one for active slots; inactive slots get 0
    guesses and keep their counters.  Covers the limit boundary (0 guesses at
    max_new - 1 generated and beyond)."""
    from nanoengine_amd.interface import SamplingParams, num_guesses

    rng = np.random.default_rng(k)
    n = 300
    dev = torch.device("cuda:0")
    history_len = rng.integers(0, 50, size=n).astype(np.int32)
    history_len[::7] = 0
    num_out = rng.integers(1, k + 2, size=n).astype(np.int32)
    max_new = rng.integers(1, 64, size=n).astype(np.int32)
    generated = np.minimum(rng.integers(0, 64, size=n), max_new).astype(np.int32)
    steps = rng.integers(0, 1 << 40, size=n).astype(np.int64)
    t = lambda a: torch.from_numpy(a.copy()).to(dev)
    d_gen, d_steps = t(generated), t(steps)
    d_guess = torch.full((n,), -5, dtype=torch.int32, device=dev)
    kernels.advance_step_counts(t(history_len), t(num_out), t(max_new), d_gen, d_steps, d_guess, k)
    torch.cuda.synchronize()
    active = history_len > 0
    exp_gen = np.where(active, generated + num_out, generated)
    exp_steps = np.where(active, steps + 1, steps)
    exp_guess = np.array([num_guesses(SamplingParams(max_new_tokens=int(m)), int(g), k) if a else 0
                          for a, m, g in zip(active, max_new, exp_gen)], dtype=np.int32)
    assert np.array_equal(d_gen.cpu().numpy(), exp_gen)
    assert np.array_equal(d_steps.cpu().numpy(), exp_steps)
    assert np.array_equal(d_guess.cpu().numpy(), exp_guess)
    assert (exp_guess == 0).any() and (exp_guess == k).any()
