"""Host bookkeeping of one batched verify step: which slots need KV blocks, where
peeked blocks go in the tables, and appending each slot's emitted tokens
(ne/engine/generation/speculative_generator.py:54-72,
ne/engine/memory/paged_allocator.py:50-55).

The functions run in the ``_host_step`` CPython extension (csrc/host_step.c, built by
build.py) when it is built, ~0.1 us per slot; the Python definitions below are the same
contract, used when it is not and as the check of the extension in the tests.
"""

from __future__ import annotations

import numpy as np


def plan_growth_py(lengths, num_drafts, owned, active, block_size: int):
    """(slots, counts, targets, total): each active slot whose length + guesses exceeds its
    blocks * block_size, in slot order, with the blocks it needs and its token count."""
    slots, counts, targets = [], [], []
    for s in np.flatnonzero(active).tolist():
        need = int(lengths[s]) + int(num_drafts[s])
        if need > int(owned[s]) * block_size:
            slots.append(s)
            counts.append(-(-need // block_size) - int(owned[s]))
            targets.append(need)
    return slots, counts, targets, sum(counts)


def assign_blocks_py(tables, owned, slots, counts, blocks) -> None:
    """Slot slots[i] gets the next counts[i] blocks at table positions owned .. + c - 1."""
    at = 0
    for s, c in zip(slots, counts):
        tables[s, owned[s] : owned[s] + c] = blocks[at : at + c]
        owned[s] += c
        at += c


def finish_step_py(active, slots, out, num_out, num_drafts, act, lengths, generated, steps, max_new, honours,
                   stop_ids: tuple, result_type, on_cached):
    """(results, finishing): mirrors advance by the emitted counts; each active slot's
    sampling step advances; a slot that may finish (length limit, or a stop token emitted
    by a slot that honours stops) gets None in results and (slot, tokens) in finishing;
    any other appends its tokens and gets result_type(tokens, None, guesses, emitted - 1).

    Emitted counts outside [0, out.shape[1]] and active slots that are out of range,
    inactive or empty raise ValueError before any mirror changes.  A failure after that
    (token_ids not a list, on_cached raising) leaves the mirrors advanced and only some
    slots' tokens appended: the runner that called it must then be discarded."""
    width = out.shape[1]
    bad = act.astype(bool) & ((num_out < 0) | (num_out > width))
    if bad.any():
        s = int(np.flatnonzero(bad)[0])
        raise ValueError(f"slot {s} emitted {int(num_out[s])} tokens (at most {width})")
    for s in active:
        if not (0 <= s < len(act) and s < len(slots) and act[s] and slots[s] is not None):
            raise ValueError(f"active slot {s} out of range, inactive or empty")
    emitted = num_out * act
    lengths += emitted
    generated += emitted
    steps += act
    may_finish = (generated >= max_new) & act
    if stop_ids:
        hon = honours & act
        if hon.any():
            rows = np.arange(out.shape[1])[None, :] < num_out[:, None]
            hit = (np.isin(out, list(stop_ids)) & rows).any(axis=1)
            may_finish |= hon & hit
    rows_out, nout, nd, fin = out.tolist(), num_out.tolist(), num_drafts.tolist(), may_finish.tolist()
    results, finishing = {}, []
    for s in active:
        seq = slots[s]
        n = nout[s]
        seq.sampling_generator.step += 1
        tokens = rows_out[s][:n]
        if fin[s]:
            results[s] = None
            finishing.append((s, tokens))
            continue
        ids = seq.token_ids
        ids.extend(tokens)
        seq.num_cached_tokens = len(ids) - 1
        if on_cached is not None:
            on_cached(seq)
        results[s] = result_type(tokens, None, nd[s], n - 1)
    return results, finishing


try:
    from nanoengine_amd._host_step import assign_blocks, finish_step, plan_growth

    NATIVE = True
except ImportError:  # not built: the same contract in Python
    plan_growth, assign_blocks, finish_step = plan_growth_py, assign_blocks_py, finish_step_py
    NATIVE = False
