"""Batched speculative verify on the HIP kernels.

The reference verifies one sequence per call (ModelRunner.score_tokens,
ne/engine/generation/model_runner.py:52-62, driven by
SpeculativeGenerator._run_speculative_step, ne/engine/speculative/
speculative_generator.py:70-85).  ``VerifyRunner`` applies the same per-sequence
semantics to up to ``max_seqs`` sequences at once, with the token histories,
lengths, block tables and cached counts resident on the device:

  1. n-gram drafting on the device histories (ne_ngram_propose), or a draft
     model's greedy guesses (``DraftModelProposer``, nanoengine_amd/draft.py).  With
     n-gram drafting the previous step already proposed them: its device work ends by
     advancing the per-sequence counters (ne_advance_step_counts) and running the
     n-gram kernel for the next step, and its one readback brings the counts home; only
     a step after new sequences were admitted proposes (and reads back) first
  2. reserve KV blocks on the host allocator for L + g tokens per sequence
     (paged_allocator.py:50-55) and upload new table rows
  3. pack rows on the device (ne_prepare_verify_step), run the Qwen3 forward,
     the LM head (argmax partials only when greedy) and the fused acceptance,
     which appends kept tokens + 1 to the device history and rolls
     ``num_cached`` back to L + kept
  4. read back accepted tokens and update the host ``Sequence`` objects; only
     then, with the guesses gone and ``num_cached_tokens`` = L + kept, tell the
     allocator which tokens are cached (a prefix cache registers verified full
     blocks only)

Step 3 has fixed shapes (every slot owns k+1 padded rows), so it can be
captured once into a HIP graph and replayed.

With a prefix-caching allocator, a new sequence takes the cached blocks of its
prompt's start and its prefill computes only the remaining rows (queries at
positions c..p-1 over a context of p keys).
"""

from __future__ import annotations

import math
from collections import deque
from typing import TYPE_CHECKING, NamedTuple
from dataclasses import dataclass

import numpy as np
import torch

from nanoengine_amd import host_step, kernels
from nanoengine_amd.draft import DeviceGuesses
from nanoengine_amd.interface import find_finish_reason
from nanoengine_amd.memory import KVCachePool, PagedSlotAllocator
from nanoengine_amd.qwen3 import AttentionBatch, Qwen3VerifyModel
from nanoengine_amd.sequence_state import Sequence

if TYPE_CHECKING:
    from nanoengine_amd.draft import DraftModelProposer


def request_length_error(num_prompt_tokens: int, max_new_tokens: int, max_model_len: int) -> str | None:
    """Why a request cannot be admitted, or None (api/routes.py:98-111): an empty prompt,
    or prompt + max_new_tokens past max_model_len.  The device history rows hold
    max_model_len + k + 1 tokens; this keeps every append of a verify step inside them."""
    if num_prompt_tokens == 0:
        return "prompt is empty"
    total = num_prompt_tokens + max_new_tokens
    if total > max_model_len:
        return f"prompt + max_new_tokens = {total} exceeds max_model_len {max_model_len}"
    return None


def verify_graph_allowed(num_active: int, step_context: int, max_batch: int | None,
                         max_context: int | None) -> bool:
    """Whether a verify step may replay the captured HIP graph.  As the reference bounds
    its decode graphs by ``cuda_graph_max_batch`` and ``cuda_graph_max_context``
    (config.py:58-61, runtime.py:150-160, cuda_graph_runner.py:106-117), a step with more
    active sequences, or whose longest sequence attends to more tokens (its length plus
    the k guess rows), runs eagerly.  None leaves that bound off."""
    if max_batch is not None and num_active > max_batch:
        return False
    return max_context is None or step_context <= max_context


class StepResult(NamedTuple):
    """Tokens emitted for one sequence by one step, with its finish reason if it ended."""

    tokens: list[int]
    finish_reason: str | None
    num_guesses: int
    num_kept: int


class _Launched(NamedTuple):
    """A verify step launched and not yet completed on the host: its slots, the read-back
    buffer its outputs go to (rb), the one holding its guess counts (gb), and the event
    recorded after its read-back copy."""

    active: list[int]
    act: np.ndarray
    traced_drafts: dict | None
    rb: int
    gb: int
    event: torch.cuda.Event


class VerifyRunner:
    def __init__(
        self,
        model: Qwen3VerifyModel,
        pool: KVCachePool,
        allocator: PagedSlotAllocator,
        max_seqs: int,
        num_speculative_tokens: int,
        max_ngram: int,
        max_model_len: int,
        stop_token_ids: frozenset[int] = frozenset(),
        use_graph: bool = False,
        proposer: "DraftModelProposer | None" = None,
        graph_max_batch: int | None = None,
        graph_max_context: int | None = None,
    ) -> None:
        self.model = model
        # None: n-gram drafting on the device histories; else a draft model's greedy guesses
        self.proposer = proposer
        self.pool = pool
        self.allocator = allocator
        # the shared-block guard only has something to check with a prefix cache, and only
        # a prefix cache acts on newly cached tokens
        self._guard_shared = type(allocator).first_writable_position is not PagedSlotAllocator.first_writable_position
        self._track_cached = type(allocator).on_tokens_cached is not PagedSlotAllocator.on_tokens_cached
        self.device = model.device
        self.k = num_speculative_tokens
        self.R = self.k + 1
        self.max_seqs = max_seqs
        self.max_ngram = max_ngram
        self.stop_token_ids = stop_token_ids
        self.block_size = allocator.block_size
        self.max_model_len = max_model_len
        self.capacity = max_model_len + self.R
        self.max_blocks = math.ceil(self.capacity / self.block_size)
        self.use_graph = use_graph
        # steps beyond these bounds run eagerly (verify_graph_allowed); a capture that ran
        # out of device memory leaves the runner eager for good
        self.graph_max_batch = graph_max_batch
        self.graph_max_context = graph_max_context
        self.graph_failed = False
        model.ensure_rope(self.capacity)
        if self.max_seqs * self.R > model.max_rows:
            raise ValueError("model activation buffers are smaller than max_seqs * (k + 1) rows")
        dev = self.device
        i32 = dict(dtype=torch.int32, device=dev)
        self.history = torch.zeros(max_seqs, self.capacity, **i32)
        self.history_len = torch.zeros(max_seqs, **i32)
        self.num_cached = torch.zeros(max_seqs, **i32)
        self.block_tables = torch.zeros(max_seqs, self.max_blocks, **i32)
        self.num_tokens = torch.zeros(max_seqs, **i32)
        self.drafts = torch.zeros(max_seqs, self.k, **i32)
        # what the host reads back after a step -- emitted tokens, their counts and the
        # next step's guess counts -- in one buffer, so that one copy fetches it
        self.step_out = torch.zeros(max_seqs * (self.R + 2), **i32)
        self.out_tokens, self.num_out, self.num_drafts = self._step_out_views(self.step_out)
        # length limit and generated count per slot, advanced on the device after each
        # step so that the next step's n-gram guesses need no host round trip
        self.max_new = torch.zeros(max_seqs, **i32)
        self.generated = torch.zeros(max_seqs, **i32)
        self.seeds = torch.zeros(max_seqs, dtype=torch.int64, device=dev)
        self.steps = torch.zeros(max_seqs, dtype=torch.int64, device=dev)
        # per-slot sampling parameters (sampling.py:30-38): temperature 0 verifies greedily
        self.temperatures = torch.zeros(max_seqs, dtype=torch.float32, device=dev)
        self.top_ps = torch.ones(max_seqs, dtype=torch.float32, device=dev)
        rows = max_seqs * self.R
        self.tokens = torch.zeros(rows, **i32)
        self.positions = torch.zeros(rows, **i32)
        self.slot_mapping = torch.zeros(rows, **i32)
        self.q_start = torch.zeros(max_seqs, **i32)
        self.q_len = torch.zeros(max_seqs, **i32)
        self.ctx_len = torch.zeros(max_seqs, **i32)
        self.row_start = torch.arange(max_seqs, **i32) * self.R
        vocab = model.config.vocab_size
        self.argmax_partials = torch.zeros(rows, kernels.lm_head_num_tiles(vocab), dtype=torch.int64,
                                           device=dev)
        self.logits: torch.Tensor | None = None  # allocated for sampled batches only
        pin = dict(pin_memory=True)
        self.h_tables = torch.zeros(max_seqs, self.max_blocks, dtype=torch.int32, **pin)
        self.h_num_tokens = torch.zeros(max_seqs, dtype=torch.int32, **pin)
        self.h_steps = torch.zeros(max_seqs, dtype=torch.int64, **pin)
        self.h_drafts = torch.zeros(max_seqs, self.k, dtype=torch.int32, **pin)
        # three host copies of step_out, used in turn: a step reads back into one while
        # its guess counts (read back by the step before it, n-gram drafting) sit in the
        # previous one, and with two steps in flight a third receives the later one's
        self.h_step_out = [torch.zeros(max_seqs * (self.R + 2), dtype=torch.int32, **pin) for _ in range(3)]
        self._read_back_events = [torch.cuda.Event() for _ in range(3)]
        self._last_rb = 0  # read-back buffer of the most recently launched step
        self._bind_read_back(1, 0)
        # numpy views of the pinned buffers: the per-step host work indexes them per
        # sequence, which costs ~1 us through torch and ~0.1 us through numpy
        self.np_tables = self.h_tables.numpy()
        self.np_num_tokens = self.h_num_tokens.numpy()
        self.np_steps = self.h_steps.numpy()
        # whether the device drafts / num_drafts already hold this step's n-gram guesses
        # (proposed at the end of the previous step, no sequence admitted since)
        self._drafts_ready = False
        # steps launched and not yet waited for (oldest first, at most two), and the
        # results of steps finished early because the batch changed, in step order
        self._inflight: deque[_Launched] = deque()
        self._pending: deque[dict[int, StepResult]] = deque()
        self.run_ahead = True  # False: every step launches and finishes in its own call
        self.ahead_launches = 0  # steps launched before the previous step's bookkeeping
        self.deep_launches = 0  # of those, launched while the previous step still ran
        # a plain paged allocator hands out blocks from the head of a FIFO free list, so a
        # step's new table entries are known before the allocator records them
        self._fifo_blocks = type(allocator) is PagedSlotAllocator
        # per-slot host state mirrored from the Sequence objects, so that a step's counts
        # and block checks are array operations: active, length L, generated tokens,
        # length limit, blocks owned
        self.np_active = np.zeros(max_seqs, dtype=bool)
        self.np_len = np.zeros(max_seqs, dtype=np.int64)
        self.np_gen = np.zeros(max_seqs, dtype=np.int64)
        self.np_max_new = np.zeros(max_seqs, dtype=np.int64)
        self.np_owned = np.zeros(max_seqs, dtype=np.int64)
        self.np_temp = np.zeros(max_seqs, dtype=np.float32)
        self.np_top_p = np.ones(max_seqs, dtype=np.float32)
        # whether each slot's sequence ends at a stop token (ignore_eos unset)
        self.np_honours_stop = np.zeros(max_seqs, dtype=bool)
        self.slots: list[Sequence | None] = [None] * max_seqs
        # the active slot list and whether any samples, kept between slot changes
        self._active: list[int] | None = None
        self._sampled: bool | None = None
        self.graph: torch.cuda.CUDAGraph | None = None
        # whether the captured step computes full logits (some slot samples) or only the
        # LM head's argmax partials (every slot greedy)
        self.graph_sampled: bool | None = None
        self.batch = AttentionBatch(self.positions, self.slot_mapping, self.q_start, self.q_len,
                                    self.ctx_len, self.block_tables, self.R, self.capacity)
        # set to a list to record, per verify step, each slot's history, drafts,
        # emitted tokens and block table (used by the parity tests)
        self.trace: list | None = None

    def _step_out_views(self, buf: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        """out_tokens [max_seqs, R], num_out [max_seqs], num_drafts [max_seqs] of a step_out buffer."""
        n, r = self.max_seqs, self.R
        return buf[: n * r].view(n, r), buf[n * r : n * (r + 1)], buf[n * (r + 1) :]

    def _bind_read_back(self, rb: int, gb: int) -> None:
        """Host views of a step: it reads back into h_step_out[rb]; its guess counts are
        the num_drafts part of h_step_out[gb] (read back by the step before it, or staged
        there by the host)."""
        if not hasattr(self, "_read_back_views"):
            views = [self._step_out_views(buf) for buf in self.h_step_out]
            self._read_back_views = [(v, tuple(t.numpy() for t in v)) for v in views]
        (self.h_out, self.h_num_out, self.h_num_drafts_next), (self.np_out, self.np_num_out,
                                                                self.np_num_drafts_next) = \
            self._read_back_views[rb]
        other = self._read_back_views[gb]
        self.h_num_drafts, self.np_num_drafts = other[0][2], other[1][2]

    # ------------------------------------------------------------------ slots
    @property
    def active_slots(self) -> list[int]:
        if self._active is None:
            self._active = [i for i, s in enumerate(self.slots) if s is not None]
        return list(self._active)

    def _slots_changed(self) -> None:
        self._active = None
        self._sampled = None

    def free_slots(self) -> list[int]:
        """Empty slots.  A slot whose sequence finished in a step whose results wait for
        the next step() call (``pending``) is not free until that call has returned them,
        so a result is never reported under a slot that a new request already holds."""
        waiting = set().union(*self._pending) if self._pending else ()
        return [i for i, s in enumerate(self.slots) if s is None and i not in waiting]

    @property
    def stop_token_ids(self) -> frozenset[int]:
        return self._stop_token_ids

    @stop_token_ids.setter
    def stop_token_ids(self, ids) -> None:
        """The per-step bookkeeping matches emitted tokens against a sorted tuple."""
        self._stop_token_ids = frozenset(ids)
        self._stop_ids = tuple(sorted(self._stop_token_ids))

    @property
    def any_sampled(self) -> bool:
        """Whether some active slot samples (temperature > 0)."""
        if self._sampled is None:
            self._sampled = bool((self.np_temp[self.np_active] > 0).any())
        return self._sampled


    def add(self, sequences: list[Sequence]) -> list[int]:
        """Place sequences in free slots, reserve their prompts, prefill them and emit
        the first token of each (model_runner.py:33-50 + speculative_generator.py:50-53)."""
        self.drain()
        free = self.free_slots()
        if len(sequences) > len(free):
            raise ValueError(f"only {len(free)} free sequence slots")
        for seq in sequences:
            problem = request_length_error(seq.num_tokens, seq.sampling_params.max_new_tokens, self.max_model_len)
            if problem is not None:
                raise ValueError(f"{seq.request_id}: {problem}")
        slots = free[: len(sequences)]
        results = {}
        # prefill contiguous runs of slots together
        run: list[tuple[int, Sequence]] = []
        for slot, seq in zip(slots, sequences, strict=True):
            if run and slot != run[-1][0] + 1:
                results.update(self._prefill(run))
                run = []
            run.append((slot, seq))
        if run:
            results.update(self._prefill(run))
        return results

    def _prefill(self, run: list[tuple[int, Sequence]]) -> dict[int, StepResult]:
        """Reserve and prefill a run of consecutive slots, then emit each first token.

        The uncached rows of the run are packed in slot order into forwards of at most
        ``model.max_rows`` rows; a prompt longer than the room left is cut into chunks
        (as the reference's chunked prefill does), each chunk's queries attending to
        every key before them (queries at positions a..e-1 over e keys)."""
        dev = self.device
        s0 = run[0][0]
        n = len(run)
        pending: deque[list] = deque()
        self._slots_changed()
        # the run's device state is staged on the host and copied once per tensor (a host
        # scalar assigned to a device tensor is one synchronous copy each)
        width = max(seq.num_tokens for _, seq in run)
        hist = np.zeros((n, width), dtype=np.int32)
        lens = np.zeros(n, dtype=np.int32)
        seeds = np.zeros(n, dtype=np.int64)
        steps = np.zeros(n, dtype=np.int64)
        for i, (slot, seq) in enumerate(run):
            self.slots[slot] = seq
            p = seq.num_tokens
            seq.num_cached_tokens = 0
            self.allocator.reserve(seq, p)  # a prefix cache sets num_cached_tokens to its hit
            c = seq.num_cached_tokens
            if c < self.allocator.first_writable_position(seq):
                raise RuntimeError(f"prefill of {seq.request_id} would write into a shared block")
            table = self.allocator.block_table(seq)
            self.np_tables[slot] = 0
            self.np_tables[slot, : len(table)] = table
            hist[i, :p] = seq.token_ids
            lens[i] = p
            seeds[i] = seq.sampling_generator.seed
            steps[i] = seq.sampling_generator.step
            params = seq.sampling_params
            self.np_temp[slot] = max(float(params.temperature), 0.0)
            self.np_top_p[slot] = float(params.top_p)
            pending.append([slot, seq, c, p])
        sl = slice(s0, s0 + n)
        self.history[sl, :width] = torch.from_numpy(hist)
        self.history_len[sl] = torch.from_numpy(lens)
        self.seeds[sl] = torch.from_numpy(seeds)
        self.steps[sl] = torch.from_numpy(steps)
        self.temperatures[sl] = torch.from_numpy(self.np_temp[sl].copy())
        self.top_ps[sl] = torch.from_numpy(self.np_top_p[sl].copy())
        self.block_tables.copy_(self.h_tables, non_blocking=True)
        while pending:
            pieces, room = [], self.model.max_rows
            while pending and room > 0:
                slot, seq, a, p = pending[0]
                e = min(p, a + room)
                pieces.append((slot, seq, a, e, p))
                room -= e - a
                if e < p:
                    pending[0][2] = e
                    break
                pending.popleft()
            self._prefill_forward(pieces)
        self.h_out[s0 : s0 + n].copy_(self.out_tokens[s0 : s0 + n], non_blocking=True)
        torch.cuda.current_stream(dev).synchronize()
        results = {}
        for i, (slot, seq) in enumerate(run):
            seq.num_cached_tokens = seq.num_tokens
            self.allocator.on_tokens_cached(seq)  # the whole prompt is verified and cached
            seq.sampling_generator.step += 1
            self.np_active[slot] = True
            self.np_honours_stop[slot] = not seq.sampling_params.ignore_eos
            self.np_max_new[slot] = seq.sampling_params.max_new_tokens
            self.np_owned[slot] = self.allocator.num_blocks_of(seq)
            self.np_steps[slot] = seq.sampling_generator.step
            results[slot] = self._emit(slot, seq, [int(self.h_out[s0 + i, 0])], 0, 0)
            self.np_len[slot] = seq.num_tokens
            self.np_gen[slot] = seq.num_generated_tokens
        self.max_new[sl] = torch.from_numpy(self.np_max_new[sl].astype(np.int32))
        self.generated[sl] = torch.from_numpy(self.np_gen[sl].astype(np.int32))
        self._drafts_ready = False  # the new slots have no guesses yet
        self._slots_changed()
        return results

    def _prefill_forward(self, pieces: list[tuple[int, Sequence, int, int, int]]) -> None:
        """One forward over (slot, seq, a, e, p) pieces of consecutive slots; the pieces
        that end their prompt (e == p, a leading run of them) get their first token."""
        dev = self.device
        tokens, positions, slots, q_start, q_len, ctx_len = [], [], [], [], [], []
        row = 0
        for slot, seq, a, e, p in pieces:
            pos = np.arange(a, e)
            tokens.append(np.asarray(seq.token_ids[a:e], dtype=np.int32))
            positions.append(pos.astype(np.int32))
            slots.append(self.allocator.slots_for(seq, pos).astype(np.int32))
            q_start.append(row)
            q_len.append(e - a)
            ctx_len.append(e)
            row += e - a
        t = lambda x: torch.from_numpy(np.concatenate(x)).to(dev)
        tok, posn, slot_map = t(tokens), t(positions), t(slots)
        qs = torch.tensor(q_start, dtype=torch.int32, device=dev)
        ql = torch.tensor(q_len, dtype=torch.int32, device=dev)
        cl = torch.tensor(ctx_len, dtype=torch.int32, device=dev)
        s0 = pieces[0][0]
        batch = AttentionBatch(posn, slot_map, qs, ql, cl, self.block_tables[s0 : s0 + len(pieces)], max(q_len),
                               max(ctx_len))
        hidden = self.model.forward(row, tok, batch, self.pool, workspace=self.model.eager_workspace)
        nf = sum(1 for piece in pieces if piece[3] == piece[4])
        if nf == 0:
            return
        last = hidden.index_select(0, (qs[:nf] + ql[:nf] - 1).long())
        sampled = bool((self.np_temp[s0 : s0 + nf] > 0).any())
        logits, partials = self.model.compute_logits(last, logits=sampled, argmax=not sampled)
        zeros = torch.zeros(nf, dtype=torch.int32, device=dev)
        sl = slice(s0, s0 + nf)
        kernels.accept(
            self.drafts[sl], zeros, torch.arange(nf, dtype=torch.int32, device=dev),
            self.model.config.vocab_size, logits=logits, argmax_partials=partials,
            temperature=self.temperatures[sl], top_p=self.top_ps[sl], any_sampled=sampled,
            seeds=self.seeds[sl], steps=self.steps[sl],
            out_tokens=self.out_tokens[sl], num_out=self.num_out[sl], history=self.history[sl],
            history_len=self.history_len[sl], num_cached=self.num_cached[sl],
        )

    # ------------------------------------------------------------- verify step
    def _device_step(self, sampled: bool) -> None:
        """Fixed-shape part of the verify step: pack, forward, LM head, accept.  ``sampled``:
        some slot samples, so the LM head writes every row's logits (greedy slots take
        their argmax from them); otherwise it writes only the argmax partials."""
        kernels.prepare_verify_step(
            self.history, self.history_len, self.drafts, self.num_drafts, self.block_tables,
            self.block_size, self.pool.scratch_slot, self.tokens, self.positions, self.slot_mapping,
            self.q_start, self.q_len, self.ctx_len,
        )
        rows = self.max_seqs * self.R
        hidden = self.model.forward(rows, self.tokens, self.batch, self.pool)
        if not sampled:
            self.model.compute_logits(hidden, logits=False, argmax=self.argmax_partials)
            logits = None
        else:
            if self.logits is None:
                self.logits = torch.empty(rows, self.model.config.vocab_size, dtype=torch.bfloat16,
                                          device=self.device)
            self.model.compute_logits(hidden, logits=self.logits, argmax=False)
            logits = self.logits
        draft_logits = None if not sampled or self.proposer is None else self.proposer.logits
        kernels.accept(
            self.drafts, self.num_drafts, self.row_start, self.model.config.vocab_size, logits=logits,
            argmax_partials=None if sampled else self.argmax_partials,
            temperature=self.temperatures, top_p=self.top_ps, any_sampled=sampled,
            seeds=self.seeds, steps=self.steps,
            out_tokens=self.out_tokens, num_out=self.num_out, history=self.history,
            history_len=self.history_len, num_cached=self.num_cached,
            # a sampled draft model's guesses are verified against its distributions
            draft_logits=draft_logits,
            draft_row_start=None if draft_logits is None else self.proposer.row_start,
        )
        if self.proposer is None:
            # the next step's guess counts, then its n-gram guesses on the updated histories
            kernels.advance_and_propose(self.history, self.history_len, self.num_out, self.max_new,
                                        self.generated, self.steps, self.num_tokens, self.k, self.max_ngram,
                                        self.drafts, self.num_drafts)

    def graph_allowed(self, lengths: np.ndarray | None = None) -> bool:
        """Whether the step over the active slots, at ``lengths`` (default: the current
        host mirrors), replays the captured graph rather than running eagerly."""
        if not self.use_graph or self.graph_failed:
            return False
        act = self.np_active
        n = int(act.sum())
        lengths = self.np_len if lengths is None else lengths
        context = int(lengths[act].max()) + self.k if n else 0
        return verify_graph_allowed(n, context, self.graph_max_batch, self.graph_max_context)

    def capture_graph(self) -> None:
        """Capture the verify step's HIP graph before any request is admitted, as the
        reference captures its decode graphs when the engine is created
        (runtime.py:150-160, cuda_graph_runner.py:94-105), so that no request waits for a
        capture: the step runs once with every slot inactive (padding rows only, which
        write the pool's scratch slot) and is then recorded.  A batch with sampled slots
        captures its own graph at its first step."""
        if not self.use_graph or self.graph is not None or self.graph_failed or self.np_active.any():
            return
        self._run_device_step()
        torch.cuda.current_stream(self.device).synchronize()

    def _run_device_step(self) -> None:
        sampled = self.any_sampled
        if not self.graph_allowed():
            self._device_step(sampled)
            return
        if self.graph is None or self.graph_sampled != sampled:
            # this step runs eagerly (which also allocates lazily created buffers and
            # workspaces); the capture below only records, so nothing runs twice
            self._device_step(sampled)
            torch.cuda.current_stream(self.device).synchronize()
            graph = torch.cuda.CUDAGraph()
            try:
                with torch.cuda.graph(graph):
                    self._device_step(sampled)
            except torch.cuda.OutOfMemoryError:
                # as cuda_graph_runner.py:193-207: without the memory to capture, every
                # later step runs eagerly (this one already ran)
                self.graph, self.graph_failed = None, True
                del graph
                torch.cuda.empty_cache()
                return
            self.graph = graph
            self.model.bind_graph()
            self.graph_sampled = sampled
            return
        self.graph.replay()

    def step(self) -> dict[int, StepResult]:
        """One verify step over every active slot; returns what each slot emitted.

        When nothing can change the batch before the next step (no slot can finish in
        this one, n-gram guesses, the plain paged allocator, a captured graph, no trace),
        the next step is launched as soon as this one's outputs are read back, before its
        tokens are appended to the sequences: the device runs it while the host does that
        bookkeeping, and the next call waits for it instead of launching one.  When no slot
        can finish in a launched step whatever it emits (no slot honours stop tokens and
        none can reach its length limit), the step after it is launched right away too,
        with blocks reserved for the most it can need, so the device never waits for the
        host between the two.  A batch change (add, release) first finishes the steps in
        flight and keeps their results for the next calls."""
        if self._pending:
            return self._pending.popleft()
        if not self._inflight:
            launched = self._launch()
            if launched is None:
                return {}
            self._inflight.append(launched)
            self._maybe_launch_deep()
        launched = self._inflight.popleft()
        launched.event.synchronize()
        return self._complete(launched, allow_ahead=True)

    @property
    def pending(self) -> bool:
        """Whether a finished step's results wait for the next step() call."""
        return bool(self._pending)

    def drain(self) -> None:
        """Finish the steps launched ahead (before the batch changes, or before the device
        is used for something else); their results are returned by the next step() calls."""
        while self._inflight:
            launched = self._inflight.popleft()
            launched.event.synchronize()
            results = self._complete(launched, allow_ahead=False)
            if results:
                self._pending.append(results)

    def _launch(self, bound: tuple[np.ndarray, np.ndarray] | None = None) -> _Launched | None:
        """Guesses, block growth and the device step of one verify step, up to its
        outputs' read-back copy (not waited for); None when no slot is active.

        ``bound`` (a step launched while the one before it still runs): the lengths and
        guess counts its blocks must cover at most, since its own are not known yet;
        its guesses are the ones the running step proposes on the device."""
        if self._active is None:
            self._active = [i for i, s in enumerate(self.slots) if s is not None]
        active = self._active
        if not active:
            return None
        slots = self.slots
        act = self.np_active.copy()
        ngram = self.proposer is None
        gb, rb = self._last_rb, (self._last_rb + 1) % len(self.h_step_out)
        self._bind_read_back(rb, gb)
        if bound is not None:
            pass
        elif not (ngram and self._drafts_ready) or self.trace is not None:
            # num_guesses for every slot at once (speculative_generator.py:71-72); n-gram
            # guesses proposed at the end of the previous step come with the device's counts
            counts = np.minimum(self.np_max_new - self.np_gen - 1, self.k)
            np.maximum(counts, 0, out=counts)
            counts *= act
            self.np_num_tokens[:] = counts
        if bound is not None:
            pass
        elif ngram:
            if not self._drafts_ready:
                self.num_tokens.copy_(self.h_num_tokens, non_blocking=True)
                self.steps.copy_(self.h_steps, non_blocking=True)
                kernels.ngram_propose(self.history, self.history_len, self.num_tokens, self.max_ngram, self.k,
                                      drafts=self.drafts, num_drafts=self.num_drafts)
                self.h_num_drafts.copy_(self.num_drafts, non_blocking=True)
                torch.cuda.current_stream(self.device).synchronize()
            # else: the previous step proposed them and read back their counts
        else:
            self.num_tokens.copy_(self.h_num_tokens, non_blocking=True)
            self.steps.copy_(self.h_steps, non_blocking=True)
            # greedy guesses from the draft's captured graphs stay on the device: the step
            # reads them there, and the host only needs their counts (not with a trace)
            guesses = self.proposer.propose({s: slots[s] for s in active},
                                            {s: int(self.np_num_tokens[s]) for s in active},
                                            temperature=self.np_temp, top_p=self.np_top_p,
                                            seeds=self.seeds,
                                            steps=self.np_steps,
                                            device_out=self.drafts if self.trace is None else None)
            self.np_num_drafts[:] = 0
            if isinstance(guesses, DeviceGuesses):
                for s, n in guesses.counts.items():
                    self.np_num_drafts[s] = n
            else:
                np_drafts = self.h_drafts.numpy()
                for s, g in guesses.items():
                    np_drafts[s, : len(g)] = g
                    self.np_num_drafts[s] = len(g)
                self.drafts.copy_(self.h_drafts, non_blocking=True)
            self.num_drafts.copy_(self.h_num_drafts, non_blocking=True)
        np_num_drafts, allocator, bs = self.np_num_drafts, self.allocator, self.block_size
        lengths, drafts = (self.np_len, np_num_drafts) if bound is None else bound
        if self._guard_shared:
            # rows write positions L-1 .. L-1+g; every block below the allocator's
            # bound may be read by other requests and must never be written
            for s in active:
                seq = slots[s]
                if seq.num_tokens - 1 < allocator.first_writable_position(seq):
                    raise RuntimeError(f"verify step of {seq.request_id} would write into a shared block")
        # slots whose length + guesses outgrow their blocks (paged_allocator.py:50-55)
        grow, counts, targets, total = host_step.plan_growth(lengths, drafts, self.np_owned, act, bs)
        deferred = None
        if grow:
            np_tables, np_owned = self.np_tables, self.np_owned
            # a FIFO allocator's next blocks, in slot order, go into the tables now; the
            # allocator records them while the device runs the step
            blocks = allocator.peek_free(total) if self._fifo_blocks else None
            if blocks is not None:
                host_step.assign_blocks(np_tables, np_owned, grow, counts, blocks)
                deferred = (grow, counts, blocks)
            else:
                for s, target in zip(grow, targets):
                    owned = int(np_owned[s])
                    added = allocator.reserve(slots[s], target)
                    np_tables[s, owned : owned + len(added)] = added
                    np_owned[s] = owned + len(added)
            self.block_tables.copy_(self.h_tables, non_blocking=True)
        traced_drafts = None
        if self.trace is not None:  # the device step overwrites the guesses with the next step's
            torch.cuda.current_stream(self.device).synchronize()
            traced_drafts = {s: self.drafts[s, : int(np_num_drafts[s])].tolist() for s in active}
        self._run_device_step()
        self.h_step_out[rb].copy_(self.step_out, non_blocking=True)
        event = self._read_back_events[rb]
        event.record()
        self._last_rb = rb
        if deferred is not None:
            allocator.take_free([slots[s] for s in deferred[0]], deferred[1], deferred[2])
        return _Launched(active, act, traced_drafts, rb, gb, event)

    def _may_run_ahead(self, act: np.ndarray) -> bool:
        """Whether the next step can be launched before this one's bookkeeping: nothing
        but this step's own outputs decides it, no slot finishes in this step, and the
        free list holds the blocks the next step grows into (a pool that runs out raises
        at the next call, after this step's tokens are appended)."""
        if (not self.run_ahead or self.proposer is not None or self.trace is not None or not self._fifo_blocks
                or self.graph is None or self.graph_sampled != self.any_sampled or len(self._stop_ids) > 64):
            return False
        out, num_out = self.np_out, self.np_num_out
        if not self.graph_allowed(self.np_len + num_out * act):  # the next step would run eagerly
            return False
        if ((self.np_gen + num_out * act >= self.np_max_new) & act).any():
            return False
        if self._stop_ids:
            hon = self.np_honours_stop & act
            if hon.any():
                rows = np.arange(out.shape[1])[None, :] < num_out[:, None]
                if (np.isin(out, self._stop_ids) & rows & hon[:, None]).any():
                    return False
        *_, blocks = host_step.plan_growth(self.np_len + num_out * act, self.np_num_drafts_next, self.np_owned, act,
                                           self.block_size)
        return blocks <= self.allocator.num_free_blocks

    def _maybe_launch_deep(self) -> None:
        """With one step in flight, launch the step after it now over the slots active on
        the host, its blocks reserved for the most the running step can emit plus the
        most guesses the next can make; the device proposes those guesses at the end of
        the running step.  A slot that finishes in the running step (its length limit or
        a stop token) is still run by the launched step, whose outputs for it are dropped
        when it completes.  The host mirrors are at the running step's start."""
        if (len(self._inflight) != 1 or not self.run_ahead or self.proposer is not None or self.trace is not None
                or not self._fifo_blocks or self.graph is None or self.graph_sampled != self.any_sampled):
            return
        running = self._inflight[0]
        act = self.np_active.copy()
        if not act.any():
            return
        guesses = self._read_back_views[running.gb][1][2]  # the running step's guess counts
        most = (guesses + 1) * act  # the most tokens it can emit per slot
        lengths = self.np_len + most
        if not self.graph_allowed(lengths):
            return
        # its guesses: at most k, and never past the sequence's last position (prompt +
        # max_new - 1 tokens hold keys), as the exact count min(k, max_new - gen - 1) is
        last = self.np_len - self.np_gen + self.np_max_new - 1
        drafts = (np.clip(last - lengths, 0, self.k) * act).astype(np.int32)
        *_, blocks = host_step.plan_growth(lengths, drafts, self.np_owned, act, self.block_size)
        if blocks > self.allocator.num_free_blocks:
            return
        self._inflight.append(self._launch(bound=(lengths, drafts)))
        self.ahead_launches += 1
        self.deep_launches += 1

    def _complete(self, launched: _Launched, allow_ahead: bool) -> dict[int, StepResult]:
        """The host side of a step whose outputs have been read back.  A slot that
        finished in the step before this one (after this one was launched) is no longer
        active: its outputs here are dropped."""
        active, act, traced_drafts = launched.active, launched.act, launched.traced_drafts
        if not np.array_equal(act, act & self.np_active):
            act = act & self.np_active
            active = [s for s in active if act[s]]
        self._bind_read_back(launched.rb, launched.gb)
        slots = self.slots
        np_num_drafts = self.np_num_drafts
        ngram = self.proposer is None
        if self.trace is not None and traced_drafts is not None:  # a step launched before tracing began is not recorded
            self.trace.append({
                s: {
                    "history": list(self.slots[s].token_ids),
                    "requested": int(self.np_num_tokens[s]),
                    "drafts": traced_drafts[s],
                    "out": self.h_out[s, : int(self.h_num_out[s])].tolist(),
                    "table": self.allocator.block_table(self.slots[s]),
                }
                for s in active
            })
        if allow_ahead and not self._inflight and act.any() and self._may_run_ahead(act):
            # the mirrors advance now (finish_step below advances copies of the old ones);
            # this step's outputs stay in their read-back buffer, which the next steps do
            # not write; its guess counts are in the buffer the next step reads back into
            out, num_out = self.np_out, self.np_num_out
            guesses = np_num_drafts.copy()
            lengths, generated, steps = self.np_len.copy(), self.np_gen.copy(), self.np_steps.copy()
            emitted = num_out * act
            self.np_len += emitted
            self.np_gen += emitted
            self.np_steps += act
            self._drafts_ready = True
            self._inflight.append(self._launch())
            self.ahead_launches += 1
            self._maybe_launch_deep()
            results, finishing = host_step.finish_step(
                active, slots, out, num_out, guesses, act, lengths, generated, steps, self.np_max_new,
                self.np_honours_stop, self._stop_ids, StepResult, None,
            )
            assert not finishing
            return results
        # the mirrors advance by the emitted counts and every slot that cannot finish this
        # step appends its tokens; slots at their length limit or with a stop token
        # emitted (when they honour stops) finish one token at a time below (a step
        # launched behind this one was launched only if no slot can finish in this one)
        finish = host_step.finish_step if len(self._stop_ids) <= 64 else host_step.finish_step_py
        results, finishing = finish(
            active, slots, self.np_out, self.np_num_out, np_num_drafts, act, self.np_len, self.np_gen,
            self.np_steps, self.np_max_new, self.np_honours_stop, self._stop_ids, StepResult,
            self.allocator.on_tokens_cached if self._track_cached else None,
        )
        for s, tokens in finishing:
            seq = slots[s]
            kept = len(tokens) - 1
            cached = len(seq.token_ids) + kept  # L-1 .. L-1+kept now hold the kept tokens
            results[s] = self._emit(s, seq, tokens, int(np_num_drafts[s]), kept, cached)
        if ngram:  # the counts read back with this step's tokens are the next step's
            self._drafts_ready = True
        if allow_ahead:
            self._maybe_launch_deep()
        return results

    def _emit(self, slot: int, seq: Sequence, tokens: list[int], g: int, kept: int,
              cached: int | None = None) -> StepResult:
        """Append tokens one by one with the finish checks of speculative_generator.py:54-67.

        ``cached`` (verify steps) is the number of positions whose keys/values now hold
        verified tokens; it is recorded, clipped to the tokens actually kept when a stop
        ends the sequence early, and reported to the allocator before a finished
        sequence is released, so its verified blocks stay reusable."""
        params = seq.sampling_params
        reason = None
        stops = self.stop_token_ids
        if (len(seq.token_ids) - seq.num_prompt_tokens + len(tokens) < params.max_new_tokens
                and (params.ignore_eos or stops.isdisjoint(tokens))):
            # no token can end the sequence: the checks below would all pass
            seq.token_ids.extend(tokens)
            emitted = tokens
        else:
            emitted = []
            for token in tokens:
                seq.token_ids.append(token)
                emitted.append(token)
                reason = find_finish_reason(token, seq.num_generated_tokens, params, self.stop_token_ids)
                if reason is not None:
                    break
        if cached is not None:
            seq.num_cached_tokens = min(cached, seq.num_tokens)
            self.allocator.on_tokens_cached(seq)
        if reason is not None:
            self._free_slot(slot)
        return StepResult(emitted, reason, g, kept)

    def release(self, slot: int) -> None:
        """Free a slot.  A result of the slot still waiting for the next step() call is
        dropped with it (the caller has given the slot up)."""
        self.drain()
        for results in self._pending:
            results.pop(slot, None)
        self._pending = deque(r for r in self._pending if r)
        self._free_slot(slot)

    def _free_slot(self, slot: int) -> None:
        """Free a slot whose sequence finished or was given up.  A step already in flight
        still runs the slot (its outputs are dropped when it completes): the slot goes
        inactive on the device after that step, its freed blocks reach later steps only
        in stream order, and its pinned table row is left as it is, since the step's copy
        of the tables may not have run yet (entries past a slot's own blocks are never
        read)."""
        seq = self.slots[slot]
        if seq is None:  # empty, or it finished in the drained step
            return
        self.allocator.free(seq)
        if self.proposer is not None:
            self.proposer.release(slot)
        self.slots[slot] = None
        self._slots_changed()
        self.np_active[slot] = False
        self.np_honours_stop[slot] = False
        self.np_owned[slot] = 0
        # inactive: the fused kernels skip this slot (zero_ on the slice is queued on the
        # stream; assigning a host scalar would copy it synchronously, waiting for every
        # step in flight)
        self.history_len[slot : slot + 1].zero_()
        if not self._inflight:
            self.h_tables[slot].zero_()
        self.np_temp[slot] = 0.0
        self.np_top_p[slot] = 1.0
