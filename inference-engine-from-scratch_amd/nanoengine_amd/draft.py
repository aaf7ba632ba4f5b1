"""Draft-model proposer for the batched verify step on the HIP kernels.

The reference's ``DraftModelProposer`` (ne/engine/speculative/proposers.py:63-106)
runs a small model of the target's family ``num_tokens`` steps ahead of one
request, with its own KV cache (a one-sequence pool, ne/engine/runtime.py:116-129):

  * ``_sync_draft`` makes the draft's tokens equal the target's and keeps its
    cache only for their common prefix (``num_cached = min(num_cached, common)``);
  * every step reserves the draft's slots, scores its uncached tokens
    (``ModelRunner.score_tokens``), and takes the last row's token as the next
    guess, greedy or sampled (the first step catches up on the tokens the target
    emitted), keeping the distribution it was drawn from for the verifier.

``DraftModelProposer`` here does the same for every slot of a ``VerifyRunner`` at
once: one forward of the draft model per guess position covers all slots that
still need guesses (their uncached tokens packed as rows, chunked to the model's
row capacity), on the same W8A16 projection, paged attention and LM-head kernels
as the target, over its own paged pool and allocator.  The next token of each
slot comes from the acceptance kernel run with no drafts: the argmax of the LM head's
partials when greedy; when sampled, an inverse-CDF draw from the draft row's softmax
under the acceptance kernel's explicit-uniform contract, with the uniform of guess j at
verify step s taken at counter step s + (j + 1) * 2^48 (apart from the verifier's own
uniforms at step s).  The sampled draft's logits stay in ``logits``, row slot * k + j,
where the verify step's acceptance reads them as the draft distributions.
"""

from __future__ import annotations

import math
from typing import NamedTuple

import numpy as np
import torch

from nanoengine_amd import kernels
from nanoengine_amd.memory import KVCachePool, PagedSlotAllocator
from nanoengine_amd.qwen3 import AttentionBatch, Qwen3VerifyModel
from nanoengine_amd.sequence_state import Sequence


class DeviceGuesses(NamedTuple):
    """Guesses left on the device (in the ``device_out`` tensor given to ``propose``):
    ``counts[slot]`` of them per slot.  The draft's host state takes them at its next
    proposal."""

    counts: dict[int, int]


class DraftModelProposer:
    """Draft-model guesses for the slots of a batched verify step."""

    def __init__(self, model: Qwen3VerifyModel, pool: KVCachePool, allocator: PagedSlotAllocator,
                 max_seqs: int, max_tokens: int, device: torch.device, k: int = 1,
                 use_graph: bool = False) -> None:
        self.model = model
        self.pool = pool
        self.allocator = allocator
        self.device = device
        self.block_size = allocator.block_size
        self.max_blocks = math.ceil(max_tokens / self.block_size)
        self.max_seqs = max_seqs
        # per slot: the draft's own Sequence (its tokens and cached count) and block table;
        # the target's length at the slot's last sync (the two token lists agree up to it)
        self.drafts: dict[int, Sequence] = {}
        self.synced: dict[int, int] = {}
        self.tables = np.zeros((max_seqs, self.max_blocks), dtype=np.int32)
        self.owned = np.zeros(max_seqs, dtype=np.int64)
        i32 = dict(dtype=torch.int32, device=device)
        self.out_tokens = torch.zeros((max_seqs, 2), **i32)
        self.num_out = torch.zeros(max_seqs, **i32)
        self.no_drafts = torch.zeros((max_seqs, 1), **i32)
        self.zero_counts = torch.zeros(max_seqs, **i32)
        self.last_rows = torch.arange(max_seqs, **i32)
        self.h_out = torch.zeros((max_seqs, 2), dtype=torch.int32, pin_memory=True)
        self.forwards = 0  # draft forwards run (a count for tests and benchmarks)
        self.device_proposals = 0  # proposals whose guesses stayed on the device
        self.k = k
        # sampled proposals: the draft's logits per (slot, guess), read by the verifier
        self.logits: torch.Tensor | None = None
        self.row_start = torch.arange(max_seqs, **i32) * k
        # each slot's temperature (0: greedy) and top-p for the current proposal
        self.temperatures = np.zeros(max_seqs, dtype=np.float32)
        self.top_ps = np.ones(max_seqs, dtype=np.float32)
        self.sampled = False  # some slot of the current proposal samples
        self.seeds: torch.Tensor | None = None
        self.steps: np.ndarray | None = None
        self.target_len: dict[int, int] = {}  # this proposal's target length per slot
        # greedy guesses after the first: one row per slot, replayed from a HIP graph
        self.use_graph = use_graph
        self.max_tokens = max_tokens
        self._dec: dict[str, torch.Tensor] | None = None
        self._dec_graph: torch.cuda.CUDAGraph | None = None
        # the catch-up forward (guess 0) of greedy slots with at most k + 1 uncached tokens:
        # k + 1 rows per slot, padded, replayed from a HIP graph with its own attention
        # scratch (the decode graph's is sized for one row per slot)
        self._cu: dict[str, torch.Tensor] | None = None
        self._cu_graph: torch.cuda.CUDAGraph | None = None
        self._cu_ws = kernels.AttentionWorkspace()
        # guesses of the last proposal still only on the device: (counts, guess 0 from the
        # catch-up), read back at the next proposal
        self._pending: tuple[dict[int, int], bool] | None = None
        model.ensure_rope(max_tokens)

    # ------------------------------------------------------------------ state
    def _sync(self, slot: int, sequence: Sequence) -> Sequence:
        """proposers.py:95-106: the draft takes the target's tokens, keeping its cache for
        their common prefix."""
        draft = self.drafts.get(slot)
        if draft is None:
            draft = Sequence.from_request(sequence.request)
            self.drafts[slot] = draft
        ids, target = draft.token_ids, sequence.token_ids
        # the target only appends, so the lists agree up to the last sync's length: only
        # the tokens since then (the draft's guesses against the target's new ones) compare
        common = min(self.synced.get(slot, 0), len(ids), len(target))
        stop = min(len(ids), len(target))
        while common < stop and ids[common] == target[common]:
            common += 1
        del ids[common:]
        ids.extend(target[common:])
        draft.num_cached_tokens = min(draft.num_cached_tokens, common)
        self.synced[slot] = len(target)
        return draft

    def _reserve(self, slot: int, draft: Sequence, num_tokens: int) -> None:
        added = self.allocator.reserve(draft, num_tokens)
        if added:
            owned = int(self.owned[slot])
            if owned + len(added) > self.max_blocks:
                raise ValueError(f"draft of slot {slot} needs more than {self.max_blocks} blocks")
            self.tables[slot, owned : owned + len(added)] = added
            self.owned[slot] = owned + len(added)

    def release(self, slot: int) -> None:
        """proposers.py:90-93: the request finished; free the draft's blocks."""
        self._finish_pending()
        draft = self.drafts.pop(slot, None)
        if draft is not None:
            self.allocator.free(draft)
        self.synced.pop(slot, None)
        self.owned[slot] = 0

    # -------------------------------------------------------------- proposals
    def propose(self, sequences: dict[int, Sequence], counts: dict[int, int],
                temperature: float | np.ndarray = 0.0, seeds: torch.Tensor | None = None,
                steps: np.ndarray | None = None, top_p: float | np.ndarray = 1.0,
                device_out: torch.Tensor | None = None) -> dict[int, list[int]] | DeviceGuesses:
        """``counts[slot]`` guesses for each slot (proposers.py:70-88): greedy, or sampled at
        ``temperature`` and ``top_p`` (compute_token_probabilities, sampling.py:30-38) with the
        slots' ``seeds`` (device int64) at verify ``steps`` (host).  ``temperature`` and
        ``top_p`` are one value for every slot or arrays indexed by slot (temperature 0:
        that slot's guesses are the draft's greedy tokens).

        ``device_out`` (int32 [max_seqs, >= k] on the device): when the guesses come from
        the captured graphs they are copied there on the stream and not waited for, and
        the call returns their counts (``DeviceGuesses``); otherwise it returns the guesses."""
        self._finish_pending()
        self.temperatures[:] = np.maximum(np.broadcast_to(np.asarray(temperature, dtype=np.float32),
                                                          self.temperatures.shape), 0.0)
        self.top_ps[:] = np.broadcast_to(np.asarray(top_p, dtype=np.float32), self.top_ps.shape)
        self.sampled = bool(any(self.temperatures[s] > 0.0 for s, n in counts.items() if n > 0))
        if self.sampled:
            if seeds is None or steps is None:
                raise ValueError("sampled draft proposals need seeds and steps")
            if self.logits is None:
                self.logits = torch.zeros((self.max_seqs * self.k, self.model.config.vocab_size),
                                          dtype=torch.bfloat16, device=self.device)
            self.seeds, self.steps = seeds, steps
        want = {s: n for s, n in counts.items() if n > 0}
        if want and max(want.values()) > self.k:
            raise ValueError(f"at most {self.k} guesses per slot")
        guesses: dict[int, list[int]] = {s: [] for s in want}
        self.target_len = {}
        for s in want:
            self._sync(s, sequences[s])
            self.target_len[s] = sequences[s].num_tokens
        if self.use_graph and not self.sampled and want and max(want.values()) > 1:
            if self._catch_up_graphed(sorted(want)):  # guess 0 stays on the device
                self._decode_graphed(want, guesses, first_on_device=True, device_out=device_out)
                if device_out is None:
                    return guesses
                self.device_proposals += 1
                return DeviceGuesses(dict(want))
            for s, token in self._next_tokens(sorted(want)).items():  # catch-up: guess 0
                self.drafts[s].token_ids.append(token)
                guesses[s].append(token)
            self._decode_graphed(want, guesses)
            return guesses
        while True:
            live = [s for s in sorted(want) if len(guesses[s]) < want[s]]
            if not live:
                break
            for s, token in self._next_tokens(live).items():
                self.drafts[s].token_ids.append(token)
                guesses[s].append(token)
        return guesses

    def _next_tokens(self, live: list[int]) -> dict[int, int]:
        """Score every live draft's uncached tokens; return each one's next token."""
        work = []  # (slot, draft, start, end): rows start..end-1, context end
        for s in live:
            draft = self.drafts[s]
            self._reserve(s, draft, draft.num_tokens)
            work.append([s, draft, draft.num_cached_tokens, draft.num_tokens])
        cap = self.model.max_rows
        done: list[int] = []  # slots whose last row has been scored, in output order
        while work:
            pieces, rows = [], 0
            while work and rows < cap:
                s, draft, a, e = work[0]
                n = min(e - a, cap - rows)
                pieces.append((s, draft, a, a + n, e))
                rows += n
                if a + n == e:
                    work.pop(0)
                else:
                    work[0][2] = a + n
            self._forward(pieces, rows, done)
        torch.cuda.current_stream(self.device).synchronize()
        self.h_out.copy_(self.out_tokens)
        return {s: int(self.h_out[i, 0]) for i, s in enumerate(done)}

    # --------------------------------------------------------- graphed catch-up
    def _catch_up_body(self) -> None:
        """k + 1 rows per slot (q_len 0: a pad slot): forward, the last real row of each
        slot gathered, its LM-head argmax partials and the argmax through the acceptance
        kernel."""
        c = self._cu
        n, r = self.max_seqs, self.k + 1
        batch = AttentionBatch(c["positions"], c["slots"], c["q_start"], c["q_len"], c["ctx"], c["tables"], r,
                               self.max_tokens)
        hidden = self.model.forward(n * r, c["tokens"], batch, self.pool, workspace=self._cu_ws)
        torch.index_select(hidden, 0, c["last_rows"], out=c["last"])
        self.model.compute_logits(c["last"], logits=False, argmax=c["partials"])
        kernels.accept(self.no_drafts, self.zero_counts, self.last_rows, self.model.config.vocab_size,
                       argmax_partials=c["partials"], temperature=0.0, out_tokens=c["out"], num_out=c["num_out"])

    def _catch_up_graphed(self, live: list[int]) -> bool:
        """Guess 0 of every live slot into the catch-up's ``out`` on the device, from one
        replay of the captured catch-up forward (the same rows, positions and context as
        the eager one, padded to k + 1 rows per slot); False, with nothing run, when a
        slot has no uncached token or more than k + 1 (a new request's prompt), which the
        eager forward takes."""
        n, r, dev = self.max_seqs, self.k + 1, self.device
        spans = {}
        for s in live:
            draft = self.drafts[s]
            a, e = draft.num_cached_tokens, draft.num_tokens
            if not 1 <= e - a <= r:
                return False
            spans[s] = (a, e)
        if self._cu is None:
            i32 = dict(dtype=torch.int32, device=dev)
            tiles = kernels.lm_head_num_tiles(self.model.config.vocab_size)
            hidden = self.model.config.hidden_size
            self._cu = dict(tokens=torch.zeros(n * r, **i32), positions=torch.zeros(n * r, **i32),
                            slots=torch.zeros(n * r, **i32), q_start=torch.arange(n, **i32) * r,
                            q_len=torch.zeros(n, **i32), ctx=torch.zeros(n, **i32),
                            tables=torch.zeros((n, self.max_blocks), **i32),
                            last_rows=torch.zeros(n, dtype=torch.long, device=dev),
                            last=torch.zeros((n, hidden), dtype=self.model.normed.dtype, device=dev),
                            partials=torch.zeros((n, tiles), dtype=torch.int64, device=dev),
                            out=torch.zeros((n, 2), **i32), num_out=torch.zeros(n, **i32))
            self._cu_rows = torch.zeros((3, n * r), dtype=torch.int32, pin_memory=True)
            self._cu_seq = torch.zeros((2, n), dtype=torch.int32, pin_memory=True)
            self._cu_last = torch.zeros(n, dtype=torch.long, pin_memory=True)
            self._cu_tables = torch.zeros((n, self.max_blocks), dtype=torch.int32, pin_memory=True)
        c = self._cu
        rows, seq, last = self._cu_rows.numpy(), self._cu_seq.numpy(), self._cu_last.numpy()
        rows[0] = 0  # tokens of pads
        rows[1] = 0  # positions of pads
        rows[2] = self.pool.scratch_slot  # pads write the pool's scratch slot
        seq[:] = 0
        last[:] = np.arange(n) * r
        for s, (a, e) in spans.items():
            draft = self.drafts[s]
            self._reserve(s, draft, e)
            pos = np.arange(a, e)
            at = s * r
            rows[0, at : at + e - a] = draft.token_ids[a:e]
            rows[1, at : at + e - a] = pos
            rows[2, at : at + e - a] = self.allocator.slots_for(draft, pos)
            seq[0, s] = e - a
            seq[1, s] = e
            last[s] = at + e - a - 1
        self._cu_tables.numpy()[:] = self.tables
        for i, name in enumerate(("tokens", "positions", "slots")):
            c[name].copy_(self._cu_rows[i], non_blocking=True)
        c["q_len"].copy_(self._cu_seq[0], non_blocking=True)
        c["ctx"].copy_(self._cu_seq[1], non_blocking=True)
        c["last_rows"].copy_(self._cu_last, non_blocking=True)
        c["tables"].copy_(self._cu_tables, non_blocking=True)
        if self._cu_graph is None:
            self._catch_up_body()  # eager once (sizes the scratch and lazily created buffers)
            torch.cuda.current_stream(dev).synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                self._catch_up_body()
            self.model.bind_graph()
            self._cu_ws.frozen = True
            self._cu_graph = graph
        else:
            self._cu_graph.replay()
        self.forwards += 1
        for s, (a, e) in spans.items():
            self.drafts[s].num_cached_tokens = e
        return True

    # ------------------------------------------------------- graphed decode steps
    def _decode_body(self) -> None:
        """One greedy decode row per slot (rows with q_len 0 are pads): forward, LM-head
        argmax partials, the argmax through the acceptance kernel, fed back as the next
        step's tokens."""
        d = self._dec
        n = self.max_seqs
        batch = AttentionBatch(d["positions"], d["slots"], d["q_start"], d["q_len"], d["ctx"], d["tables"], 1,
                               self.max_tokens)
        hidden = self.model.forward(n, d["tokens"], batch, self.pool)
        self.model.compute_logits(hidden, logits=False, argmax=d["partials"])
        kernels.accept(self.no_drafts, self.zero_counts, self.last_rows, self.model.config.vocab_size,
                       argmax_partials=d["partials"], temperature=0.0, out_tokens=d["out"], num_out=d["num_out"])
        d["tokens"].copy_(d["out"][:, 0])

    def _decode_graphed(self, want: dict[int, int], guesses: dict[int, list[int]],
                        first_on_device: bool = False, device_out: torch.Tensor | None = None) -> None:
        """Guesses 1 .. want[s] - 1 of every slot: the metadata of each step is staged on
        the host up front, and each step replays the captured decode row per slot.
        ``first_on_device``: guess 0 is in the catch-up's ``out`` (not yet in ``guesses``);
        it feeds the first decode row there and is read back with the others.
        ``device_out``: every guess is copied there on the stream instead of being read back
        now; the next proposal takes them into the drafts' host state."""
        dev, n, k = self.device, self.max_seqs, self.k
        if self._dec is None:
            i32 = dict(dtype=torch.int32, device=dev)
            tiles = kernels.lm_head_num_tiles(self.model.config.vocab_size)
            self._dec = dict(tokens=torch.zeros(n, **i32), positions=torch.zeros(n, **i32),
                             slots=torch.zeros(n, **i32), q_start=torch.arange(n, **i32),
                             q_len=torch.zeros(n, **i32), ctx=torch.zeros(n, **i32),
                             tables=torch.zeros((n, self.max_blocks), **i32),
                             partials=torch.zeros((n, tiles), dtype=torch.int64, device=dev),
                             out=torch.zeros((n, 2), **i32), num_out=torch.zeros(n, **i32),
                             guesses=torch.zeros((n, k), **i32))
            self._dec_host = torch.zeros((k, 4, n), dtype=torch.int32, pin_memory=True)
            self._dec_tokens = torch.zeros(n, dtype=torch.int32, pin_memory=True)
            self._dec_tables = torch.zeros((n, self.max_blocks), dtype=torch.int32, pin_memory=True)
        d = self._dec
        stage = self._dec_host.numpy()
        stage[:] = 0
        steps = max(want.values())
        toks = self._dec_tokens.numpy()
        toks[:] = 0
        for s, count in want.items():
            draft = self.drafts[s]
            length = self.target_len[s]
            self._reserve(s, draft, length + count)
            if not first_on_device:
                toks[s] = guesses[s][0]
            pos = np.arange(length, length + count - 1)  # guess j reads guess j - 1 at L + j - 1
            slot_ids = self.allocator.slots_for(draft, pos)
            for j in range(1, count):
                stage[j, 0, s] = length + j - 1
                stage[j, 1, s] = slot_ids[j - 1]
                stage[j, 2, s] = 1
                stage[j, 3, s] = length + j
        for j in range(1, steps):  # pads write the pool's scratch slot
            stage[j, 1, stage[j, 2] == 0] = self.pool.scratch_slot
        self._dec_tables.numpy()[:] = self.tables
        d["tables"].copy_(self._dec_tables, non_blocking=True)

        def stage_tokens():
            if first_on_device:
                d["tokens"].copy_(self._cu["out"][:, 0])
            else:
                d["tokens"].copy_(self._dec_tokens, non_blocking=True)

        stage_tokens()
        if first_on_device:
            d["guesses"][:, 0].copy_(self._cu["out"][:, 0])
        for j in range(1, steps):
            for i, name in enumerate(("positions", "slots", "q_len", "ctx")):
                d[name].copy_(self._dec_host[j, i], non_blocking=True)
            if self._dec_graph is None:
                self._decode_body()  # eager once (allocates lazily created workspaces)
                torch.cuda.current_stream(dev).synchronize()
                graph = torch.cuda.CUDAGraph()
                # re-stage this step's tokens: the eager pass already advanced them
                stage_tokens()
                torch.cuda.current_stream(dev).synchronize()
                with torch.cuda.graph(graph):
                    self._decode_body()
                self.model.bind_graph()
                self._dec_graph = graph
            self._dec_graph.replay()
            self.forwards += 1
            d["guesses"][:, j].copy_(d["out"][:, 0])
        if device_out is not None:
            device_out[:, : k].copy_(d["guesses"])
            self._pending = (dict(want), first_on_device)
            return
        torch.cuda.current_stream(dev).synchronize()
        self._take_guesses(d["guesses"].cpu().numpy(), want, first_on_device, guesses)

    def _take_guesses(self, got: np.ndarray, want: dict[int, int], first_on_device: bool,
                      guesses: dict[int, list[int]] | None) -> None:
        """The decoded guesses ``got[slot, j]`` into each draft's tokens (and ``guesses``);
        a slot released since the proposal is skipped."""
        for s, count in want.items():
            draft = self.drafts.get(s)
            if draft is None:
                continue
            for j in range(0 if first_on_device else 1, count):
                draft.token_ids.append(int(got[s, j]))
                if guesses is not None:
                    guesses[s].append(int(got[s, j]))
            draft.num_cached_tokens = self.target_len[s] + count - 1

    def _finish_pending(self) -> None:
        """Take the guesses the last proposal left on the device into the drafts' host
        state (the read-back waits for the work queued before it)."""
        if self._pending is None:
            return
        want, first_on_device = self._pending
        self._pending = None
        self._take_guesses(self._dec["guesses"].cpu().numpy(), want, first_on_device, None)

    def _forward(self, pieces, rows: int, done: list[int]) -> None:
        """One draft forward over packed pieces; the pieces that reach their draft's last
        token get their greedy next token in out_tokens[len(done) ...]."""
        dev = self.device
        tokens, positions, slot_map, q_start, q_len, ctx_len, tables = [], [], [], [], [], [], []
        row = 0
        for s, draft, a, b, e in pieces:
            pos = np.arange(a, b)
            tokens.append(np.asarray(draft.token_ids[a:b], dtype=np.int32))
            positions.append(pos.astype(np.int32))
            slot_map.append(self.allocator.slots_for(draft, pos).astype(np.int32))
            q_start.append(row)
            q_len.append(b - a)
            ctx_len.append(b)
            tables.append(self.tables[s])
            row += b - a
        up = lambda x: torch.from_numpy(np.ascontiguousarray(np.concatenate(x))).to(dev)
        tok, posn, slots = up(tokens), up(positions), up(slot_map)
        qs = torch.tensor(q_start, dtype=torch.int32, device=dev)
        ql = torch.tensor(q_len, dtype=torch.int32, device=dev)
        cl = torch.tensor(ctx_len, dtype=torch.int32, device=dev)
        bt = torch.from_numpy(np.stack(tables)).to(dev)
        batch = AttentionBatch(posn, slots, qs, ql, cl, bt, max(q_len), max(ctx_len))
        self.model.ensure_rope(max(ctx_len))
        hidden = self.model.forward(rows, tok, batch, self.pool, workspace=self.model.eager_workspace)
        self.forwards += 1
        for s, draft, a, b, e in pieces:
            draft.num_cached_tokens = b
        ends = [i for i, (s, draft, a, b, e) in enumerate(pieces) if b == e]
        if not ends:
            return
        last_rows = torch.tensor([q_start[i] + q_len[i] - 1 for i in ends], dtype=torch.long, device=dev)
        last = hidden.index_select(0, last_rows)
        n, o = len(ends), len(done)
        vocab = self.model.config.vocab_size
        if not self.sampled:
            _, partials = self.model.compute_logits(last, logits=False, argmax=True)
            kernels.accept(
                self.no_drafts[:n], self.zero_counts[:n], self.last_rows[:n], vocab, argmax_partials=partials,
                temperature=0.0, out_tokens=self.out_tokens[o : o + n], num_out=self.num_out[o : o + n],
            )
        else:
            slots = [pieces[i][0] for i in ends]
            # guess j of slot s: the draft's row s * k + j (j = tokens past the target's)
            rows = [s * self.k + len(pieces[i][1].token_ids) - self.target_len[s] for i, s in zip(ends, slots)]
            logits, _ = self.model.compute_logits(last, logits=True, argmax=False)
            self.logits.index_copy_(0, torch.tensor(rows, dtype=torch.long, device=dev), logits)
            sel = torch.tensor(slots, dtype=torch.long, device=dev)
            steps = np.array([int(self.steps[s]) + ((r - s * self.k + 1) << 48) for s, r in zip(slots, rows)],
                             dtype=np.int64)
            temps = self.temperatures[slots]  # a greedy slot's row takes its argmax
            kernels.accept(
                self.no_drafts[:n], self.zero_counts[:n], self.last_rows[:n], vocab, logits=logits,
                temperature=torch.from_numpy(temps).to(dev),
                top_p=torch.from_numpy(self.top_ps[slots]).to(dev), any_sampled=bool((temps > 0).any()),
                seeds=self.seeds.index_select(0, sel), steps=torch.from_numpy(steps).to(dev),
                out_tokens=self.out_tokens[o : o + n], num_out=self.num_out[o : o + n],
            )
        done.extend(pieces[i][0] for i in ends)
