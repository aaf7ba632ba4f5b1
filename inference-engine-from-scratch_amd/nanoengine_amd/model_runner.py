"""One model step over a batch of sequences, in the reference's ModelRunner form.

Counterparts of ne/engine/generation/batch_builder.py:15-65 (``build_step_inputs``) and
ne/engine/generation/model_runner.py:14-80 (``ModelRunner.run_step`` / ``score_tokens``)
on the HIP forward (``Qwen3VerifyModel``).  The batched speculative loop does not come
through here: ``VerifyRunner`` packs its steps on the device.  This is the per-call seam
for callers of the reference's API, e.g. a speculative generator that scores one
sequence's guesses with ``score_tokens``.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from nanoengine_amd import kernels
from nanoengine_amd.attention_context import AttentionContext, build_attention_mask
from nanoengine_amd.interface import GREEDY_TEMPERATURE
from nanoengine_amd.qwen3 import AttentionBatch, Qwen3VerifyModel

PADDING_TOKEN_ID = 0


@dataclass(frozen=True)
class StepInputs:
    token_ids: torch.Tensor  # [b, q]
    context: AttentionContext
    last_token_indices: torch.Tensor  # [b] index of each sequence's last real token in q


def build_step_inputs(sequences: list, allocator, pool, device: torch.device,
                      token_counts: list[int] | None = None) -> StepInputs:
    """Each sequence brings its next ``token_counts[i]`` uncached tokens (default: all of
    them), padded to the longest; padding rows write to the pool's scratch slot.  The
    context also carries the block tables, real-row counts and context lengths the paged
    kernels read.  KV memory for the new tokens must already be reserved."""
    counts = token_counts or [s.num_uncached_tokens for s in sequences]
    ends = [s.num_cached_tokens + n for s, n in zip(sequences, counts, strict=True)]
    q = max(counts)
    c = max(ends)
    token_rows, position_rows = [], []
    for s, end in zip(sequences, ends, strict=True):
        start = s.num_cached_tokens
        pad = [PADDING_TOKEN_ID] * (q - (end - start))
        token_rows.append(s.token_ids[start:end] + pad)
        position_rows.append(list(range(start, end)) + pad)
    token_ids = torch.tensor(token_rows, device=device)
    positions = torch.tensor(position_rows, device=device)
    n = torch.tensor(counts, device=device)
    is_real = torch.arange(q, device=device)[None, :] < n[:, None]
    context_slots = allocator.build_context_slots(sequences, c)
    slot_mapping = context_slots.gather(1, positions).masked_fill(~is_real, pool.scratch_slot)
    context_lengths = torch.tensor(ends, device=device)
    blocks = math.ceil(c / pool.block_size)
    tables = [(allocator.block_table(s)[:blocks] + [0] * blocks)[:blocks] for s in sequences]
    context = AttentionContext(
        positions=positions,
        slot_mapping=slot_mapping,
        context_slots=context_slots,
        attention_mask=build_attention_mask(positions, context_lengths, c),
        key_caches=pool.key_caches,
        value_caches=pool.value_caches,
        key_scales=pool.key_scales,
        value_scales=pool.value_scales,
        block_tables=torch.tensor(tables, dtype=torch.int32, device=device),
        block_size=pool.block_size,
        query_lengths=n.to(torch.int32),
        context_lengths=context_lengths.to(torch.int32),
        max_context_length=c,
    )
    return StepInputs(token_ids=token_ids, context=context, last_token_indices=n - 1)


class ModelRunner:
    """Runs the HIP forward for padded steps of a few sequences (model_runner.py:14-80)."""

    def __init__(self, model: Qwen3VerifyModel, pool, allocator, device: torch.device) -> None:
        self._model = model
        self._pool = pool
        self.allocator = allocator
        self._device = device

    @property
    def vocab_size(self) -> int:
        return self._model.config.vocab_size

    def _forward(self, inputs: StepInputs):
        """The step's real rows packed sequence after sequence, through the model; returns
        the hidden states and each sequence's first row."""
        ctx = inputs.context
        counts = ctx.query_lengths.tolist()
        q = inputs.token_ids.shape[1]
        real = torch.arange(q, device=self._device)[None, :] < ctx.query_lengths[:, None].long()
        tokens = inputs.token_ids[real].to(torch.int32)
        starts = [0]
        for n in counts[:-1]:
            starts.append(starts[-1] + n)
        batch = AttentionBatch(
            positions=ctx.positions[real].to(torch.int32),
            slot_mapping=ctx.slot_mapping[real].to(torch.int32),
            q_start=torch.tensor(starts, dtype=torch.int32, device=self._device),
            q_len=ctx.query_lengths,
            ctx_len=ctx.context_lengths,
            block_tables=ctx.block_tables,
            max_q_len=max(counts),
            max_ctx_len=ctx.max_context_length,
        )
        rows = sum(counts)
        if rows > self._model.max_rows:
            raise ValueError(f"{rows} rows exceed the model's capacity of {self._model.max_rows}; "
                             "pass smaller token_counts (chunked prefill)")
        self._model.ensure_rope(ctx.max_context_length)
        hidden = self._model.forward(rows, tokens, batch, self._pool, workspace=self._model.eager_workspace)
        return hidden, starts, counts

    @torch.inference_mode()
    def score_tokens(self, sequence, token_count: int) -> torch.Tensor:
        """Cache the next ``token_count`` tokens of one sequence and return the logits after
        each of them, ``[token_count, vocab]`` bf16 (model_runner.py:52-62)."""
        inputs = build_step_inputs([sequence], self.allocator, self._pool, self._device, [token_count])
        hidden, _, _ = self._forward(inputs)
        sequence.num_cached_tokens += token_count
        self.allocator.on_tokens_cached(sequence)
        logits, _ = self._model.compute_logits(hidden[:token_count])
        return logits

    @torch.inference_mode()
    def run_step(self, sequences: list, token_counts: list[int] | None = None) -> list[int]:
        """Cache the next ``token_counts`` tokens of each sequence (default: all uncached)
        and pick a token after each one's last (model_runner.py:33-50): the argmax, or for a
        sampled request a draw under the explicit-uniform contract of the acceptance kernel
        at the request's temperature and top-p, advancing its sampling stream."""
        inputs = build_step_inputs(sequences, self.allocator, self._pool, self._device, token_counts)
        hidden, starts, counts = self._forward(inputs)
        last = torch.tensor([s + n - 1 for s, n in zip(starts, counts, strict=True)], device=self._device)
        logits, _ = self._model.compute_logits(hidden[last].contiguous())
        b = len(sequences)
        params = [s.sampling_params for s in sequences]
        sampled = [p.temperature != GREEDY_TEMPERATURE for p in params]
        drafts = torch.zeros((b, 1), dtype=torch.int32, device=self._device)
        no_drafts = torch.zeros((b,), dtype=torch.int32, device=self._device)
        row_start = torch.arange(b, dtype=torch.int32, device=self._device)
        kwargs = {}
        if any(sampled):
            kwargs = dict(
                temperature=torch.tensor([p.temperature for p in params], dtype=torch.float32, device=self._device),
                top_p=torch.tensor([p.top_p for p in params], dtype=torch.float32, device=self._device),
                seeds=torch.tensor([s.sampling_generator.seed for s in sequences], dtype=torch.int64,
                                   device=self._device),
                steps=torch.tensor([s.sampling_generator.step for s in sequences], dtype=torch.int64,
                                   device=self._device),
                any_sampled=True,
            )
        out, _ = kernels.accept(drafts, no_drafts, row_start, self.vocab_size, logits=logits, **kwargs)
        tokens = out[:, 0].tolist()
        for s, is_sampled in zip(sequences, sampled, strict=True):
            if is_sampled:
                s.sampling_generator.step += 1
        final_counts = token_counts or counts
        for s, n in zip(sequences, final_counts, strict=True):
            s.num_cached_tokens += n
            self.allocator.on_tokens_cached(s)
        return tokens
