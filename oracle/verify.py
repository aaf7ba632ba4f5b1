"""Verify-step semantics of the reference, restated on the CPU.

  sampling:  ne/engine/sampling.py:11-62
  verifier:  ne/engine/speculative/verifier.py:21-60 (torch.Generator draws, as the reference)
  runner:    ne/engine/generation/model_runner.py:33-80 (run_step / score_tokens)
  loop:      ne/engine/speculative/speculative_generator.py:42-90
"""

from __future__ import annotations

import time
from dataclasses import dataclass, field

import torch

from oracle import ngram
from oracle import paging
from oracle.model import CacheContext, KVCachePool, Qwen3ForCausalLM

GREEDY_TEMPERATURE = 0.0


def create_sampling_generator(seed: int | None) -> torch.Generator:
    """sampling.py:11-18."""
    generator = torch.Generator()
    if seed is None:
        generator.seed()
    else:
        generator.manual_seed(seed)
    return generator


def apply_top_p(probabilities: torch.Tensor, top_p: float) -> torch.Tensor:
    """sampling.py:21-27."""
    sorted_p, sorted_ids = torch.sort(probabilities, descending=True)
    before = torch.cumsum(sorted_p, dim=-1) - sorted_p
    sorted_p[before >= top_p] = 0.0
    kept = torch.zeros_like(probabilities).scatter(-1, sorted_ids, sorted_p)
    return kept / kept.sum(dim=-1, keepdim=True)


def compute_token_probabilities(logits: torch.Tensor, temperature: float, top_p: float = 1.0):
    """sampling.py:30-38."""
    if temperature == GREEDY_TEMPERATURE:
        return torch.nn.functional.one_hot(torch.argmax(logits, dim=-1), logits.shape[-1]).float()
    probabilities = torch.softmax(logits.float() / temperature, dim=-1)
    if top_p < 1.0:
        probabilities = apply_top_p(probabilities, top_p)
    return probabilities


def sample_from_probabilities(probabilities: torch.Tensor, generator: torch.Generator) -> int:
    """sampling.py:41-42."""
    return int(torch.multinomial(probabilities, 1, generator=generator).item())


def pick_token(probabilities, temperature, generator) -> int:
    """verifier.py:21-24."""
    if temperature == GREEDY_TEMPERATURE:
        return int(torch.argmax(probabilities).item())
    return sample_from_probabilities(probabilities, generator)


def verify_proposal(guesses: list[int], draft_probabilities: torch.Tensor | None,
                    target_logits: torch.Tensor, temperature: float, top_p: float,
                    generator: torch.Generator) -> list[int]:
    """verifier.py:27-60."""
    target = compute_token_probabilities(target_logits, temperature, top_p)
    vocab = target.shape[-1]
    kept: list[int] = []
    for index, guess in enumerate(guesses):
        if draft_probabilities is None:
            draft = torch.nn.functional.one_hot(torch.tensor(guess), vocab).float()
        else:
            draft = draft_probabilities[index].float()
        acceptance = (target[index, guess] / draft[guess].clamp(min=1e-12)).clamp(max=1.0).item()
        if acceptance >= 1.0 or (
            acceptance > 0.0 and torch.rand((), generator=generator).item() < acceptance
        ):
            kept.append(guess)
            continue
        residual = (target[index] - draft).clamp(min=0.0)
        if residual.sum() <= 0:
            residual = target[index]
        residual = residual / residual.sum()
        return [*kept, pick_token(residual, temperature, generator)]
    return [*kept, pick_token(target[len(guesses)], temperature, generator)]


def find_finish_reason(token_id: int, num_generated: int, max_new_tokens: int, ignore_eos: bool,
                       stop_token_ids: frozenset[int]) -> str | None:
    """sampling.py:54-62."""
    if not ignore_eos and token_id in stop_token_ids:
        return "stop"
    if num_generated >= max_new_tokens:
        return "length"
    return None


@dataclass
class Sequence:
    """sequence_state.py:12-57 (the fields the verify step touches)."""

    request_id: str
    token_ids: list[int]
    num_prompt_tokens: int
    max_new_tokens: int
    temperature: float = 0.0
    top_p: float = 1.0
    ignore_eos: bool = True
    seed: int | None = 0
    num_cached_tokens: int = 0
    generator: torch.Generator = field(default=None)

    def __post_init__(self) -> None:
        if self.generator is None:
            self.generator = create_sampling_generator(self.seed)

    @property
    def num_generated(self) -> int:
        return len(self.token_ids) - self.num_prompt_tokens


class ModelRunner:
    """model_runner.py:14-80 with a KV pool and an allocator keyed by request id."""

    def __init__(self, model: Qwen3ForCausalLM, pool: KVCachePool, allocator) -> None:
        self.model = model
        self.pool = pool
        self.allocator = allocator

    def _inputs(self, sequences: list[Sequence], counts: list[int]):
        step = paging.build_step_inputs(
            [s.token_ids for s in sequences], [s.num_cached_tokens for s in sequences], counts,
            lambda c: self.allocator.build_context_slots([s.request_id for s in sequences], c),
            self.pool.scratch_slot,
        )
        context = CacheContext(step.positions, step.slot_mapping, step.context_slots,
                               step.attention_mask, self.pool.key_caches, self.pool.value_caches,
                               self.pool.key_scales, self.pool.value_scales)
        return step, context

    @torch.inference_mode()
    def run_step(self, sequences: list[Sequence]) -> list[int]:
        """model_runner.py:33-50 (eager path), greedy or sampled per sequence."""
        counts = [len(s.token_ids) - s.num_cached_tokens for s in sequences]
        step, context = self._inputs(sequences, counts)
        hidden = self.model(step.token_ids, context)
        rows = torch.arange(len(sequences))
        logits = self.model.compute_logits(hidden[rows, step.last_token_indices])
        tokens = torch.argmax(logits, dim=-1).tolist()
        for row, s in enumerate(sequences):
            if s.temperature != GREEDY_TEMPERATURE:
                probs = compute_token_probabilities(logits[row], s.temperature, s.top_p)
                tokens[row] = sample_from_probabilities(probs, s.generator)
        for s, c in zip(sequences, counts, strict=True):
            s.num_cached_tokens += c
        return tokens

    @torch.inference_mode()
    def score_tokens(self, sequence: Sequence, token_count: int) -> torch.Tensor:
        """model_runner.py:52-62: logits after each of the next ``token_count`` tokens."""
        step, context = self._inputs([sequence], [token_count])
        hidden = self.model(step.token_ids, context)
        sequence.num_cached_tokens += token_count
        return self.model.compute_logits(hidden[0, :token_count])


@dataclass
class SpeculativeStats:
    proposed: int = 0
    accepted: int = 0
    steps: int = 0
    step_seconds: list[float] = field(default_factory=list)
    accepted_per_step: list[int] = field(default_factory=list)
    finish_reason: str | None = None


def generate_speculative(runner: ModelRunner, sequence: Sequence, k: int, max_ngram: int,
                         stop_token_ids: frozenset[int] = frozenset(),
                         stats: SpeculativeStats | None = None) -> list[int]:
    """speculative_generator.py:42-85: prefill, then verify steps until a finish reason."""
    stats = stats if stats is not None else SpeculativeStats()
    runner.allocator.reserve(sequence.request_id, len(sequence.token_ids))
    new_tokens = runner.run_step([sequence])
    emitted: list[int] = []
    while True:
        for token in new_tokens:
            sequence.token_ids.append(token)
            emitted.append(token)
            reason = find_finish_reason(token, sequence.num_generated, sequence.max_new_tokens,
                                        sequence.ignore_eos, stop_token_ids)
            if reason is not None:
                runner.allocator.free(sequence.request_id)
                stats.finish_reason = reason
                return emitted
        started = time.perf_counter()
        g = ngram.num_guesses(sequence.max_new_tokens, sequence.num_generated, k)
        guesses = ngram.propose(sequence.token_ids, g, max_ngram) if g else []
        length_before = len(sequence.token_ids)
        sequence.token_ids.extend(guesses)
        runner.allocator.reserve(sequence.request_id, len(sequence.token_ids))
        logits = runner.score_tokens(sequence, 1 + len(guesses))
        new_tokens = verify_proposal(guesses, None, logits, sequence.temperature, sequence.top_p,
                                     sequence.generator)
        kept = len(new_tokens) - 1
        del sequence.token_ids[length_before:]
        sequence.num_cached_tokens = length_before + kept
        stats.proposed += len(guesses)
        stats.accepted += kept
        stats.steps += 1
        stats.accepted_per_step.append(kept)
        stats.step_seconds.append(time.perf_counter() - started)
