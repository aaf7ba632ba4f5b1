"""Speculative decoding on the HIP path, behind the reference's interfaces.

* ``NgramProposer.propose(sequence, num_tokens) -> Proposal`` and ``release``
  (ne/engine/speculative/proposers.py:24-60) run the device n-gram kernel.
* ``verify_proposal(proposal, target_logits, params, generator)``
  (ne/engine/speculative/verifier.py:27-60) runs the fused acceptance kernel on
  device logits ``[len(guesses) + 1, vocab]``.
* ``SpeculativeGenerator`` (ne/engine/speculative/speculative_generator.py:21-90)
  serves one request at a time; ``BatchedSpeculativeGenerator`` serves many at
  once on the same ``VerifyRunner`` (one verify step covers every sequence).
"""

from __future__ import annotations

from collections.abc import Iterator
from dataclasses import dataclass

import torch

from nanoengine_amd import kernels
from nanoengine_amd.interface import (
    GREEDY_TEMPERATURE,
    GenerationRequest,
    SamplingParams,
    SamplingStream,
    TokenEvent,
)
from nanoengine_amd.metrics import EngineMetrics
from nanoengine_amd.runner import StepResult, VerifyRunner
from nanoengine_amd.sequence_state import Sequence


@dataclass(frozen=True)
class Proposal:
    token_ids: list[int]
    # [len(token_ids), vocab] distributions the guesses were drawn from (a sampled draft
    # model); None: deterministic guesses (n-gram)
    probabilities: torch.Tensor | None = None


class NgramProposer:
    """Prompt lookup on the device (proposers.py:39-60)."""

    def __init__(self, max_ngram: int, min_ngram: int = 1, device: torch.device | None = None) -> None:
        self._max_ngram = max_ngram
        self._min_ngram = min_ngram
        self._device = device or torch.device("cuda", torch.cuda.current_device())

    def propose(self, sequence: Sequence, num_tokens: int) -> Proposal:
        if num_tokens <= 0:
            return Proposal([])
        tokens = sequence.token_ids
        history = torch.tensor([tokens if tokens else [0]], dtype=torch.int32, device=self._device)
        drafts, count = kernels.ngram_propose(
            history, torch.tensor([len(tokens)], dtype=torch.int32, device=self._device),
            torch.tensor([num_tokens], dtype=torch.int32, device=self._device), self._max_ngram,
            num_tokens, min_ngram=self._min_ngram,
        )
        n = int(count.cpu()[0])
        return Proposal(drafts.cpu()[0, :n].tolist())

    def release(self, sequence: Sequence) -> None:
        return None


def verify_proposal(proposal: Proposal, target_logits: torch.Tensor, params: SamplingParams,
                    generator: SamplingStream) -> list[int]:
    """Kept guesses plus one target token (verifier.py:27-60) from device logits, with the
    request's temperature and top-p (sampling.py:21-38).

    ``proposal.probabilities`` (a sampled draft) are the fp32 distributions the guesses
    were drawn from; the kernel uses them as given, as the reference does
    (verifier.py:44-45).  Greedy acceptance does not use them."""
    guesses = proposal.token_ids
    g = len(guesses)
    if target_logits.shape[0] != g + 1:
        raise ValueError("target_logits must have one row per guess plus one")
    dev = target_logits.device
    vocab = target_logits.shape[1]
    k = max(g, 1)
    drafts = torch.zeros(1, k, dtype=torch.int32)
    drafts[0, :g] = torch.tensor(guesses, dtype=torch.int32)
    sampled = params.temperature != GREEDY_TEMPERATURE
    draft_probs = None
    if sampled and proposal.probabilities is not None and g > 0:
        draft_probs = proposal.probabilities.to(dev, torch.float32).contiguous()
        if draft_probs.shape != (g, vocab):
            raise ValueError("probabilities must be [len(guesses), vocab]")
    out, n = kernels.accept(
        drafts.to(dev), torch.tensor([g], dtype=torch.int32, device=dev),
        torch.zeros(1, dtype=torch.int32, device=dev), vocab,
        logits=target_logits.to(torch.bfloat16).contiguous(), temperature=float(params.temperature),
        top_p=float(params.top_p),
        seeds=torch.tensor([generator.seed], dtype=torch.int64, device=dev),
        steps=torch.tensor([generator.step], dtype=torch.int64, device=dev),
        draft_probs=draft_probs,
        draft_row_start=torch.zeros(1, dtype=torch.int32, device=dev) if draft_probs is not None else None,
    )
    generator.step += 1
    count = int(n.cpu()[0])
    return out.cpu()[0, :count].tolist()


class SpeculativeGenerator:
    """One request at a time (speculative_generator.py:21-90) on a one-slot VerifyRunner."""

    def __init__(self, runner: VerifyRunner, metrics: EngineMetrics | None = None) -> None:
        self._runner = runner
        self._metrics = metrics

    @property
    def vocab_size(self) -> int:
        return self._runner.model.config.vocab_size

    def generate(self, request: GenerationRequest) -> Iterator[TokenEvent]:
        sequence = Sequence.from_request(request)
        ((slot, result),) = self._runner.add([sequence]).items()
        try:
            while True:
                for i, token in enumerate(result.tokens):
                    last = i == len(result.tokens) - 1
                    finished = last and result.finish_reason is not None
                    yield TokenEvent(request.request_id, token, finished,
                                     result.finish_reason if finished else None)
                if result.finish_reason is not None:
                    return
                result = self._runner.step()[slot]
                record_acceptance(self._metrics, result)
        finally:
            self._runner.release(slot)


class BatchedSpeculativeGenerator:
    """Many requests on one VerifyRunner: every verify step covers all of them."""

    def __init__(self, runner: VerifyRunner, metrics: EngineMetrics | None = None) -> None:
        self._runner = runner
        self._metrics = metrics

    def generate_all(self, requests: list[GenerationRequest]) -> dict[str, list[TokenEvent]]:
        sequences = [Sequence.from_request(r) for r in requests]
        events: dict[str, list[TokenEvent]] = {r.request_id: [] for r in requests}
        pending = list(zip(requests, sequences, strict=True))
        slot_request: dict[int, GenerationRequest] = {}
        while pending or self._runner.active_slots or self._runner.pending:
            free = self._runner.free_slots()
            if pending and free:
                batch = pending[: len(free)]
                pending = pending[len(free):]
                results = self._runner.add([s for _, s in batch])
                for (req, _), slot in zip(batch, sorted(results), strict=True):
                    slot_request[slot] = req
                self._record(results, slot_request, events)
                if self._metrics is not None:  # batch_engine_loop.py:176
                    self._metrics.prefix_cache_hit_tokens.set(self._runner.allocator.num_prefix_hit_tokens)
                continue
            results = self._runner.step()
            for result in results.values():
                record_acceptance(self._metrics, result)
            self._record(results, slot_request, events)
        return events

    @staticmethod
    def _record(results: dict[int, StepResult], slot_request, events) -> None:
        for slot, result in results.items():
            req = slot_request[slot]
            for i, token in enumerate(result.tokens):
                finished = i == len(result.tokens) - 1 and result.finish_reason is not None
                events[req.request_id].append(
                    TokenEvent(req.request_id, token, finished, result.finish_reason if finished else None))


def record_acceptance(metrics: EngineMetrics | None, result: StepResult) -> None:
    """speculative_generator.py:87-90."""
    if metrics is not None:
        metrics.speculative_proposed_tokens.inc(result.num_guesses)
        metrics.speculative_accepted_tokens.inc(result.num_kept)
