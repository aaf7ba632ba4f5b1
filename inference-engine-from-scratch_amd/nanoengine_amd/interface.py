"""Request and event types (same fields as ne/engine/interface.py:8-39) plus the
sampling helpers of ne/engine/sampling.py that stay on the host."""

from __future__ import annotations

import os
from collections.abc import AsyncIterator
from dataclasses import dataclass
from typing import Protocol

GREEDY_TEMPERATURE = 0.0
FINISH_REASON_STOP = "stop"
FINISH_REASON_LENGTH = "length"


@dataclass(frozen=True)
class SamplingParams:
    max_new_tokens: int
    temperature: float = 0.0
    top_p: float = 1.0
    seed: int | None = None
    ignore_eos: bool = False


@dataclass(frozen=True)
class GenerationRequest:
    request_id: str
    prompt_token_ids: list[int]
    sampling_params: SamplingParams


@dataclass(frozen=True)
class TokenEvent:
    request_id: str
    token_id: int
    is_finished: bool
    finish_reason: str | None


class InferenceEngine(Protocol):
    async def start(self) -> None: ...

    async def stop(self) -> None: ...

    def submit(self, request: GenerationRequest) -> AsyncIterator[TokenEvent]: ...


@dataclass
class SamplingStream:
    """Per-request randomness (the role of create_sampling_generator, sampling.py:11-18).

    Draws are Philox4x32-10 uniforms keyed by ``seed`` at counter ``step``; one
    step is one sampling event of the request (its first token, then each verify
    step), so a fixed seed always gives the same tokens.
    """

    seed: int
    step: int = 0


def create_sampling_generator(seed: int | None) -> SamplingStream:
    if seed is None:
        seed = int.from_bytes(os.urandom(8), "little") & ((1 << 63) - 1)
    return SamplingStream(seed=int(seed) & ((1 << 63) - 1))


def find_finish_reason(token_id: int, num_generated_tokens: int, params: SamplingParams,
                       stop_token_ids: frozenset[int]) -> str | None:
    """sampling.py:54-62: ``stop`` on a stop token unless ignore_eos, ``length`` at the limit."""
    if not params.ignore_eos and token_id in stop_token_ids:
        return FINISH_REASON_STOP
    if num_generated_tokens >= params.max_new_tokens:
        return FINISH_REASON_LENGTH
    return None


def num_guesses(params: SamplingParams, num_generated_tokens: int, k: int) -> int:
    """speculative_generator.py:71-72: never guess past the length limit."""
    return max(0, min(k, params.max_new_tokens - num_generated_tokens - 1))
