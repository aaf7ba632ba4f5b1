"""One request's generation state (ne/engine/sequence_state.py:12-57)."""

from __future__ import annotations

import time
from dataclasses import dataclass, field

from nanoengine_amd.interface import (
    GenerationRequest,
    SamplingParams,
    SamplingStream,
    create_sampling_generator,
)


@dataclass(eq=False)
class Sequence:
    """A request's tokens so far, prompt first, then the generated ones.  The keys and
    values of the first ``num_cached_tokens`` are in the KV pool.  Instances compare by
    identity, so a sequence is found in a list only as the same object."""

    request: GenerationRequest
    sampling_generator: SamplingStream
    token_ids: list[int]
    num_prompt_tokens: int
    num_cached_tokens: int = 0
    arrival_time: float = field(default_factory=time.perf_counter)

    @classmethod
    def from_request(cls, request: GenerationRequest) -> "Sequence":
        return cls(
            request=request,
            sampling_generator=create_sampling_generator(request.sampling_params.seed),
            token_ids=list(request.prompt_token_ids),
            num_prompt_tokens=len(request.prompt_token_ids),
        )

    @property
    def request_id(self) -> str:
        return self.request.request_id

    @property
    def sampling_params(self) -> SamplingParams:
        return self.request.sampling_params

    @property
    def num_tokens(self) -> int:
        return len(self.token_ids)

    @property
    def num_generated_tokens(self) -> int:
        return len(self.token_ids) - self.num_prompt_tokens

    @property
    def num_uncached_tokens(self) -> int:
        return len(self.token_ids) - self.num_cached_tokens
