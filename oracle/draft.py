"""Draft-model proposals, restating DraftModelProposer.propose for greedy requests
(ne/engine/speculative/proposers.py:63-106).

TEST INFRASTRUCTURE ONLY (see the package header): the GPU tests compare the HIP
``DraftModelProposer`` with this on the same draft weights.

The reference keeps a KV cache per draft and rolls it back to the common prefix of
its tokens and the target's (``_sync_draft``, :95-106); that reuse changes no guess.
Guess j is the draft model's greedy next token after the target's tokens and
guesses 0..j-1, which is what ``propose`` computes here with full forwards.

Pinned by tests/test_oracle_pins.py: the guesses equal a step-by-step greedy decode
of the same model through the oracle's cached ``ModelRunner`` path (a separate code
path: paged KV cache, one scored token per step), and a proposal of n tokens is the
first n tokens of a longer one.
"""

from __future__ import annotations

import torch

from oracle.model import Qwen3ForCausalLM


@torch.inference_mode()
def propose(draft_model: Qwen3ForCausalLM, token_ids: list[int], num_tokens: int) -> list[int]:
    """proposers.py:70-88 with GREEDY_TEMPERATURE: argmax of the last row, appended."""
    tokens = list(token_ids)
    guesses: list[int] = []
    for _ in range(num_tokens):
        logits = draft_model.compute_logits(draft_model(torch.tensor([tokens])))[0, -1]
        guess = int(torch.argmax(logits))
        tokens.append(guess)
        guesses.append(guess)
    return guesses


@torch.inference_mode()
def draft_logits(draft_model: Qwen3ForCausalLM, token_ids: list[int], guesses: list[int]) -> torch.Tensor:
    """Logits the draft saw for each guess, teacher-forced on ``guesses``: row j is the
    distribution guess j was taken from (``[len(guesses), vocab]``)."""
    full = torch.tensor([list(token_ids) + list(guesses)])
    logits = draft_model.compute_logits(draft_model(full))[0]
    n = len(token_ids)
    return logits[n - 1 : n - 1 + len(guesses)]
