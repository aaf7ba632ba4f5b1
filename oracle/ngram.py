"""n-gram prompt lookup, restating NgramProposer.propose
(ne/engine/speculative/proposers.py:39-57) and its use by the speculative loop
(ne/engine/speculative/speculative_generator.py:71-73)."""

from __future__ import annotations

import numpy as np


def propose(token_ids: list[int], num_tokens: int, max_ngram: int, min_ngram: int = 1) -> list[int]:
    """proposers.py:44-57: longest recent n-gram seen before -> the tokens that followed it."""
    for ngram_size in range(max_ngram, min_ngram - 1, -1):
        if len(token_ids) <= ngram_size:
            continue
        suffix = token_ids[-ngram_size:]
        for start in range(len(token_ids) - ngram_size - 1, -1, -1):
            if token_ids[start : start + ngram_size] == suffix:
                follow_start = start + ngram_size
                guesses = token_ids[follow_start : follow_start + num_tokens]
                if guesses:
                    return guesses
    return []


def num_guesses(max_new_tokens: int, num_generated: int, k: int) -> int:
    """speculative_generator.py:71-72: never guess past the length limit."""
    return max(0, min(k, max_new_tokens - num_generated - 1))


def propose_batch_numpy(
    history: np.ndarray, lengths: np.ndarray, num_tokens: np.ndarray, max_ngram: int, max_drafts: int,
    min_ngram: int = 1,
) -> tuple[np.ndarray, np.ndarray]:
    """Vectorised form of ``propose`` for long histories (same result, numpy speed).

    Used where the histories are too long for the pure-Python loop; tests check
    it against ``propose`` on random inputs.
    """
    b = history.shape[0]
    drafts = np.zeros((b, max_drafts), dtype=np.int32)
    counts = np.zeros((b,), dtype=np.int32)
    for s in range(b):
        want = min(int(num_tokens[s]), max_drafts)
        if want <= 0:
            continue
        tokens = history[s, : lengths[s]].astype(np.int64)
        length = tokens.shape[0]
        for n in range(max_ngram, min_ngram - 1, -1):
            if length <= n:
                continue
            suffix = tokens[length - n :]
            last_start = length - n - 1
            windows = np.lib.stride_tricks.sliding_window_view(tokens[: last_start + n], n)
            hits = np.nonzero(np.all(windows == suffix, axis=1))[0]
            if hits.size:
                follow = int(hits[-1]) + n
                guess = tokens[follow : follow + want]
                drafts[s, : guess.size] = guess
                counts[s] = guess.size
                break
    return drafts, counts
