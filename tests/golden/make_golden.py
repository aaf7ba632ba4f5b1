"""Write the committed golden fixtures under tests/golden/.

* ``reference_kats.json`` -- the known-answer vectors held by the reference's own
  tests (inputs and expected outputs transcribed as data; the cited test line is
  kept next to each case).
* ``sampled_accept.json`` -- acceptance under the integer-mass contract (one-hot guesses, per-sequence top-p) for a
  small seeded batch, produced by the C oracle (oracle/csrc/accept_oracle.c).

Run from the repository root: ``python tests/golden/make_golden.py``.
"""

from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import accept as oracle_accept  # noqa: E402

HERE = Path(__file__).resolve().parent

REFERENCE_KATS = {
    "ngram": {
        "source": "nanoengine/tests/engine/test_speculative_decoding.py:35-42",
        "max_ngram": 2,
        "num_tokens": 3,
        "cases": [
            {"token_ids": [1, 2, 3, 4, 5, 9, 1, 2], "expected": [3, 4, 5]},
            {"token_ids": [1, 2, 3, 4], "expected": []},
        ],
    },
    "greedy_verify": {
        "source": "nanoengine/tests/engine/test_speculative_decoding.py:45-55",
        "vocab": 6,
        "row_best": [2, 4, 1, 5],
        "low": -10.0,
        "high": 10.0,
        "cases": [
            {"guesses": [2, 4, 1], "expected": [2, 4, 1, 5]},
            {"guesses": [2, 3, 1], "expected": [2, 4]},
        ],
    },
    "rejection_sampling_chi_square": {
        "source": "nanoengine/tests/engine/test_speculative_decoding.py:58-74",
        "target": [0.4, 0.3, 0.15, 0.1, 0.05],
        "draft": [0.05, 0.1, 0.15, 0.3, 0.4],
        "trials": 6000,
        "seed": 7,
        "critical_value": 18.47,
    },
    "int8_round_trip": {
        "source": "nanoengine/tests/engine/test_quantization_and_cuda_graphs.py:46-52",
        "shape": [6, 4, 16],
        "bound": "abs(dequant - x) <= scale / 2 + 1e-6",
    },
    "int8_linear_relative_error": {
        "source": "nanoengine/tests/engine/test_quantization_and_cuda_graphs.py:55-64",
        "in_features": 64,
        "out_features": 32,
        "rows": 5,
        "seed": 0,
        "max_relative_error": 0.02,
    },
    "kv_bytes_per_token": {
        "source": "nanoengine/tests/engine/test_quantization_and_cuda_graphs.py:82-89, "
        "nanoengine/tests/engine/test_kv_cache.py:126-131",
        "int8_fp16": 58240,
        "fp16": 114688,
    },
    "paged_allocator_growth": {
        "source": "nanoengine/tests/engine/test_memory_allocators.py:52-65",
        "num_blocks": 4,
        "block_size": 4,
        "reserve": [4, 5],
        "expected_table": [0, 1],
        "context_length": 6,
        "expected_slots": [[0, 1, 2, 3, 4, 5]],
    },
    "interleaved_tables": {
        "source": "nanoengine/tests/engine/test_kv_cache.py:93-101",
        "num_blocks": 12,
        "block_size": 4,
        "prompts": [[1, 2, 3, 4], [5, 6, 7, 8]],
        "steps": 4,
        "expected_tables": [[0, 2], [1, 3]],
    },
    "rotate_half": {
        "source": "nanoengine/tests/models/test_qwen3_model.py:63-74",
        "input": [1.0, 2.0, 3.0, 4.0],
        "expected": [-3.0, -4.0, 1.0, 2.0],
    },
    "top_p": {
        "source": "nanoengine/tests/engine/test_sampling_and_generation.py:46-52",
        "probabilities": [0.05, 0.6, 0.3, 0.05],
        "top_p": 0.8,
        "expected_nonzero": [1, 2],
    },
    "greedy_argmax": {
        "source": "nanoengine/tests/engine/test_sampling_and_generation.py:18-22",
        "logits": [0.1, 3.0, -1.0, 2.9],
        "expected": 1,
    },
    "contiguous_allocator": {
        "source": "nanoengine/tests/engine/test_memory_allocators.py:34-49",
        "num_regions": 2,
        "region_length": 8,
        "reserve": [["a", 2], ["b", 8]],
        "expected_reserved_slots": 16,
        "refused": [["c", 1], ["a", 9]],
        "free": "a",
        "accepted_after_free": ["c", 1],
        "context": ["b", 3],
        "region_start_multiple": 8,
    },
    "speculative_stop_token": {
        "source": "nanoengine/tests/engine/test_speculative_decoding.py:100-112; prompt "
        "nanoengine/tests/engine/test_batch_engine_loop.py:20 (PROMPTS[0]); settings "
        "test_batch_engine_loop.py:30-39 and nanoengine/src/nanoengine/config.py:55,64-67; "
        "model nanoengine/tests/conftest.py:23-43",
        "model": {"vocab_size": 64, "hidden_size": 32, "intermediate_size": 64, "num_hidden_layers": 2,
                  "num_attention_heads": 4, "num_key_value_heads": 2, "head_dim": 16, "rms_norm_eps": 1e-6,
                  "rope_theta": 10000.0, "seed": 7, "std": 0.5},
        "prompt": [3, 9, 27],
        "max_new_tokens": 12,
        "greedy_reference_new_tokens": 12,
        "stop_token_greedy_index": 3,
        "kv_block_size": 4,
        "num_speculative_tokens": 4,
        "ngram_max_size": 3,
        "expected_finish_reason": "stop",
        "max_events": 4,
    },
}


def make_sampled_case() -> dict:
    rng = np.random.default_rng(20261201)
    vocab, num_seqs, k, temperature = 600, 8, 4, 0.8
    num_drafts = rng.integers(0, k + 1, size=num_seqs)
    row_start = np.concatenate([[0], np.cumsum(num_drafts + 1)[:-1]])
    rows = int((num_drafts + 1).sum())
    logits = (rng.standard_normal((rows, vocab)) * 3).astype(np.float32)
    bits = oracle_accept.bf16_bits(logits)  # truncate to bf16 patterns
    values = oracle_accept.bf16_to_f32(bits)
    drafts = np.zeros((num_seqs, k), dtype=np.int32)
    for s in range(num_seqs):
        for i in range(num_drafts[s]):
            top = int(np.argmax(values[row_start[s] + i]))
            drafts[s, i] = top if rng.random() < 0.6 else int(rng.integers(0, vocab))
    seeds = rng.integers(0, 2**62, size=num_seqs)
    steps = rng.integers(0, 100, size=num_seqs)
    top_p = [1.0 if s % 2 == 0 else 0.9 for s in range(num_seqs)]
    expected = []
    for s in range(num_seqs):
        lo = int(row_start[s])
        expected.append(oracle_accept.sampled_accept_v3(
            bits[lo : lo + num_drafts[s] + 1], drafts[s, : num_drafts[s]].tolist(), temperature, top_p[s],
            int(seeds[s]), int(steps[s])))
    return {
        "contract": "integer-mass contract for one-hot guesses, inference-engine-from-scratch_amd/csrc/accept.hip header",
        "vocab": vocab,
        "temperature": temperature,
        "top_p": top_p,
        "num_drafts": num_drafts.tolist(),
        "row_start": row_start.tolist(),
        "drafts": drafts.tolist(),
        "seeds": [int(x) for x in seeds],
        "steps": [int(x) for x in steps],
        "logit_bits": bits.reshape(-1).tolist(),
        "expected": expected,
    }


def main() -> None:
    (HERE / "reference_kats.json").write_text(json.dumps(REFERENCE_KATS, indent=1) + "\n")
    (HERE / "sampled_accept.json").write_text(json.dumps(make_sampled_case()) + "\n")
    print("wrote", HERE / "reference_kats.json", HERE / "sampled_accept.json")


if __name__ == "__main__":
    main()
