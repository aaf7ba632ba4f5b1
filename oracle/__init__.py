"""CPU oracle for nanoengine's speculative-decoding verify step.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import, call, link or run anything in
this package, and only to check results against (or as the timed CPU baseline).  The
product path (``inference-engine-from-scratch_amd/``) never imports it.

Each module restates one piece of the reference (citations are relative to the
reference tree, ``ne/`` = ``nanoengine/src/nanoengine/``) in plain Python,
numpy, C (``csrc/accept_oracle.c``) or torch on the CPU:

  ngram.py      NgramProposer.propose             ne/engine/speculative/proposers.py:39-57
  draft.py      DraftModelProposer.propose        ne/engine/speculative/proposers.py:63-106
                (greedy guesses)
  paging.py     block / paged / contiguous slot   ne/engine/memory/*.py, batch_builder.py
                allocators, step inputs, masks
  prefix_cache.py  hash-chained block keys,       ne/engine/memory/prefix_cache.py:21-158
                refcounted LRU block pool, prefix
                caching slot allocator
  quant.py      quantize_vectors, Int8Linear      ne/models/int8_quantization.py:30-73
  attention.py  cached GQA attention              ne/models/attention_context.py:32-109
  model.py      Qwen3 forward, logits, init       ne/models/qwen3.py:13-203
  verify.py     verify_proposal (reference        ne/engine/speculative/verifier.py:21-60,
                semantics) and the serial          ne/engine/sampling.py:11-62,
                speculative loop                   ne/engine/speculative/speculative_generator.py
  accept.py     acceptance under the library's
                explicit-uniform contract (greedy
                in numpy; sampled via the C oracle)

How each function is pinned (so a plausible mistake fails a check) is listed
in ``tests/test_oracle_pins.py``: the reference tests' known-answer vectors
(``tests/golden/reference_kats.json``), closed forms, brute force on tiny
inputs, fp64 textbook restatements and an independent third-party Qwen3
implementation (Hugging Face transformers) for the dense forward.
"""
