"""Host-side logic of the product package (CPU only): settings, allocator, random
initialisation order, RoPE table, split choices.  No kernel is launched."""

from __future__ import annotations

import json
from pathlib import Path

import pytest
import torch
from hypothesis import given, settings
from hypothesis import strategies as st

from nanoengine_amd import kernels
from nanoengine_amd.config import EngineSettings
from nanoengine_amd.interface import SamplingParams, num_guesses
from nanoengine_amd.memory import OutOfKVMemoryError, PagedSlotAllocator, count_kv_bytes_per_token
from nanoengine_amd.qwen3 import Qwen3Config, pair_rows, quantize_rows, random_state_dict
from oracle import model as om
from oracle import quant as oq

KATS = json.loads((Path(__file__).parent / "golden" / "reference_kats.json").read_text())
CPU = torch.device("cpu")


def test_random_init_matches_the_module_built_reference_order():
    """Drawing every parameter in registration order after the constructors' own draws
    gives the same tensors as building the modules (nt/conftest.py:38-43 pattern)."""
    cfg = Qwen3Config(64, 32, 64, 2, 4, 2, 16, 1e-6, 1e4, True)
    ours = random_state_dict(cfg, seed=7, std=0.5)
    ref = om.build_random_model(om.Qwen3Config(64, 32, 64, 2, 4, 2, 16, 1e-6, 1e4, True), seed=7, std=0.5)
    ref_state = ref.state_dict()
    assert set(ours) == set(ref_state)
    for name, t in ours.items():
        assert torch.equal(t, ref_state[name]), name


def test_rope_table_equals_the_reference_tables_bit_for_bit():
    positions = torch.tensor([[0, 1, 5, 127, 4095, 16999]])
    cos, sin = om.build_rotary_tables(positions, 128, 1e6, torch.bfloat16)
    table = kernels.rope_table(17000, 1e6)
    got = table[positions[0]]
    assert torch.equal(got[:, 0], cos[0, 0, :, :64]) and torch.equal(got[:, 1], sin[0, 0, :, :64])
    assert torch.equal(cos[..., :64], cos[..., 64:])  # dims i and i + 64 share the angle


def test_weight_quantisation_matches_int8_linear_from_linear():
    w = torch.randn(48, 64).to(torch.bfloat16)
    q, s = quantize_rows(w)
    rq, rs = oq.quantize_linear(w)
    assert torch.equal(q, rq) and torch.equal(s, rs)


def test_gate_up_pairing_interleaves_groups_of_16_rows():
    gate = torch.arange(32)[:, None].expand(32, 2)
    up = 100 + torch.arange(32)[:, None].expand(32, 2)
    paired = pair_rows(gate, up)[:, 0].tolist()
    assert paired == list(range(16)) + list(range(100, 116)) + list(range(16, 32)) + list(range(116, 132))


def test_kv_bytes_per_token_reference_kat():
    kat = KATS["kv_bytes_per_token"]
    assert count_kv_bytes_per_token(28, 8, 128, torch.float16, is_int8_cache=True) == kat["int8_fp16"]
    assert count_kv_bytes_per_token(28, 8, 128, torch.float16) == kat["fp16"]


def test_paged_allocator_reference_kat_and_rollback_frees_nothing():
    kat = KATS["paged_allocator_growth"]
    alloc = PagedSlotAllocator(kat["num_blocks"], kat["block_size"], CPU)
    for n in kat["reserve"]:
        alloc.reserve("r", n)
    assert alloc.block_table("r") == kat["expected_table"]
    assert alloc.build_context_slots(["r"], kat["context_length"]).tolist() == kat["expected_slots"]
    # a shorter reservation (a rollback of rejected guesses) keeps every block
    alloc.reserve("r", 1)
    assert alloc.block_table("r") == kat["expected_table"]
    with pytest.raises(OutOfKVMemoryError):
        alloc.reserve("r", 100)


@settings(max_examples=60, deadline=None)
@given(st.lists(st.tuples(st.integers(0, 5), st.integers(0, 40), st.booleans()), max_size=40))
def test_allocator_never_loses_or_shares_a_block(ops):
    """nt/engine/test_memory_allocators.py:68-89: every block is either free or owned by
    exactly one request, whatever the sequence of reserves and frees."""
    alloc = PagedSlotAllocator(16, 4, CPU)
    for rid, n, free in ops:
        name = f"r{rid}"
        if free:
            alloc.free(name)
        else:
            try:
                alloc.reserve(name, n)
            except OutOfKVMemoryError:
                pass
        owned = [b for i in range(6) for b in alloc.block_table(f"r{i}")]
        assert len(owned) == len(set(owned))
        assert len(owned) + alloc.num_free_blocks == 16


def test_settings_select_the_hip_path_and_keep_the_reference_checks():
    ok = EngineSettings(device="cuda", dtype="bfloat16", kv_cache="paged", quantization="int8",
                        kv_cache_dtype="int8", speculative="ngram", scheduler="continuous")
    assert ok.hip_verify_path_error() is None
    assert "dtype" in EngineSettings(device="cuda", kv_cache="paged", quantization="int8",
                                     speculative="ngram").hip_verify_path_error()
    with pytest.raises(ValueError):  # ne/config.py:91-97: speculation without a KV cache
        EngineSettings(speculative="ngram")
    # prefix-cached speculation is accepted (only verified blocks are registered);
    # the draft-model path keeps the reference's refusal
    assert EngineSettings(kv_cache="paged", prefix_cache=True, speculative="ngram").prefix_cache
    with pytest.raises(ValueError):
        EngineSettings(kv_cache="paged", prefix_cache=True, speculative="draft")
    with pytest.raises(ValueError):  # ne/config.py:85-86
        EngineSettings(kv_cache="contiguous", prefix_cache=True)
    env = {"NANOENGINE_DEVICE": "cuda", "NANOENGINE_KV_CACHE": "paged", "NANOENGINE_CUDA_GRAPHS": "true",
           "NANOENGINE_NUM_SPECULATIVE_TOKENS": "8"}
    s = EngineSettings.from_env(env)
    assert s.device == "cuda" and s.cuda_graphs is True and s.num_speculative_tokens == 8


def test_verify_graph_gating_follows_the_reference_bounds():
    """cuda_graph_max_batch / cuda_graph_max_context (ne/config.py:58-61) bound which verify
    steps replay the captured graph, as they bound the reference's decode graphs
    (runtime.py:150-160, cuda_graph_runner.py:106-117): more active sequences than the
    batch bound, or a step context (length + k guess rows) above the context bound, runs
    eagerly; the settings reach the runner through create_verify_engine's arguments."""
    from nanoengine_amd.runner import verify_graph_allowed

    assert verify_graph_allowed(8, 1024, 8, 1024)
    assert not verify_graph_allowed(9, 100, 8, 1024)
    assert not verify_graph_allowed(1, 1025, 8, 1024)
    assert verify_graph_allowed(64, 10**6, None, None)
    assert verify_graph_allowed(0, 0, 8, 1024)
    d = EngineSettings()
    assert (d.cuda_graph_max_batch, d.cuda_graph_max_context) == (8, 1024)  # ne/config.py:59-61
    env = {"NANOENGINE_CUDA_GRAPH_MAX_BATCH": "64", "NANOENGINE_CUDA_GRAPH_MAX_CONTEXT": "4096"}
    s = EngineSettings.from_env(env)
    assert (s.cuda_graph_max_batch, s.cuda_graph_max_context) == (64, 4096)
    for bad in ("cuda_graph_max_batch", "cuda_graph_max_context"):
        with pytest.raises(ValueError):
            EngineSettings(**{bad: 0})
    src = (Path(__file__).parents[1] / "inference-engine-from-scratch_amd" / "nanoengine_amd" / "runtime.py").read_text()
    assert "graph_max_batch=settings.cuda_graph_max_batch" in src
    assert "graph_max_context=settings.cuda_graph_max_context" in src


def test_num_guesses_never_passes_the_length_limit():
    p = SamplingParams(max_new_tokens=128)
    assert [num_guesses(p, n, 4) for n in (0, 124, 126, 127)] == [4, 3, 1, 0]


def test_splitk_split_counts_fill_the_gpu_and_divide_k():
    for rows in (1, 5, 80, 320, 4096):
        for k in (2048, 3072):
            s = kernels.splitk_splits(rows, 1024, k)
            assert s in (1, 2, 3, 4) and k % (128 * s) == 0


def test_requests_longer_than_max_model_len_are_refused():
    """api/routes.py:98-111: prompt + max_tokens above max_model_len, or an empty prompt,
    is refused before admission (the device history rows are sized by max_model_len)."""
    from nanoengine_amd.runner import request_length_error

    assert request_length_error(64, 128, 192) is None
    assert request_length_error(64, 129, 192) == "prompt + max_new_tokens = 193 exceeds max_model_len 192"
    assert request_length_error(0, 4, 192) == "prompt is empty"


def test_attention_workspace_held_by_a_graph_refuses_to_grow():
    """Once a captured graph holds the workspace's address, a larger request raises
    instead of moving the buffer; a request that fits reuses it."""
    ws = kernels.AttentionWorkspace()
    cpu = torch.device("cpu")
    buf = ws.get(cpu, 4096, ("a",))
    ws.frozen = True
    assert ws.get(cpu, 1024, ("b",)) is buf
    with pytest.raises(RuntimeError, match="captured HIP graph"):
        ws.get(cpu, 8192, ("c",))


@settings(max_examples=60, deadline=None)
@given(st.lists(st.lists(st.tuples(st.integers(0, 5), st.integers(1, 40)), max_size=6), max_size=12),
       st.lists(st.integers(0, 5), max_size=12))
def test_peek_then_take_equals_reserving_in_slot_order(steps, frees):
    """The verify step writes a step's new table entries from peek_free and records them
    with take_free while the device runs: tables and free list must end as the
    reference's reserve, called for each growing sequence in slot order, leaves them
    (paged_allocator.py:50-55, block_allocator.py:20-27)."""
    one, two = PagedSlotAllocator(64, 4, CPU), PagedSlotAllocator(64, 4, CPU)
    for i, grows in enumerate(steps):
        targets = {}
        for rid, n in grows:  # one target per sequence, the largest, as a step has
            targets[f"r{rid}"] = max(n, targets.get(f"r{rid}", 0))
        names = sorted(targets)
        counts = [max(0, -(-targets[r] // 4) - two.num_blocks_of(r)) for r in names]
        blocks = two.peek_free(sum(counts))
        if blocks is None:
            continue
        for r in names:
            one.reserve(r, targets[r])
        two.take_free(names, counts, blocks)
        if i < len(frees):
            one.free(f"r{frees[i]}")
            two.free(f"r{frees[i]}")
        for r in (f"r{j}" for j in range(6)):
            assert one.block_table(r) == two.block_table(r)
        assert list(one._blocks._free) == list(two._blocks._free)


def test_stop_ids_set_after_construction_reach_the_step_bookkeeping():
    """The per-step bookkeeping (the C finish_step) matches tokens against the sorted
    tuple behind VerifyRunner.stop_token_ids; assigning the set later updates it."""
    from nanoengine_amd.runner import VerifyRunner

    runner = VerifyRunner.__new__(VerifyRunner)
    runner.stop_token_ids = {7, 3}
    assert runner.stop_token_ids == frozenset({3, 7}) and runner._stop_ids == (3, 7)
    runner.stop_token_ids = frozenset()
    assert runner._stop_ids == ()


@settings(max_examples=60, deadline=None)
@given(st.lists(st.tuples(st.integers(0, 4), st.integers(0, 5), st.booleans()), min_size=1, max_size=12),
       st.integers(0, 2 ** 16))
def test_draft_sync_keeps_the_common_prefix_of_the_draft_and_the_target(steps, seed):
    """DraftModelProposer._sync (proposers.py:95-106), which compares only the tokens since
    the slot's last sync, equals the reference rule on whole lists: the draft takes the
    target's tokens and keeps its cache for their common prefix.  Each round the draft
    appends guesses, the target keeps a prefix of them and appends a token of its own
    (which may repeat the next guess), sometimes without the draft having proposed."""
    import random

    from nanoengine_amd.draft import DraftModelProposer
    from nanoengine_amd.interface import GenerationRequest
    from nanoengine_amd.sequence_state import Sequence

    rng = random.Random(seed)
    proposer = DraftModelProposer.__new__(DraftModelProposer)
    proposer.drafts, proposer.synced = {}, {}
    target = Sequence.from_request(GenerationRequest("r", [rng.randrange(50) for _ in range(6)],
                                                     SamplingParams(max_new_tokens=200)))
    draft_cached = None
    for guesses, kept, proposed in steps:
        before = proposer.drafts.get(0)
        old_ids = list(before.token_ids) if before is not None else None
        old_cached = before.num_cached_tokens if before is not None else 0
        draft = proposer._sync(0, target)
        want_common = 0
        if old_ids is not None:
            for a, b in zip(old_ids, target.token_ids):
                if a != b:
                    break
                want_common += 1
        assert draft.token_ids == target.token_ids and draft.token_ids is not target.token_ids
        assert draft.num_cached_tokens == min(old_cached, want_common)
        # the draft scores its tokens and proposes; the target verifies
        draft.num_cached_tokens = len(draft.token_ids) + (guesses - 1 if guesses and proposed else 0)
        if not proposed:
            guesses = 0
        g = [rng.randrange(50) for _ in range(guesses)]
        draft.token_ids.extend(g)
        keep = min(kept, guesses)
        target.token_ids.extend(g[:keep])
        target.token_ids.append(rng.randrange(50))
