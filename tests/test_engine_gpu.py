"""The whole batched verify step on the GPU against the oracle's restatement of the
reference path (Qwen3 forward with Int8Linear and an int8 paged KV cache,
ne/models/*.py; verify loop, ne/engine/speculative/*.py).

Shapes are Qwen3-0.6B's per layer (hidden 1024, 16 Q / 8 KV heads, head_dim 128,
MLP 3072) with fewer layers and a smaller vocabulary so the CPU oracle runs in
seconds.  Checked:
  * logits of a verify step: max-abs <= 1e-2 and relative error <= 2e-2 against
    the oracle's score_tokens logits (bf16 model, int8 W + KV);
  * greedy tokens: every emitted token equals the oracle's fp32 argmax wherever
    the oracle's top-2 margin exceeds 2e-2 * the logit scale (teacher-forced);
  * drafts, accepted counts and block tables bit-exact: each recorded step's
    drafts equal oracle.ngram.propose on the same history, the emitted tokens are
    the accepted prefix plus one, and replaying the per-sequence reservations on
    the oracle allocator reproduces every block table.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import model as om
from oracle import ngram as oracle_ngram
from oracle.paging import PagedSlotAllocator as OraclePaged
from oracle.verify import ModelRunner as OracleRunner
from oracle.verify import Sequence as OracleSequence
from nanoengine_amd.config import EngineSettings
from nanoengine_amd.interface import GenerationRequest, SamplingParams
from nanoengine_amd.qwen3 import Qwen3Config, random_state_dict
from nanoengine_amd.runtime import create_verify_engine
from nanoengine_amd.sequence_state import Sequence

pytestmark = pytest.mark.gpu

CFG = Qwen3Config(4096, 1024, 3072, 2, 16, 8, 128, 1e-6, 1e6, True)
OCFG = om.Qwen3Config(4096, 1024, 3072, 2, 16, 8, 128, 1e-6, 1e6, True)


def motif_prompts(n, seed=0):
    g = torch.Generator().manual_seed(seed)
    prompts = []
    for _ in range(n):
        motif = torch.randint(0, 512, (16,), generator=g).tolist()
        prompts.append(motif * 4)
    return prompts


def make_state(norm_ones: bool):
    state = random_state_dict(CFG, seed=0, std=0.02)
    if norm_ones:  # O(1) activations: a sharper test of relative accuracy than 0.02-scale norms
        for name in state:
            if name.endswith("norm.weight") or "layernorm" in name:
                state[name] = torch.ones_like(state[name])
    return state


def oracle_model(state, dtype):
    model = om.Qwen3ForCausalLM(OCFG)
    model.load_state_dict(state)
    model = model.to(dtype).eval()
    om.quantize_linear_layers(model)
    return model


def engine_for(state, num_seqs, kv_int8=True, graphs=False, prefill_rows=None):
    settings = EngineSettings(device="cuda", dtype="bfloat16", kv_cache="paged", scheduler="continuous",
                              quantization="int8", kv_cache_dtype="int8" if kv_int8 else "auto",
                              speculative="ngram", num_speculative_tokens=4, ngram_max_size=3,
                              max_num_seqs=num_seqs, max_model_len=256, kv_cache_memory_mb=64,
                              cuda_graphs=graphs)
    return create_verify_engine(CFG, state, settings, max_prefill_rows=prefill_rows or 64 * num_seqs)


@pytest.mark.parametrize("norm_ones,prefill_rows", [(False, None), (True, None), (False, 24)],
                         ids=["small-norms", "unit-norms", "chunked-prefill-24-rows"])
def test_verify_step_logits_match_oracle(norm_ones, prefill_rows):
    """prefill_rows=24: the 64-token prompts prefill in forwards of at most 24 rows
    (chunks over 24, 48 and 64 keys, cut across sequence boundaries)."""
    state = make_state(norm_ones)
    prompts = motif_prompts(4)
    eng = engine_for(state, 4, prefill_rows=prefill_rows)
    assert prefill_rows is None or eng.model.max_rows == prefill_rows
    params = SamplingParams(max_new_tokens=32, temperature=0.8, seed=1, ignore_eos=True)
    seqs = [Sequence.from_request(GenerationRequest(f"r{i}", p, params)) for i, p in enumerate(prompts)]
    eng.runner.add(seqs)
    eng.runner.trace = []
    eng.runner.step()  # sampled mode leaves the step's logits in runner.logits
    torch.cuda.synchronize()
    ours = eng.runner.logits.float().cpu()
    step = eng.runner.trace[0]
    ref_model = oracle_model(state, torch.bfloat16)
    pool = om.KVCachePool(OCFG, 64 * 16, torch.bfloat16, is_int8=True)
    runner = OracleRunner(ref_model, pool, OraclePaged(64, 16))
    for slot, rec in step.items():
        seq = OracleSequence(f"o{slot}", list(prompts[slot]), 64, 32)
        runner.allocator.reserve(seq.request_id, len(seq.token_ids))
        runner.run_step([seq])  # prefill (its sampled token is replaced by ours below)
        seq.token_ids = list(rec["history"]) + rec["drafts"]
        runner.allocator.reserve(seq.request_id, len(seq.token_ids))
        ref = runner.score_tokens(seq, 1 + len(rec["drafts"])).float()
        got = ours[slot * 5 : slot * 5 + 1 + len(rec["drafts"])]
        # 1e-2 max-abs at the configured N(0, 0.02) scale; with unit norm weights the
        # logits reach ~3-4, where one bf16 ulp is 0.016-0.03 and both sides round,
        # so there the bar is 2e-2 of the logit scale
        bar = 2e-2 * float(ref.abs().max()) if norm_ones else 1e-2
        assert float((got - ref).abs().max()) <= bar
        rel = float((got - ref).norm() / ref.norm())
        assert rel <= 2e-2, f"slot {slot}: relative error {rel:.3e}"


@pytest.mark.parametrize("graphs", [False, True])
def test_greedy_generation_matches_oracle_where_margin_is_clear(graphs):
    state = make_state(norm_ones=True)
    prompts = motif_prompts(6, seed=3)
    eng = engine_for(state, 6, graphs=graphs)
    eng.runner.trace = []
    params = SamplingParams(max_new_tokens=40, ignore_eos=True)
    reqs = [GenerationRequest(f"r{i}", p, params) for i, p in enumerate(prompts)]
    events = eng.batched_generator().generate_all(reqs)
    ref32 = om.Qwen3ForCausalLM(OCFG)
    ref32.load_state_dict(state)
    ref32 = ref32.eval()
    om.quantize_linear_layers(ref32)
    checked = 0
    for i, req in enumerate(reqs):
        toks = [e.token_id for e in events[req.request_id]]
        assert len(toks) == 40 and events[req.request_id][-1].finish_reason == "length"
        full = torch.tensor([prompts[i] + toks])
        with torch.inference_mode():
            logits = ref32.compute_logits(ref32(full))[0]
        scale = float(logits.abs().max())
        for j, tok in enumerate(toks):
            row = logits[len(prompts[i]) - 1 + j]
            top2 = torch.topk(row, 2)
            if float(top2.values[0] - top2.values[1]) > 2e-2 * scale:
                assert tok == int(top2.indices[0]), f"seq {i} token {j}"
                checked += 1
    assert checked > 0
    # drafts, accepted prefixes and block tables bit-exact against the oracle's rules
    oracle_alloc = OraclePaged(eng.allocator._blocks.num_blocks, 16)
    for i, p in enumerate(prompts):  # prefill reservations happen in slot order
        oracle_alloc.reserve(f"r{i}", len(p))
    for step in eng.runner.trace:
        for slot, rec in sorted(step.items()):
            want = oracle_ngram.propose(rec["history"], rec["requested"], 3) if rec["requested"] else []
            assert rec["drafts"] == want
            kept = len(rec["out"]) - 1
            assert rec["out"][:kept] == rec["drafts"][:kept]
            oracle_alloc.reserve(f"r{slot}", len(rec["history"]) + len(rec["drafts"]))
            assert rec["table"] == oracle_alloc.block_table(f"r{slot}")
        for slot, rec in sorted(step.items()):  # finished requests free their blocks
            if len(rec["history"]) + len(rec["out"]) - len(prompts[slot]) >= 40:
                oracle_alloc.free(f"r{slot}")


def test_serial_generator_matches_batched():
    state = make_state(norm_ones=True)
    prompts = motif_prompts(2, seed=5)
    params = SamplingParams(max_new_tokens=24, ignore_eos=True)
    batched = engine_for(state, 2).batched_generator().generate_all(
        [GenerationRequest(f"r{i}", p, params) for i, p in enumerate(prompts)])
    serial_engine = engine_for(state, 1)
    for i, p in enumerate(prompts):
        serial = list(serial_engine.serial_generator().generate(GenerationRequest(f"s{i}", p, params)))
        assert [e.token_id for e in serial] == [e.token_id for e in batched[f"r{i}"]]
    assert serial_engine.allocator.num_reserved_slots == 0  # freed when each request ends


def test_stop_token_ends_a_request_early():
    state = make_state(norm_ones=True)
    prompt = motif_prompts(1, seed=9)[0]
    eng = engine_for(state, 1)
    params = SamplingParams(max_new_tokens=12, ignore_eos=True)
    tokens = [e.token_id for e in eng.serial_generator().generate(GenerationRequest("a", prompt, params))]
    stop = tokens[3]
    eng.runner.stop_token_ids = frozenset({stop})
    events = list(eng.serial_generator().generate(
        GenerationRequest("b", prompt, SamplingParams(max_new_tokens=12))))
    assert events[-1].finish_reason == "stop" and events[-1].token_id == stop
    assert len(events) == tokens.index(stop) + 1


# ------------------------------------------------------------------ prefix cache
def prefix_engine(state, num_seqs, graphs=False):
    settings = EngineSettings(device="cuda", dtype="bfloat16", kv_cache="paged", scheduler="continuous",
                              quantization="int8", kv_cache_dtype="int8", speculative="ngram",
                              num_speculative_tokens=4, ngram_max_size=3, max_num_seqs=num_seqs,
                              max_model_len=256, kv_cache_memory_mb=64, cuda_graphs=graphs,
                              prefix_cache=True)
    return create_verify_engine(CFG, state, settings, max_prefill_rows=64 * num_seqs)


def shared_prefix_prompts(n, seed):
    """A 48-token shared start (three 16-token blocks, motif-repeating so drafts are
    accepted) followed by a distinct suffix per prompt."""
    g = torch.Generator().manual_seed(seed)
    motif = torch.randint(0, 512, (16,), generator=g).tolist()
    prompts = []
    for i in range(n):
        suffix = torch.randint(0, 512, (5 + 3 * i,), generator=g).tolist()
        prompts.append(motif * 3 + suffix + motif[:8])
    return prompts


def pool_bytes(pool, slots):
    idx = torch.tensor(slots, dtype=torch.long, device=pool.key_caches[0].device)
    parts = []
    for i in range(len(pool.key_caches)):
        for t in (pool.key_caches[i], pool.value_caches[i], pool.key_scales[i], pool.value_scales[i]):
            parts.append(t.index_select(0, idx).view(torch.uint8).reshape(-1).cpu())
    return torch.cat(parts)


def test_prefix_hit_verify_logits_match_a_full_prefill_on_the_oracle():
    """Sequences that take 48 cached tokens prefill only their suffix (queries at
    positions 48..p-1 over p keys); their verify-step logits must equal, to the same
    bar as without the cache, the oracle's logits after a full prefill."""
    state = make_state(norm_ones=False)
    prompts = shared_prefix_prompts(4, seed=11)
    eng = prefix_engine(state, 4)
    params = SamplingParams(max_new_tokens=32, temperature=0.8, seed=1, ignore_eos=True)
    seqs = [Sequence.from_request(GenerationRequest(f"r{i}", p, params)) for i, p in enumerate(prompts)]
    eng.runner.add(seqs[:1])  # registers the shared blocks
    eng.runner.add(seqs[1:])
    assert eng.allocator.num_prefix_hit_tokens == 3 * 48
    warm_table = eng.allocator.block_table(seqs[0])
    for seq in seqs[1:]:
        assert eng.allocator.block_table(seq)[:3] == warm_table[:3]
    eng.runner.trace = []
    eng.runner.step()
    torch.cuda.synchronize()
    ours = eng.runner.logits.float().cpu()
    step = eng.runner.trace[0]
    ref_model = oracle_model(state, torch.bfloat16)
    pool = om.KVCachePool(OCFG, 64 * 16, torch.bfloat16, is_int8=True)
    runner = OracleRunner(ref_model, pool, OraclePaged(64, 16))
    for slot, rec in step.items():
        seq = OracleSequence(f"o{slot}", list(prompts[slot]), 64, 32)
        runner.allocator.reserve(seq.request_id, len(seq.token_ids))
        runner.run_step([seq])
        seq.token_ids = list(rec["history"]) + rec["drafts"]
        runner.allocator.reserve(seq.request_id, len(seq.token_ids))
        ref = runner.score_tokens(seq, 1 + len(rec["drafts"])).float()
        got = ours[slot * 5 : slot * 5 + 1 + len(rec["drafts"])]
        assert float((got - ref).abs().max()) <= 1e-2, f"slot {slot}"
        rel = float((got - ref).norm() / ref.norm())
        assert rel <= 2e-2, f"slot {slot}: relative error {rel:.3e}"


@pytest.mark.parametrize("graphs", [False, True])
def test_prefix_cached_speculation_keeps_shared_blocks_and_matches_oracle(graphs):
    """Greedy speculation over shared prefix blocks: the shared blocks' bytes (keys,
    values and scales of every layer) never change while the sharers verify, accept
    and roll back; every emitted token equals the fp32 oracle's argmax where its
    top-2 margin is clear; later requests reuse blocks that finished requests
    registered from verified tokens only."""
    state = make_state(norm_ones=True)
    prompts = shared_prefix_prompts(5, seed=4)
    eng = prefix_engine(state, 5, graphs=graphs)
    params = SamplingParams(max_new_tokens=40, ignore_eos=True)
    seqs = [Sequence.from_request(GenerationRequest(f"r{i}", p, params)) for i, p in enumerate(prompts)]
    emitted = {i: [] for i in range(5)}
    for slot, res in eng.runner.add(seqs[:1]).items():
        emitted[slot] += res.tokens
    shared = eng.allocator.block_table(seqs[0])[:3]
    slots = [b * 16 + o for b in shared for o in range(16)]
    before = pool_bytes(eng.pool, slots)
    for slot, res in eng.runner.add(seqs[1:]).items():
        emitted[slot] += res.tokens
    assert eng.allocator.num_prefix_hit_tokens == 4 * 48
    assert all(eng.allocator.pool.reference_count(b) == 5 for b in shared)
    while eng.runner.active_slots:
        for slot, res in eng.runner.step().items():
            emitted[slot] += res.tokens
    assert torch.equal(pool_bytes(eng.pool, slots), before), "a shared block was written"
    ref32 = om.Qwen3ForCausalLM(OCFG)
    ref32.load_state_dict(state)
    ref32 = ref32.eval()
    om.quantize_linear_layers(ref32)
    checked = 0
    for i in range(5):
        toks = emitted[i]
        assert len(toks) == 40
        with torch.inference_mode():
            logits = ref32.compute_logits(ref32(torch.tensor([prompts[i] + toks])))[0]
        scale = float(logits.abs().max())
        for j, tok in enumerate(toks):
            row = logits[len(prompts[i]) - 1 + j]
            top2 = torch.topk(row, 2)
            if float(top2.values[0] - top2.values[1]) > 2e-2 * scale:
                assert tok == int(top2.indices[0]), f"seq {i} token {j}"
                checked += 1
    assert checked > 0
    # a request repeating a finished sequence's verified history reuses its blocks
    history = prompts[2] + emitted[2]
    again = Sequence.from_request(GenerationRequest("again", history, SamplingParams(max_new_tokens=2)))
    hits = eng.allocator.num_prefix_hit_tokens
    eng.runner.add([again])
    assert eng.allocator.num_prefix_hit_tokens - hits == ((len(history) - 1) // 16) * 16
