"""Draft-model speculation on the GPU (DraftModelProposer, nanoengine_amd/draft.py)
against the oracle (ne/engine/speculative/proposers.py:63-106; the reference's own
checks are nt/engine/test_speculative_decoding.py:75-96).

Target: Qwen3-0.6B per-layer shapes with 2 layers and a 4096-token vocabulary (as in
test_engine_gpu.py); draft: the same shapes with 1 layer and other weights.  Checked:
  * every draft guess equals the oracle draft model's greedy token on the same
    history and earlier guesses wherever the draft's top-2 margin is clear (the draft
    runs in bf16 with int8 W + KV, the oracle in fp32 with int8 W);
  * the emitted tokens equal the target's greedy tokens wherever the target's margin
    is clear (speculation never changes greedy output);
  * with the target's own weights as the draft every clear guess is accepted;
  * sampled requests are refused (the acceptance kernel takes no draft distributions).
"""

from __future__ import annotations

import pytest
import torch

from oracle import draft as odr
from oracle import model as om
from nanoengine_amd.config import EngineSettings
from nanoengine_amd.interface import GenerationRequest, SamplingParams
from nanoengine_amd.qwen3 import Qwen3Config, random_state_dict
from nanoengine_amd.runtime import create_verify_engine
from nanoengine_amd.sequence_state import Sequence

pytestmark = pytest.mark.gpu

CFG = Qwen3Config(4096, 1024, 3072, 2, 16, 8, 128, 1e-6, 1e6, True)
OCFG = om.Qwen3Config(4096, 1024, 3072, 2, 16, 8, 128, 1e-6, 1e6, True)
DCFG = Qwen3Config(4096, 1024, 3072, 1, 16, 8, 128, 1e-6, 1e6, True)
ODCFG = om.Qwen3Config(4096, 1024, 3072, 1, 16, 8, 128, 1e-6, 1e6, True)


def unit_norms(state):
    for name in state:
        if name.endswith("norm.weight") or "layernorm" in name:
            state[name] = torch.ones_like(state[name])
    return state


def prompts(n, seed):
    g = torch.Generator().manual_seed(seed)
    out = []
    for _ in range(n):
        motif = torch.randint(0, 512, (16,), generator=g).tolist()
        out.append(motif * 3 + torch.randint(0, 4096, (8,), generator=g).tolist())
    return out


def engine(state, draft_cfg, draft_state, num_seqs, graphs=False):
    settings = EngineSettings(device="cuda", dtype="bfloat16", kv_cache="paged", scheduler="continuous",
                              quantization="int8", kv_cache_dtype="int8", speculative="draft",
                              num_speculative_tokens=4, max_num_seqs=num_seqs, max_model_len=256,
                              kv_cache_memory_mb=64, cuda_graphs=graphs)
    return create_verify_engine(CFG, state, settings, max_prefill_rows=64 * num_seqs,
                                draft_config=draft_cfg, draft_state_dict=draft_state)


def oracle(cfg, state):
    model = om.Qwen3ForCausalLM(cfg)
    model.load_state_dict(state)
    model = model.eval()
    om.quantize_linear_layers(model)
    return model


def clear(row, scale):
    top2 = torch.topk(row, 2)
    return float(top2.values[0] - top2.values[1]) > 2e-2 * scale


@pytest.mark.parametrize("graphs", [False, True])
def test_draft_guesses_and_output_match_the_oracle(graphs):
    state = unit_norms(random_state_dict(CFG, seed=0, std=0.02))
    dstate = unit_norms(random_state_dict(DCFG, seed=7, std=0.02))
    ps = prompts(4, seed=2)
    eng = engine(state, DCFG, dstate, 4, graphs=graphs)
    eng.runner.trace = []
    params = SamplingParams(max_new_tokens=24, ignore_eos=True)
    reqs = [GenerationRequest(f"r{i}", p, params) for i, p in enumerate(ps)]
    events = eng.batched_generator().generate_all(reqs)
    assert eng.runner.proposer.forwards > 0
    draft32 = oracle(ODCFG, dstate)
    checked_guesses = 0
    for step in eng.runner.trace:
        for slot, rec in step.items():
            assert len(rec["drafts"]) == rec["requested"]
            kept = len(rec["out"]) - 1
            assert rec["out"][:kept] == rec["drafts"][:kept]
            if not rec["drafts"]:
                continue
            rows = odr.draft_logits(draft32, rec["history"], rec["drafts"])
            scale = float(rows.abs().max())
            for j, guess in enumerate(rec["drafts"]):
                if clear(rows[j], scale):
                    assert guess == int(rows[j].argmax()), f"slot {slot} guess {j}"
                    checked_guesses += 1
    assert checked_guesses > 0
    target32 = oracle(OCFG, state)
    checked = 0
    for i, req in enumerate(reqs):
        toks = [e.token_id for e in events[req.request_id]]
        assert len(toks) == 24
        with torch.inference_mode():
            logits = target32.compute_logits(target32(torch.tensor([ps[i] + toks])))[0]
        scale = float(logits.abs().max())
        for j, tok in enumerate(toks):
            row = logits[len(ps[i]) - 1 + j]
            if clear(row, scale):
                assert tok == int(row.argmax()), f"seq {i} token {j}"
                checked += 1
    assert checked > 0


def test_target_as_its_own_draft_accepts_every_clear_guess():
    state = unit_norms(random_state_dict(CFG, seed=0, std=0.02))
    ps = prompts(3, seed=4)
    eng = engine(state, CFG, state, 3)
    eng.runner.trace = []
    params = SamplingParams(max_new_tokens=20, ignore_eos=True)
    eng.batched_generator().generate_all([GenerationRequest(f"r{i}", p, params) for i, p in enumerate(ps)])
    target32 = oracle(OCFG, state)
    proposed = accepted = 0
    for step in eng.runner.trace:
        for rec in step.values():
            kept = len(rec["out"]) - 1
            proposed += len(rec["drafts"])
            accepted += kept
            if kept < len(rec["drafts"]):
                # a rejection may only happen where the target's choice is not clear
                with torch.inference_mode():
                    full = torch.tensor([rec["history"] + rec["drafts"]])
                    logits = target32.compute_logits(target32(full))[0]
                row = logits[len(rec["history"]) - 1 + kept]
                assert not clear(row, float(logits.abs().max()))
    assert proposed > 0 and accepted >= 0.9 * proposed


def test_sampled_requests_are_refused_with_a_draft_model():
    state = random_state_dict(CFG, seed=0, std=0.02)
    dstate = random_state_dict(DCFG, seed=7, std=0.02)
    eng = engine(state, DCFG, dstate, 2)
    params = SamplingParams(max_new_tokens=8, temperature=0.8, seed=1)
    seq = Sequence.from_request(GenerationRequest("s", prompts(1, seed=1)[0], params))
    with pytest.raises(NotImplementedError, match="greedy"):
        eng.runner.add([seq])
