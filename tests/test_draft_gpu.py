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
  * sampled guesses are the draws of the contract from the draft's rows, and the
    acceptance with draft distributions equals the C oracle bit for bit.
"""

from __future__ import annotations

import numpy as np
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
                              kv_cache_memory_mb=64, cuda_graphs=graphs,
                              cuda_graph_max_batch=num_seqs, cuda_graph_max_context=262)
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
    # with graphs, the catch-up forwards after the first proposal replay a captured graph
    assert (eng.runner.proposer._cu_graph is not None) == graphs
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


def test_accept_with_draft_rows_matches_the_c_oracle():
    """ne_accept with draft rows (sampled; verifier.py:36-56) bit for bit against the C
    oracle: 48 sequences, 0..4 guesses, draft rows near the target rows (acceptances)
    or independent of them (rejections and residual draws), vocab not a multiple of 256."""
    from oracle import accept as oacc
    from nanoengine_amd import kernels

    torch.manual_seed(5)
    b, k, vocab, temp = 48, 4, 5003, 0.8
    target = torch.randn(b * (k + 1), vocab) * 2
    draft = torch.randn(b * k, vocab) * 2
    near = torch.arange(b) % 2 == 0
    for s in range(b):
        if near[s]:
            draft[s * k : (s + 1) * k] = target[s * (k + 1) : s * (k + 1) + k] + 0.3 * torch.randn(k, vocab)
    t_bf, d_bf = target.bfloat16(), draft.bfloat16()
    counts = torch.arange(b, dtype=torch.int32) % (k + 1)
    drafts = torch.randint(0, vocab, (b, k), dtype=torch.int32)
    for s in range(b):  # some guesses are the draft row's top tokens
        drafts[s, 0] = int(d_bf[s * k].float().argmax())
    seeds = torch.arange(b, dtype=torch.int64) * 7919 + 3
    steps = torch.arange(b, dtype=torch.int64) + 11
    dev = torch.device("cuda")
    out, n = kernels.accept(drafts.to(dev), counts.to(dev), (torch.arange(b, dtype=torch.int32) * (k + 1)).to(dev),
                            vocab, logits=t_bf.to(dev), temperature=temp, seeds=seeds.to(dev), steps=steps.to(dev),
                            draft_logits=d_bf.to(dev), draft_row_start=(torch.arange(b, dtype=torch.int32) * k).to(dev))
    out, n = out.cpu(), n.cpu()
    tb = t_bf.view(torch.int16).numpy().view("uint16")
    db = d_bf.view(torch.int16).numpy().view("uint16")
    rejected = accepted = 0
    for s in range(b):
        g = int(counts[s])
        want = oacc.sampled_accept_draft(tb[s * (k + 1) : s * (k + 1) + g + 1], db[s * k : s * k + max(g, 1)],
                                         drafts[s, :g].tolist(), temp, int(seeds[s]), int(steps[s]))
        got = out[s, : int(n[s])].tolist()
        assert got == want, f"sequence {s}"
        accepted += len(want) - 1
        rejected += g > len(want) - 1
    assert accepted > 0 and rejected > 0


def test_sampled_draft_step_matches_the_c_oracle():
    """One sampled verify step with a draft model: each guess is the draw from its draft
    row at counter step s + (j + 1) * 2^48, and the emitted tokens are the C oracle's
    draft-distribution acceptance on the step's target and draft logits."""
    from oracle import accept as oacc

    state = unit_norms(random_state_dict(CFG, seed=0, std=0.02))
    dstate = unit_norms(random_state_dict(DCFG, seed=7, std=0.02))
    eng = engine(state, DCFG, dstate, 4)
    params = SamplingParams(max_new_tokens=16, temperature=0.8, seed=3, ignore_eos=True)
    seqs = [Sequence.from_request(GenerationRequest(f"r{i}", p, params)) for i, p in enumerate(prompts(4, seed=6))]
    eng.runner.add(seqs)
    eng.runner.trace = []
    eng.runner.step()
    torch.cuda.synchronize()
    rec_step = eng.runner.trace[0]
    k = eng.runner.k
    t_bits = eng.runner.logits.view(torch.int16).cpu().numpy().view("uint16")
    d_bits = eng.runner.proposer.logits.view(torch.int16).cpu().numpy().view("uint16")
    for slot, rec in rec_step.items():
        seed = seqs[slot].sampling_generator.seed
        step = int(eng.runner.h_steps[slot]) - 1  # the step counter advanced after the step
        g = len(rec["drafts"])
        assert g == rec["requested"] > 0
        for j, guess in enumerate(rec["drafts"]):
            drawn = oacc.sampled_accept_v3(d_bits[slot * k + j : slot * k + j + 1], [], 0.8, 1.0, seed,
                                           step + ((j + 1) << 48))
            assert drawn == [guess], f"slot {slot} guess {j}"
        want = oacc.sampled_accept_draft(t_bits[slot * (k + 1) : slot * (k + 1) + g + 1],
                                         d_bits[slot * k : slot * k + g], rec["drafts"], 0.8, seed, step)
        assert rec["out"] == want, f"slot {slot}"


def test_verify_proposal_with_draft_probabilities_matches_the_c_oracle():
    """speculative.verify_proposal (verifier.py:27-60) with Proposal.probabilities: the
    distributions enter the kernel as rows T * log(q), and the result equals the C
    oracle's draft-distribution rule on the same rows."""
    from oracle import accept as oacc
    from nanoengine_amd.interface import create_sampling_generator
    from nanoengine_amd.speculative import Proposal, verify_proposal

    torch.manual_seed(9)
    vocab, temp = 3001, 0.7
    for trial in range(12):
        g = 1 + trial % 4
        target = (torch.randn(g + 1, vocab) * 2).bfloat16()
        q = torch.softmax(torch.randn(g, vocab) * 2 / temp, dim=-1)
        guesses = [int(torch.multinomial(q[i], 1)) for i in range(g)]
        gen = create_sampling_generator(100 + trial)
        step = gen.step
        params = SamplingParams(max_new_tokens=8, temperature=temp)
        got = verify_proposal(Proposal(guesses, q), target.to("cuda"), params, gen)
        d_rows = (torch.log(q.to("cuda")) * temp).bfloat16().cpu()  # as verify_proposal forms them
        want = oacc.sampled_accept_draft(target.view(torch.int16).numpy().view("uint16"),
                                         d_rows.view(torch.int16).numpy().view("uint16"), guesses, temp,
                                         gen.seed, step)
        assert got == want, f"trial {trial}"


def test_mixed_greedy_and_sampled_draft_batch_matches_the_oracles():
    """A draft-model batch whose slots sample at their own temperatures (0, 0.8, 0, 1.3):
    a sampled slot's guesses are the contract's draws from its draft rows at its own
    temperature and its tokens the C oracle's draft-distribution acceptance; a greedy
    slot's guesses are its draft rows' first-index argmax and its tokens the greedy
    acceptance of its target rows (verifier.py:27-60 per sequence)."""
    from oracle import accept as oacc
    import numpy as np

    state = unit_norms(random_state_dict(CFG, seed=0, std=0.02))
    dstate = unit_norms(random_state_dict(DCFG, seed=7, std=0.02))
    eng = engine(state, DCFG, dstate, 4)
    temps = [0.0, 0.8, 0.0, 1.3]
    seqs = [Sequence.from_request(GenerationRequest(
        f"r{i}", p, SamplingParams(max_new_tokens=16, temperature=t, seed=10 + i, ignore_eos=True)))
        for i, (p, t) in enumerate(zip(prompts(4, seed=8), temps))]
    eng.runner.add(seqs)
    eng.runner.trace = []
    for _ in range(2):
        eng.runner.step()
    torch.cuda.synchronize()
    rec_step = eng.runner.trace[-1]
    k = eng.runner.k
    t_bits = eng.runner.logits.view(torch.int16).cpu().numpy().view("uint16")
    d_bits = eng.runner.proposer.logits.view(torch.int16).cpu().numpy().view("uint16")
    checked = set()
    for slot, rec in rec_step.items():
        g = len(rec["drafts"])
        assert g == rec["requested"] > 0
        temp = temps[slot]
        t_rows = t_bits[slot * (k + 1) : slot * (k + 1) + g + 1]
        d_rows = d_bits[slot * k : slot * k + g]
        if temp == 0.0:
            draft_argmax = np.argmax(oacc.bf16_to_f32(d_rows), axis=1).tolist()
            assert rec["drafts"] == draft_argmax, f"slot {slot}"
            assert rec["out"] == oacc.greedy_accept(oacc.bf16_to_f32(t_rows), rec["drafts"]), f"slot {slot}"
        else:
            seed = seqs[slot].sampling_generator.seed
            step = int(eng.runner.h_steps[slot]) - 1
            for j, guess in enumerate(rec["drafts"]):
                drawn = oacc.sampled_accept_v3(d_bits[slot * k + j : slot * k + j + 1], [], temp, 1.0, seed,
                                               step + ((j + 1) << 48))
                assert drawn == [guess], f"slot {slot} guess {j}"
            assert rec["out"] == oacc.sampled_accept_draft(t_rows, d_rows, rec["drafts"], temp, seed, step)
        checked.add(temp > 0)
    assert checked == {False, True}


def test_guesses_left_on_the_device_equal_the_read_back_ones():
    """With graphs, the draft's greedy guesses stay on the device for the verify step and
    the host takes them at the next proposal; with a trace they are read back before the
    step.  Every step's tokens, guess counts and kept counts are the same both ways."""
    state = unit_norms(random_state_dict(CFG, seed=0, std=0.02))
    dstate = unit_norms(random_state_dict(DCFG, seed=7, std=0.02))
    ps = prompts(4, seed=3)

    def run(trace):
        eng = engine(state, DCFG, dstate, 4, graphs=True)
        if trace:
            eng.runner.trace = []
        seqs = [Sequence.from_request(GenerationRequest(f"r{i}", p, SamplingParams(max_new_tokens=20,
                                                                                   ignore_eos=True)))
                for i, p in enumerate(ps)]
        steps = [eng.runner.add(seqs)]
        while eng.runner.active_slots or eng.runner.pending:
            steps.append(eng.runner.step())
        out = [{s: (r.tokens, r.num_guesses, r.num_kept) for s, r in res.items()} for res in steps]
        return out, [list(q.token_ids) for q in seqs], eng.runner.proposer

    read_back, ids_a, _ = run(True)
    on_device, ids_b, proposer = run(False)
    assert on_device == read_back and ids_a == ids_b
    assert proposer._cu_graph is not None and proposer.device_proposals > 0
    assert sum(r[1] for step in on_device[1:] for r in step.values()) > 0


@pytest.mark.parametrize("seed", [5, 23])
def test_random_add_step_release_keep_every_draft_request_on_its_generation(seed):
    """Seeded random admissions, releases and steps of 9 requests on 3 slots with graphed
    draft proposals (their guesses left on the device and taken by the host at the next
    proposal or release).  Greedy verification keeps the target's own argmax, so whatever
    the draft guesses and wherever a release cuts a request off, every request's tokens
    are a prefix of the generation it gets when nothing is released, and all of it when it
    finishes by itself."""
    state = unit_norms(random_state_dict(CFG, seed=0, std=0.02))
    dstate = unit_norms(random_state_dict(DCFG, seed=7, std=0.02))
    n_req, n_slots = 9, 3
    ps = prompts(n_req, seed=40 + seed)
    lens = [int(x) for x in np.random.default_rng(seed).integers(2, 31, size=n_req)]

    def run(p_release):
        eng = engine(state, DCFG, dstate, n_slots, graphs=True)
        runner = eng.runner
        rng = np.random.default_rng(seed)
        seqs = [Sequence.from_request(GenerationRequest(f"r{i}", p, SamplingParams(max_new_tokens=n,
                                                                                   ignore_eos=True)))
                for i, (p, n) in enumerate(zip(ps, lens))]
        got = {i: [] for i in range(n_req)}
        end, owner, nxt = {}, {}, 0

        def record(results):
            for slot, r in results.items():
                got[owner[slot]].extend(r.tokens)
                if r.finish_reason is not None:
                    end[owner.pop(slot)] = r.finish_reason

        while nxt < n_req or owner:
            x = rng.random()
            if nxt < n_req and len(owner) < n_slots and x < 0.3:
                free = runner.free_slots()[:1]
                res = runner.add([seqs[nxt]])
                owner[free[0]] = nxt
                nxt += 1
                record(res)
            elif owner and x > 1 - p_release:
                slot = sorted(owner)[int(rng.integers(0, len(owner)))]
                runner.release(slot)
                end[owner.pop(slot)] = "released"
            else:
                record(runner.step())
        assert eng.allocator.num_reserved_slots == 0
        return got, end, runner.proposer.device_proposals

    full, full_end, _ = run(0.0)
    got, end, on_device = run(0.1)
    assert on_device > 0 and "released" in end.values()
    for i in range(n_req):
        assert got[i] == full[i][: len(got[i])], i
        if end[i] != "released":
            assert (got[i], end[i]) == (full[i], full_end[i]), i
