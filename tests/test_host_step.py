"""The verify step's host bookkeeping (nanoengine_amd.host_step): the CPython extension
built from csrc/host_step.c against the Python definitions of the same contract
(speculative_generator.py:54-72, paged_allocator.py:50-55) on random slot states --
mirrors, tables, token lists, sampling steps and results must all agree."""

from __future__ import annotations

import copy

import numpy as np
import pytest

from nanoengine_amd import host_step
from nanoengine_amd.interface import GenerationRequest, SamplingParams
from nanoengine_amd.runner import StepResult
from nanoengine_amd.sequence_state import Sequence

pytestmark = pytest.mark.skipif(not host_step.NATIVE, reason="the _host_step extension is not built")


def _state(seed: int, S: int = 64, R: int = 5):
    rng = np.random.default_rng(seed)
    act = rng.random(S) < 0.8
    lengths = rng.integers(1, 300, S).astype(np.int64)
    owned = ((lengths + 15) // 16 - rng.integers(0, 2, S)).clip(0).astype(np.int64)
    nd = rng.integers(0, R, S).astype(np.int32)
    out = rng.integers(0, 600, (S, R)).astype(np.int32)
    nout = np.minimum(nd + 1, rng.integers(1, R + 1, S)).astype(np.int32)
    gen = rng.integers(0, 100, S).astype(np.int64)
    max_new = rng.integers(50, 140, S).astype(np.int64)
    steps = rng.integers(0, 50, S).astype(np.int64)
    honours = rng.random(S) < 0.5
    slots = [Sequence.from_request(GenerationRequest(f"s{i}", rng.integers(0, 600, int(lengths[i])).tolist(),
                                                     SamplingParams(max_new_tokens=int(max_new[i]))))
             if act[i] else None for i in range(S)]
    return dict(act=act, lengths=lengths, owned=owned, nd=nd, out=out, nout=nout, gen=gen, max_new=max_new,
                steps=steps, honours=honours, slots=slots)


@pytest.mark.parametrize("seed", range(6))
def test_plan_and_assign_match_python(seed):
    st = _state(seed)
    want = host_step.plan_growth_py(st["lengths"], st["nd"], st["owned"], st["act"], 16)
    got = host_step.plan_growth(st["lengths"], st["nd"], st["owned"], st["act"], 16)
    assert got == want
    slots, counts, _, total = got
    blocks = list(range(1000, 1000 + total))
    t1, t2 = np.zeros((64, 40), np.int32), np.zeros((64, 40), np.int32)
    o1, o2 = st["owned"].copy(), st["owned"].copy()
    host_step.assign_blocks_py(t1, o1, slots, counts, blocks)
    host_step.assign_blocks(t2, o2, slots, counts, blocks)
    assert np.array_equal(t1, t2) and np.array_equal(o1, o2)


@pytest.mark.parametrize("seed", range(6))
@pytest.mark.parametrize("stops", [(), (7, 300, 599)])
def test_finish_step_matches_python(seed, stops):
    st = _state(100 + seed)
    active = np.flatnonzero(st["act"]).tolist()
    runs = []
    for fn in (host_step.finish_step_py, host_step.finish_step):
        s = copy.deepcopy(st)
        cached = []
        results, finishing = fn(active, s["slots"], s["out"], s["nout"], s["nd"], s["act"], s["lengths"], s["gen"],
                                s["steps"], s["max_new"], s["honours"], stops, StepResult, cached.append)
        runs.append((results, finishing, s, [q.request_id for q in cached]))
    (r1, f1, s1, c1), (r2, f2, s2, c2) = runs
    assert list(r1) == list(r2) and r1 == r2
    assert f1 == f2 and c1 == c2
    for key in ("lengths", "gen", "steps"):
        assert np.array_equal(s1[key], s2[key])
    for a, b in zip(s1["slots"], s2["slots"]):
        if a is not None:
            assert a.token_ids == b.token_ids and a.num_cached_tokens == b.num_cached_tokens
            assert a.sampling_generator.step == b.sampling_generator.step


@pytest.mark.parametrize("seed", range(8))
@pytest.mark.parametrize("stops", [(), (7, 300, 599)])
def test_launch_ahead_check_matches_the_finishing_slots(seed, stops):
    """VerifyRunner._may_run_ahead (numpy, before the next step is launched) is True
    exactly when finish_step would report no finishing slot for the same outputs: the
    length limit and the stop tokens of slots that honour them, read the same way."""
    from nanoengine_amd.runner import VerifyRunner

    st = _state(seed)
    rng = np.random.default_rng(100 + seed)
    # limits near the emitted counts, so that some seeds finish nothing and some finish a few
    st["max_new"] = st["gen"] + st["nout"] + rng.integers(0 if seed % 2 else 1, 4, st["gen"].shape[0])
    if not stops:
        st["honours"][:] = False
    runner = VerifyRunner.__new__(VerifyRunner)
    runner.run_ahead, runner.proposer, runner.trace = True, None, None
    runner._fifo_blocks, runner.use_graph, runner.graph = True, True, object()
    runner.graph_failed, runner.graph_max_batch, runner.graph_max_context, runner.k = False, None, None, 4
    runner.np_active = st["act"]
    runner.graph_sampled, runner._sampled = False, False
    runner.stop_token_ids = stops
    runner.np_out, runner.np_num_out = st["out"], st["nout"]
    runner.np_gen, runner.np_max_new, runner.np_honours_stop = st["gen"], st["max_new"], st["honours"]
    runner.np_len, runner.np_owned, runner.block_size = st["lengths"], st["owned"], 16
    runner.np_num_drafts_next = st["nd"]
    _, _, _, need = host_step.plan_growth(st["lengths"] + st["nout"] * st["act"], st["nd"], st["owned"], st["act"], 16)

    class Pool:
        num_free_blocks = need + (seed % 3) - 1  # one short, exactly enough, one spare

    runner.allocator = Pool()
    ahead = runner._may_run_ahead(st["act"])
    slots = copy.deepcopy(st["slots"])
    _, finishing = host_step.finish_step_py(
        [i for i in range(len(slots)) if slots[i] is not None], slots, st["out"], st["nout"], st["nd"],
        st["act"], st["lengths"].copy(), st["gen"].copy(), st["steps"].copy(), st["max_new"], st["honours"],
        tuple(sorted(stops)), StepResult, None)
    assert ahead == (not finishing and Pool.num_free_blocks >= need)


@pytest.mark.parametrize("seed", range(12))
@pytest.mark.parametrize("honour", [False, True])
def test_deep_launch_reserves_for_every_outcome_of_the_running_step(seed, honour):
    """VerifyRunner._maybe_launch_deep (the step after a running one, launched before the
    running step's outputs are known) runs the slots active on the host, whether or not
    one can finish in the running step; its block bound covers every outcome of the
    running step (1 .. g + 1 tokens) followed by the guesses the device then requests
    (min(k, max_new - generated - 1), none at the limit) and the bonus row, and reaches
    at most one token past the sequence's last position (prompt + max_new - 1 tokens)."""
    from collections import deque

    from nanoengine_amd.runner import VerifyRunner, _Launched

    st = _state(seed)
    rng = np.random.default_rng(200 + seed)
    k = 4
    act = st["act"]
    # limits from "finishes in the running step for some outcome" to far away; the device
    # never requests more guesses than max_new - generated - 1
    st["max_new"] = st["gen"] + st["nd"] + 1 + rng.integers(0, 12, act.shape[0])
    honours = st["honours"] & honour
    runner = VerifyRunner.__new__(VerifyRunner)
    runner.run_ahead, runner.proposer, runner.trace = True, None, None
    runner._fifo_blocks, runner.use_graph, runner.graph = True, True, object()
    runner.graph_failed, runner.graph_max_batch, runner.graph_max_context, runner.k = False, None, None, k
    runner.graph_sampled, runner._sampled = False, False
    runner.np_active, runner.np_honours_stop = act, honours
    runner.np_len, runner.np_gen, runner.np_max_new = st["lengths"], st["gen"], st["max_new"]
    runner.np_owned, runner.block_size = st["owned"], 16
    runner._read_back_views = [(None, (None, None, st["nd"])), None, None]  # the running step's guess counts
    runner._inflight = deque([_Launched(np.flatnonzero(act).tolist(), act, None, 1, 0, None)])
    runner.ahead_launches = runner.deep_launches = 0

    class Pool:
        num_free_blocks = 10 ** 6

    runner.allocator = Pool()
    bounds = []
    runner._launch = lambda bound=None: bounds.append(bound) or "launched"
    runner._maybe_launch_deep()
    assert len(bounds) == 1
    b_len, b_drafts = bounds[0]
    assert b_len.dtype == np.int64 and b_drafts.dtype == np.int32
    bound = b_len + b_drafts
    g, gen, lengths, max_new = st["nd"].astype(np.int64), st["gen"], st["lengths"], st["max_new"]
    for s in np.flatnonzero(act):
        for e in range(1, int(g[s]) + 2):  # the running step emits e tokens
            nxt = max(0, min(k, int(max_new[s] - gen[s] - e - 1)))
            assert int(lengths[s]) + e + nxt <= bound[s]
        assert bound[s] <= lengths[s] - gen[s] + max_new[s]
    assert not b_drafts[~act].any()
    assert runner.deep_launches == 1 and list(runner._inflight)[-1] == "launched"

    # too few free blocks for the bound: nothing is launched
    runner._inflight = deque([_Launched(np.flatnonzero(act).tolist(), act, None, 1, 0, None)])
    *_, need = host_step.plan_growth(b_len, b_drafts, st["owned"], act, 16)
    Pool.num_free_blocks = need - 1
    bounds.clear()
    runner._maybe_launch_deep()
    assert not bounds or need == 0


@pytest.mark.parametrize("fn_name", ["finish_step_py", "finish_step"])
@pytest.mark.parametrize("case", ["emitted-too-many", "emitted-negative", "inactive-slot", "empty-slot",
                                  "slot-out-of-range"])
def test_finish_step_refuses_bad_inputs_before_changing_any_mirror(fn_name, case):
    """Both implementations check every slot's inputs first: a bad emitted count or a bad
    active slot raises ValueError with the mirrors, token lists and sampling steps untouched."""
    fn = getattr(host_step, fn_name)
    st = _state(7)
    active = np.flatnonzero(st["act"]).tolist()
    victim = active[len(active) // 2]
    if case == "emitted-too-many":
        st["nout"][victim] = st["out"].shape[1] + 1
    elif case == "emitted-negative":
        st["nout"][victim] = -1
    elif case == "inactive-slot":
        active.append(int(np.flatnonzero(~st["act"])[0]))
    elif case == "empty-slot":
        st["slots"][victim] = None
    else:
        active.append(len(st["slots"]))
    before = copy.deepcopy(st)
    with pytest.raises(ValueError):
        fn(active, st["slots"], st["out"], st["nout"], st["nd"], st["act"], st["lengths"], st["gen"], st["steps"],
           st["max_new"], st["honours"], (), StepResult, None)
    for key in ("lengths", "gen", "steps"):
        assert np.array_equal(st[key], before[key])
    for a, b in zip(st["slots"], before["slots"]):
        if a is not None:
            assert a.token_ids == b.token_ids and a.sampling_generator.step == b.sampling_generator.step


def test_finish_step_keeps_a_sequence_alive_while_its_callback_drops_it_from_the_slot_list():
    """on_cached may change the slot list it was given: here it removes the list's entry
    for the sequence it is called with, so during the call the list no longer holds it.
    The extension holds each sequence across its own calls; the step completes, every
    slot gets its result and every sequence its tokens."""
    st = _state(9)
    st["max_new"][:] = 10_000  # no slot finishes: every slot appends and calls on_cached
    active = np.flatnonzero(st["act"]).tolist()
    slots = list(st["slots"])
    want = {s: slots[s].token_ids + st["out"][s, : st["nout"][s]].tolist() for s in active}
    seen = {}

    def on_cached(seq):
        s = slots.index(seq)
        slots[s] = None
        seen[s] = seq

    results, finishing = host_step.finish_step(active, slots, st["out"], st["nout"], st["nd"], st["act"],
                                               st["lengths"], st["gen"], st["steps"], st["max_new"],
                                               st["honours"], (), StepResult, on_cached)
    assert not finishing and sorted(results) == active
    assert sorted(seen) == active
    for s in active:
        assert seen[s].token_ids == want[s]
