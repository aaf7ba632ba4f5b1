"""A1, A9, A10: n-gram drafting and fused acceptance, bit-exact against the oracle.

n-gram: oracle.ngram.propose restates NgramProposer.propose
(ne/engine/speculative/proposers.py:44-57); drafts and counts must be identical.
Greedy acceptance: oracle.accept.greedy_accept restates verify_proposal's greedy
path (ne/engine/speculative/verifier.py:27-60); accepted counts, tokens, history
append and the rolled-back cached count must be identical.
Sampled acceptance: the C oracle implements the explicit-uniform contract; results
must be identical token for token.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import accept as oracle_accept
from oracle import ngram as oracle_ngram
from nanoengine_amd import kernels

pytestmark = pytest.mark.gpu


def run_ngram(device, histories, num_tokens, max_ngram=3, max_drafts=4):
    cap = max(max(len(h) for h in histories), 1)
    hist = torch.zeros(len(histories), cap, dtype=torch.int32)
    for i, h in enumerate(histories):
        hist[i, : len(h)] = torch.tensor(h, dtype=torch.int32)
    lens = torch.tensor([len(h) for h in histories], dtype=torch.int32)
    nt = torch.tensor(num_tokens, dtype=torch.int32)
    drafts, counts = kernels.ngram_propose(hist.to(device), lens.to(device), nt.to(device), max_ngram,
                                           max_drafts)
    torch.cuda.synchronize()
    counts = counts.cpu().tolist()
    return [drafts.cpu()[i, : counts[i]].tolist() for i in range(len(histories))]


def test_ngram_reference_kats(device):
    # nt/engine/test_speculative_decoding.py:35-42
    got = run_ngram(device, [[1, 2, 3, 4, 5, 9, 1, 2], [1, 2, 3, 4]], [3, 3], max_ngram=2, max_drafts=3)
    assert got == [[3, 4, 5], []]


@pytest.mark.parametrize("vocab", [3, 8, 50])
def test_ngram_random_matches_oracle(device, vocab):
    rng = np.random.default_rng(vocab)
    histories = [rng.integers(0, vocab, size=int(n)).tolist() for n in rng.integers(0, 600, size=64)]
    histories += [[], [7], [7, 7], [1, 2, 1, 2, 1]]
    num_tokens = rng.integers(0, 5, size=len(histories)).tolist()
    got = run_ngram(device, histories, num_tokens)
    want = [oracle_ngram.propose(h, n, 3) if n else [] for h, n in zip(histories, num_tokens)]
    assert got == want


@pytest.mark.parametrize("k", [4, 8])
def test_advance_and_propose_equals_advance_then_propose(device, k):
    """The verify step's tail in one launch: counters, guess counts and drafts equal those
    of ne_advance_step_counts followed by ne_ngram_propose on the same state, for active
    and inactive slots and limits that leave 0 .. k guesses; the drafts equal the oracle's."""
    rng = np.random.default_rng(40 + k)
    n, cap = 64, 700
    lens = rng.integers(0, 600, n).astype(np.int32)
    lens[::9] = 0  # inactive slots
    hist = torch.from_numpy(rng.integers(0, 6, (n, cap)).astype(np.int32))
    num_out = torch.from_numpy(rng.integers(1, k + 2, n).astype(np.int32))
    generated = torch.from_numpy(rng.integers(0, 100, n).astype(np.int32))
    max_new = (generated + num_out + torch.from_numpy(rng.integers(0, k + 3, n).astype(np.int32))).to(torch.int32)
    steps = torch.from_numpy(rng.integers(0, 1000, n).astype(np.int64))
    hl = torch.from_numpy(lens)
    ins = [t.to(device) for t in (hist, hl, num_out, max_new, generated, steps)]
    a = [t.clone() for t in ins]  # separate launches
    guesses_a = torch.full((n,), -1, dtype=torch.int32, device=device)
    kernels.advance_step_counts(a[1], a[2], a[3], a[4], a[5], guesses_a, k)
    drafts_a, count_a = kernels.ngram_propose(a[0], a[1], guesses_a, 3, k)
    b = [t.clone() for t in ins]  # one launch
    guesses_b = torch.full((n,), -1, dtype=torch.int32, device=device)
    drafts_b = torch.zeros(n, k, dtype=torch.int32, device=device)
    count_b = torch.full((n,), -1, dtype=torch.int32, device=device)
    kernels.advance_and_propose(b[0], b[1], b[2], b[3], b[4], b[5], guesses_b, k, 3, drafts_b, count_b)
    torch.cuda.synchronize()
    for x, y in zip(a, b):
        assert torch.equal(x, y)
    assert torch.equal(guesses_a, guesses_b) and torch.equal(count_a, count_b)
    counts = count_b.cpu().tolist()
    assert all(torch.equal(drafts_a[i, : counts[i]], drafts_b[i, : counts[i]]) for i in range(n))
    g = guesses_b.cpu().tolist()
    assert sorted(set(g)) == list(range(0, k + 1)) or len(set(g)) > 3
    for i in range(n):
        want = oracle_ngram.propose(hist[i, : lens[i]].tolist(), g[i], 3) if g[i] and lens[i] else []
        assert drafts_b[i, : counts[i]].cpu().tolist() == want


def test_ngram_long_history_k8(device):
    rng = np.random.default_rng(5)
    histories = [rng.integers(0, 20, size=17417).tolist() for _ in range(4)]
    got = run_ngram(device, histories, [8, 8, 3, 0], max_drafts=8)
    want = [oracle_ngram.propose(h, n, 3) if n else [] for h, n in zip(histories, [8, 8, 3, 0])]
    assert got == want


def test_ngram_match_found_deep_in_the_history(device):
    """Distinct tokens with one planted earlier occurrence of the last n tokens, at
    depths on both sides of 1,024 and 2,048 starts from the newest, at start 0, only for
    n = 2 or n = 1, twice (the later copy wins) or nowhere."""
    L = 5000
    base = list(range(10000, 10000 + L))
    cases = []
    for p in (0, 1, L - 1030, L - 1027, L - 1026, L - 1025, L - 2051, L - 2050, L - 8, 2500):
        cases.append(base + base[p:p + 3])  # last trigram occurs at start p
    cases.append(base + [base[2000], base[2001], 7])  # only the last token (7) is new: no match
    cases.append(base + [3, base[1200], base[1201]])  # n = 2 only, deep
    cases.append(base + [3, 4, base[40]])  # n = 1 only, near the start
    cases.append(base[:3000] + [5, 6, 9] + base[3000:] + [5, 6, 9])  # one copy, mid-history
    cases.append([5, 6, 9] + base + [5, 6, 9] + base[:100] + [5, 6, 9])  # two copies: the later wins
    got = run_ngram(device, cases, [8] * len(cases), max_drafts=8)
    want = [oracle_ngram.propose(h, 8, 3) for h in cases]
    assert got == want
    assert all(w for w in want[:10]) and want[10] == []


def test_ngram_sixteen_token_matches_at_the_scan_pass_edges(device):
    """max_ngram 16 over 12,000 distinct tokens: the kernel compares 4,096 window ends per
    pass against a stretch of history held in LDS that reaches 15 tokens below the pass's
    lowest end.  Planted 16-token matches end on both sides of the first and second pass
    edges (end e = len - 2 - d for d around 4,096 and 8,192), at the history's start, and
    5-token-only matches (the token before the suffix is new) end at the same edges."""
    L = 12000
    base = list(range(20000, 20000 + L))
    cases = []
    for d in (4094, 4095, 4096, 4097, 8191, 8192, 8193):
        # history base + base[p:p+16] has len L + 16, so the planted end p + 15 is len - 2 - d
        p = L - 1 - d
        cases.append(base + base[p:p + 16])
    cases.append(base + base[0:16])  # the match starts at token 0
    for d in (4095, 4096, 8192):
        # history base + [new] + base[p:p+5] has len L + 6: the 5-token match ends at p + 4
        p = L - d
        cases.append(base + [7] + base[p:p + 5])
    got = run_ngram(device, cases, [8] * len(cases), max_ngram=16, max_drafts=8)
    want = [oracle_ngram.propose(h, 8, 16) for h in cases]
    assert got == want
    assert all(want)
    for d, w in zip((4094, 4095, 4096, 4097, 8191, 8192, 8193), want):
        p = L - 1 - d
        assert w == base[p + 16:p + 24]  # the planted window, and not some other one


def bf16_logits(rows, vocab, rng, scale=1.0):
    return torch.tensor(rng.standard_normal((rows, vocab)) * scale, dtype=torch.float32).to(torch.bfloat16)


def make_accept_case(rng, num_seqs, vocab, max_drafts, match_prob=0.7, scale=1.0):
    num_drafts = rng.integers(0, max_drafts + 1, size=num_seqs)
    row_start = np.concatenate([[0], np.cumsum(num_drafts + 1)[:-1]]).astype(np.int32)
    logits = bf16_logits(int((num_drafts + 1).sum()), vocab, rng, scale)
    targets = torch.argmax(logits.float(), dim=1).numpy()
    drafts = np.zeros((num_seqs, max_drafts), dtype=np.int32)
    for b in range(num_seqs):
        for i in range(num_drafts[b]):
            t = targets[row_start[b] + i]
            drafts[b, i] = t if rng.random() < match_prob else rng.integers(0, vocab)
    return logits, drafts, num_drafts.astype(np.int32), row_start


@pytest.mark.parametrize("vocab", [1000, 151936])
def test_greedy_accept_matches_oracle_and_updates_state(device, vocab):
    rng = np.random.default_rng(vocab)
    b, k = 64, 4
    logits, drafts, nd, rs = make_accept_case(rng, b, vocab, k)
    cap = 64
    hist_len = rng.integers(5, 30, size=b).astype(np.int32)
    history = torch.zeros(b, cap, dtype=torch.int32)
    d = lambda a: torch.as_tensor(a).to(device)
    h_dev, hl_dev = history.to(device), d(hist_len)
    cached = torch.zeros(b, dtype=torch.int32, device=device)
    out, nout = kernels.accept(d(drafts), d(nd), d(rs), vocab, logits=logits.to(device),
                               history=h_dev, history_len=hl_dev, num_cached=cached)
    torch.cuda.synchronize()
    out, nout = out.cpu(), nout.cpu()
    lf = logits.float().numpy()
    for s in range(b):
        want = oracle_accept.greedy_accept(lf[rs[s] : rs[s] + nd[s] + 1], drafts[s, : nd[s]].tolist())
        assert out[s, : nout[s]].tolist() == want
        assert h_dev[s, hist_len[s] : hist_len[s] + len(want)].cpu().tolist() == want
        assert int(hl_dev[s]) == hist_len[s] + len(want)
        assert int(cached[s]) == hist_len[s] + len(want) - 1


def test_greedy_reference_kat(device):
    # nt/engine/test_speculative_decoding.py:45-55: rows best = [2, 4, 1, 5]
    logits = torch.full((8, 6), -10.0)
    for row, best in enumerate([2, 4, 1, 5, 2, 4, 1, 5]):
        logits[row, best] = 10.0
    drafts = torch.tensor([[2, 4, 1], [2, 3, 1]], dtype=torch.int32)
    out, nout = kernels.accept(drafts.to(device), torch.tensor([3, 3], dtype=torch.int32).to(device),
                               torch.tensor([0, 4], dtype=torch.int32).to(device), 6,
                               logits=logits.to(torch.bfloat16).to(device))
    torch.cuda.synchronize()
    assert out[0, : nout[0]].tolist() == [2, 4, 1, 5]
    assert out[1, : nout[1]].tolist() == [2, 4]


def test_greedy_ties_take_first_index(device):
    logits = torch.zeros(2, 300, dtype=torch.bfloat16)
    logits[0, [7, 9, 200]] = 3.0
    logits[1, [5, 6]] = 1.0
    out, nout = kernels.accept(torch.tensor([[7]], dtype=torch.int32).to(device),
                               torch.tensor([1], dtype=torch.int32).to(device),
                               torch.tensor([0], dtype=torch.int32).to(device), 300,
                               logits=logits.to(device))
    torch.cuda.synchronize()
    assert out[0, : nout[0]].tolist() == [7, 5]


def test_greedy_from_lm_head_partials(device):
    rng = np.random.default_rng(3)
    vocab, b = 8192, 16
    hidden = torch.tensor(rng.standard_normal((b * 5, 1024)) * 0.02, dtype=torch.float32).to(torch.bfloat16)
    embed = torch.tensor(rng.standard_normal((vocab, 1024)) * 0.02, dtype=torch.float32).to(torch.bfloat16)
    logits, partials = kernels.lm_head(hidden.to(device), embed.to(device), logits=True, argmax_partials=True)
    tg = torch.argmax(logits.float(), dim=1).cpu().numpy()
    drafts = np.stack([tg[5 * s : 5 * s + 4] for s in range(b)]).astype(np.int32)
    drafts[::3, 2] = (drafts[::3, 2] + 1) % vocab
    nd = np.full(b, 4, dtype=np.int32)
    rs = (np.arange(b) * 5).astype(np.int32)
    d = lambda a: torch.as_tensor(a).to(device)
    o1, n1 = kernels.accept(d(drafts), d(nd), d(rs), vocab, logits=logits)
    o2, n2 = kernels.accept(d(drafts), d(nd), d(rs), vocab, argmax_partials=partials)
    torch.cuda.synchronize()
    assert torch.equal(n1, n2) and torch.equal(o1, o2)


@pytest.mark.parametrize("vocab,temperature", [(151936, 0.8), (1000, 1.0), (50, 0.3)])
def test_sampled_accept_matches_c_oracle(device, vocab, temperature):
    rng = np.random.default_rng(vocab)
    b, k = 32, 4
    logits, drafts, nd, rs = make_accept_case(rng, b, vocab, k, match_prob=0.5, scale=3.0)
    seeds = rng.integers(0, 2**62, size=b).astype(np.int64)
    steps = rng.integers(0, 1000, size=b).astype(np.int64)
    d = lambda a: torch.as_tensor(a).to(device)
    out, nout = kernels.accept(d(drafts), d(nd), d(rs), vocab, logits=logits.to(device),
                               temperature=temperature, seeds=d(seeds), steps=d(steps))
    torch.cuda.synchronize()
    out, nout = out.cpu(), nout.cpu()
    bits = logits.view(torch.int16).numpy().view(np.uint16)
    for s in range(b):
        want = oracle_accept.sampled_accept_v3(bits[rs[s] : rs[s] + nd[s] + 1], drafts[s, : nd[s]].tolist(),
                                               temperature, 1.0, int(seeds[s]), int(steps[s]))
        assert out[s, : nout[s]].tolist() == want, f"sequence {s}"


def test_sampled_golden_fixture(device):
    from pathlib import Path
    import json

    path = Path(__file__).parent / "golden" / "sampled_accept.json"
    case = json.loads(path.read_text())
    vocab = case["vocab"]
    bits = np.array(case["logit_bits"], dtype=np.uint16).reshape(-1, vocab)
    logits = torch.from_numpy(bits.view(np.int16).copy()).view(torch.bfloat16)
    d = lambda a: torch.as_tensor(np.asarray(a)).to(device)
    out, nout = kernels.accept(d(np.array(case["drafts"], dtype=np.int32)), d(np.array(case["num_drafts"], dtype=np.int32)),
                               d(np.array(case["row_start"], dtype=np.int32)), vocab, logits=logits.to(device),
                               temperature=case["temperature"], seeds=d(np.array(case["seeds"], dtype=np.int64)),
                               steps=d(np.array(case["steps"], dtype=np.int64)),
                               top_p=d(np.array(case["top_p"], dtype=np.float32)))
    torch.cuda.synchronize()
    got = [out[s, : nout[s]].tolist() for s in range(len(case["expected"]))]
    assert got == case["expected"]


@pytest.mark.parametrize("top_p", [0.5, 0.9])
def test_top_p_mixed_batch_matches_c_oracle(device, top_p):
    """A10 with top-p (sampling.py:21-38) at the full vocabulary: per-sequence temperatures
    (some 0: greedy rows in the same call, read from the logits) and top-p values, each
    sequence's tokens identical to the C oracle's contract (or to the greedy oracle)."""
    vocab, b, k = 151936, 24, 4
    rng = np.random.default_rng(int(top_p * 100))
    logits, drafts, nd, rs = make_accept_case(rng, b, vocab, k, match_prob=0.5, scale=3.0)
    temps = rng.choice([0.0, 0.7, 1.0, 1.3], size=b).astype(np.float32)
    temps[:2] = [0.0, 0.8]
    tops = np.where(rng.random(b) < 0.75, top_p, 1.0).astype(np.float32)
    seeds = rng.integers(0, 2**62, size=b).astype(np.int64)
    steps = rng.integers(0, 1000, size=b).astype(np.int64)
    d = lambda a: torch.as_tensor(a).to(device)
    out, nout = kernels.accept(d(drafts), d(nd), d(rs), vocab, logits=logits.to(device), temperature=d(temps),
                               top_p=d(tops), any_sampled=True, seeds=d(seeds), steps=d(steps))
    torch.cuda.synchronize()
    out, nout = out.cpu(), nout.cpu()
    bits = logits.view(torch.int16).numpy().view(np.uint16)
    lf = logits.float().numpy()
    for s in range(b):
        rows = slice(rs[s], rs[s] + nd[s] + 1)
        guesses = drafts[s, : nd[s]].tolist()
        if temps[s] == 0:
            want = oracle_accept.greedy_accept(lf[rows], guesses)
        else:
            want = oracle_accept.sampled_accept_v3(bits[rows], guesses, float(temps[s]), float(tops[s]),
                                                   int(seeds[s]), int(steps[s]))
        assert out[s, : nout[s]].tolist() == want, f"sequence {s} (T={temps[s]}, top_p={tops[s]})"


def _v3_batch(device, rows_per_seq, guesses, temps, tops, seed0=11):
    """Run ne_accept on explicit rows (uint16 bf16 patterns per sequence) and compare every
    sequence with the C oracle's integer-mass contract."""
    vocab = rows_per_seq[0].shape[1]
    b, k = len(rows_per_seq), max(1, max(len(g) for g in guesses))
    bits = np.concatenate(rows_per_seq)
    rs = np.concatenate([[0], np.cumsum([r.shape[0] for r in rows_per_seq])[:-1]]).astype(np.int32)
    nd = np.array([len(g) for g in guesses], dtype=np.int32)
    drafts = np.zeros((b, k), dtype=np.int32)
    for s, g in enumerate(guesses):
        drafts[s, : len(g)] = g
    seeds = np.arange(seed0, seed0 + b, dtype=np.int64) * 7919
    steps = np.arange(b, dtype=np.int64) * 3
    logits = torch.from_numpy(bits.view(np.int16).copy()).view(torch.bfloat16)
    d = lambda a: torch.as_tensor(a).to(device)
    out, nout = kernels.accept(d(drafts), d(nd), d(rs), vocab, logits=logits.to(device),
                               temperature=d(np.asarray(temps, dtype=np.float32)),
                               top_p=d(np.asarray(tops, dtype=np.float32)), any_sampled=True,
                               seeds=d(seeds), steps=d(steps))
    torch.cuda.synchronize()
    out, nout = out.cpu(), nout.cpu()
    for s in range(b):
        want = oracle_accept.sampled_accept_v3(rows_per_seq[s], list(guesses[s]), float(temps[s]), float(tops[s]),
                                               int(seeds[s]), int(steps[s]))
        assert out[s, : nout[s]].tolist() == want, f"sequence {s}"
    return [out[s, : nout[s]].tolist() for s in range(b)]


def test_v3_count_wraps_on_both_halves_of_a_histogram_word(device):
    """One bf16 value filling most of a 151,936-token row wraps its 16-bit histogram count
    (twice): an even key (low half, whose carries enter its neighbour's half), an odd key
    (high half), and both keys of one word together.  Counts, weights and draws equal the
    C oracle's."""
    vocab = 151936
    rng = np.random.default_rng(41)

    def row_with(values_counts):
        vals = (rng.standard_normal(vocab) * 0.5).astype(np.float32)
        pos = rng.permutation(vocab)
        at = 0
        for v, n in values_counts:
            vals[pos[at : at + n]] = v
            at += n
        return oracle_accept.bf16_bits(vals)

    even = np.float32(1.0)       # bf16 0x3F80: key 0xBF80 (even)
    odd = np.float32(1.0078125)  # bf16 0x3F81: key 0xBF81 (odd), the same histogram word
    assert oracle_accept.key16(oracle_accept.bf16_bits(np.array([even, odd])))[0] % 2 == 0
    rows, guesses, temps, tops = [], [], [], []
    for vc in ([(even, 140000)], [(odd, 140000)], [(even, 70000), (odd, 70000)], [(odd, 131072)],
               [(even, 65536), (odd, 65535)]):
        r = np.stack([row_with(vc) for _ in range(3)])
        rows.append(r)
        guesses.append([int(np.flatnonzero(oracle_accept.bf16_to_f32(r[0]) == vc[0][0])[0]), 5])
        temps.append(0.7)
        tops.append(0.95)
    _v3_batch(device, rows, guesses, temps, tops)


def test_v3_top_p_ties_out_of_vocabulary_and_all_weight_guesses(device):
    """Top-p thresholds inside a run of equal logits (a guess among the ties, before and
    after the kept ones), a guess outside the vocabulary (weighs 0: always rejected, the
    draw removes nothing), a guess holding all the kept weight (always kept), a row where
    only one token has weight, many rows in one call: identical to the C oracle."""
    rng = np.random.default_rng(42)
    vocab = 3000
    rows, guesses, temps, tops = [], [], [], []
    for s in range(40):
        vals = np.round(rng.standard_normal((4, vocab)) * 2).astype(np.float32)  # few values: many ties
        bits = oracle_accept.bf16_bits(vals)
        f = oracle_accept.bf16_to_f32(bits)
        g = []
        for i in range(3):
            top = np.flatnonzero(f[i] == f[i].max())
            choice = s % 4
            if choice == 0:
                g.append(int(top[-1]))            # the last of the largest ties
            elif choice == 1:
                g.append(int(rng.integers(0, vocab)))
            elif choice == 2:
                g.append(vocab + 5 if i == 1 else int(top[0]))  # outside the vocabulary
            else:
                g.append(int(top[0]))
        rows.append(bits)
        guesses.append(g)
        temps.append(float(rng.choice([0.5, 1.0, 2.0])))
        tops.append(float(rng.choice([1.0, 0.3, 0.6, 0.9])))
    one = np.full((2, vocab), -300.0, dtype=np.float32)
    one[:, 17] = 4.0  # only token 17 has weight: a guess of 17 is always kept, others draw 17
    rows += [oracle_accept.bf16_bits(one)] * 2
    guesses += [[17], [3]]
    temps += [1.0, 1.0]
    tops += [0.5, 1.0]
    out = _v3_batch(device, rows, guesses, temps, tops)
    assert out[-2] == [17, 17] and out[-1] == [17]


@pytest.mark.parametrize("form", ["draft_logits", "draft_probs"])
def test_draft_distributions_with_top_p_match_c_oracle(device, form):
    """Guesses verified against a draft distribution (verifier.py:36-56): the draft model's
    bf16 logits (q' = the same temperature / top-p softmax) or fp32 probabilities used as
    given; top_p 0.9 on the target; identical to the C oracle."""
    vocab, b, k, temp, top_p = 32000, 16, 4, 0.9, 0.9
    rng = np.random.default_rng(77 if form == "draft_probs" else 78)
    logits, drafts, nd, rs = make_accept_case(rng, b, vocab, k, match_prob=0.5, scale=3.0)
    drow = (np.arange(b) * k).astype(np.int32)
    dlog = torch.tensor(rng.standard_normal((b * k, vocab)) * 3.0, dtype=torch.float32).to(torch.bfloat16)
    dbits = dlog.view(torch.int16).numpy().view(np.uint16)
    dprobs = torch.softmax(dlog.float() / temp, dim=1).contiguous()
    seeds = rng.integers(0, 2**62, size=b).astype(np.int64)
    steps = rng.integers(0, 1000, size=b).astype(np.int64)
    d = lambda a: torch.as_tensor(a).to(device)
    kw = {"draft_logits": dlog.to(device)} if form == "draft_logits" else {"draft_probs": dprobs.to(device)}
    out, nout = kernels.accept(d(drafts), d(nd), d(rs), vocab, logits=logits.to(device), temperature=temp,
                               top_p=top_p, seeds=d(seeds), steps=d(steps), draft_row_start=d(drow), **kw)
    torch.cuda.synchronize()
    out, nout = out.cpu(), nout.cpu()
    bits = logits.view(torch.int16).numpy().view(np.uint16)
    for s in range(b):
        rows = slice(rs[s], rs[s] + nd[s] + 1)
        dr = slice(drow[s], drow[s] + k)
        extra = {"draft_bits": dbits[dr]} if form == "draft_logits" else {"draft_probs": dprobs.numpy()[dr]}
        want = oracle_accept.sampled_accept_v2(bits[rows], drafts[s, : nd[s]].tolist(), temp, top_p,
                                               int(seeds[s]), int(steps[s]), **extra)
        assert out[s, : nout[s]].tolist() == want, f"sequence {s}"


def test_history_append_stops_at_the_row_capacity(device):
    """A history row holds history_stride tokens: an append that would pass it writes only
    what fits (the host refuses such requests; this bounds the kernel regardless)."""
    vocab = 64
    logits = torch.full((5, vocab), -5.0)
    for r, t in enumerate([3, 4, 5, 6, 7]):
        logits[r, t] = 5.0
    drafts = torch.tensor([[3, 4, 5, 6]], dtype=torch.int32)
    history = torch.full((2, 10), -9, dtype=torch.int32)  # row 1 must stay untouched
    hl = torch.tensor([8, 0], dtype=torch.int32)
    d = lambda a: a.to(device)
    h = d(history)
    hld = d(hl)
    cached = torch.zeros(2, dtype=torch.int32, device=device)
    out, nout = kernels.accept(d(torch.cat([drafts, drafts])), d(torch.tensor([4, 4], dtype=torch.int32)),
                               d(torch.tensor([0, 0], dtype=torch.int32)), vocab,
                               logits=d(logits.to(torch.bfloat16)), history=h, history_len=hld, num_cached=cached)
    torch.cuda.synchronize()
    assert out[0, : nout[0]].tolist() == [3, 4, 5, 6, 7]
    assert h.cpu()[0].tolist() == [-9] * 8 + [3, 4]
    assert h.cpu()[1].tolist() == [-9] * 10
    assert hld.cpu().tolist() == [10, 0]
