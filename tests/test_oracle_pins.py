"""Pins the CPU oracle before results are checked against it (CPU only).

Every oracle function is checked against something that does not share its
formula: the known-answer vectors of the reference's own tests (transcribed in
tests/golden/reference_kats.json with their source lines), closed forms, brute
force on tiny inputs, an fp64 textbook restatement, published test vectors
(Random123's Philox4x32-10 KATs) and an independent Qwen3 implementation
(Hugging Face transformers).  Each check is chosen so that a plausible slip in
the oracle (a dropped term, a wrong sign, index or tie rule) fails it.
"""

from __future__ import annotations

import json
import math
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import accept as oacc
from oracle import attention as oatt
from oracle import model as om
from oracle import ngram as ong
from oracle import paging as opg
from oracle import quant as oq
from oracle import verify as ov

KATS = json.loads((Path(__file__).parent / "golden" / "reference_kats.json").read_text())


# ------------------------------------------------------------------ A1 n-gram
def test_ngram_reference_kat():
    kat = KATS["ngram"]
    for case in kat["cases"]:
        assert ong.propose(case["token_ids"], kat["num_tokens"], kat["max_ngram"]) == case["expected"]


def _ngram_brute(tokens, k, max_n, min_n=1):
    """All (n, start) matches enumerated; the largest n wins, then the latest start."""
    L = len(tokens)
    matches = [(n, s) for n in range(min_n, max_n + 1) if L > n
               for s in range(0, L - n) if tokens[s:s + n] == tokens[L - n:]]
    if not matches:
        return []
    best_n = max(n for n, _ in matches)
    start = max(s for n, s in matches if n == best_n)
    return tokens[start + best_n:start + best_n + k]


def test_ngram_matches_brute_force_and_batch_form():
    rng = np.random.default_rng(0)
    for trial in range(400):
        L = int(rng.integers(1, 40))
        vocab = int(rng.integers(2, 6))
        toks = rng.integers(0, vocab, size=L).tolist()
        k = int(rng.integers(1, 6))
        n = int(rng.integers(1, 5))
        want = _ngram_brute(toks, k, n)
        assert ong.propose(toks, k, n) == want, (toks, k, n)
        hist = np.zeros((1, 48), dtype=np.int32)
        hist[0, :L] = toks
        d, c = ong.propose_batch_numpy(hist, np.array([L]), np.array([k]), n, 8)
        assert d[0, : c[0]].tolist() == want


def test_num_guesses_never_passes_the_length_limit():
    # speculative_generator.py:131-132: min(k, remaining - 1), floored at 0
    assert ong.num_guesses(128, 0, 4) == 4
    assert ong.num_guesses(128, 125, 4) == 2
    assert ong.num_guesses(128, 127, 4) == 0
    assert ong.num_guesses(128, 128, 4) == 0


# ------------------------------------------------------------------ A9 greedy verify
def _kat_logits():
    kat = KATS["greedy_verify"]
    logits = torch.full((len(kat["row_best"]), kat["vocab"]), kat["low"])
    for row, best in enumerate(kat["row_best"]):
        logits[row, best] = kat["high"]
    return kat, logits


def test_greedy_verify_reference_kat_both_restatements():
    kat, logits = _kat_logits()
    for case in kat["cases"]:
        g = case["guesses"]
        got_ref = ov.verify_proposal(g, None, logits, 0.0, 1.0, ov.create_sampling_generator(0))
        got_acc = oacc.greedy_accept(logits[: len(g) + 1].numpy(), g)
        assert got_ref == case["expected"] and got_acc == case["expected"]


def test_greedy_takes_first_index_on_ties():
    rows = np.zeros((2, 8), dtype=np.float32)
    rows[0, [3, 5]] = 1.0
    rows[1, [1, 6]] = 2.0
    assert oacc.greedy_accept(rows, [3]) == [3, 1]
    assert oacc.greedy_accept(rows, [5]) == [3]
    kat = KATS["greedy_argmax"]
    assert int(np.argmax(np.asarray(kat["logits"]))) == kat["expected"]


# ------------------------------------------------------------------ A10 sampled verify
def _chi_square(counts, probs, trials):
    expected = np.asarray(probs) * trials
    return float(((np.asarray(counts) - expected) ** 2 / expected).sum())


def test_reference_semantics_rejection_sampling_chi_square():
    """The reference's own statistical test (test_speculative_decoding.py:58-74) on the
    oracle's restatement of verify_proposal with torch generator draws."""
    kat = KATS["rejection_sampling_chi_square"]
    target = torch.tensor(kat["target"])
    draft = torch.tensor(kat["draft"])
    logits = torch.log(target).repeat(2, 1)
    gen = ov.create_sampling_generator(kat["seed"])
    counts = np.zeros(5)
    for _ in range(kat["trials"]):
        guess = int(torch.multinomial(draft, 1, generator=gen).item())
        out = ov.verify_proposal([guess], draft[None, :], logits, 1.0, 1.0, gen)
        counts[out[0]] += 1
    assert _chi_square(counts, kat["target"], kat["trials"]) < kat["critical_value"]


def test_explicit_uniform_contract_keeps_the_target_distribution():
    """Under the build's Philox + inverse-CDF contract (C oracle), the first token
    after an n-gram guess drawn from the reversed distribution still follows the
    target distribution: accept with p[g], else resample p without g."""
    kat = KATS["rejection_sampling_chi_square"]
    target = np.asarray(kat["target"], dtype=np.float64)
    rows = np.log(target).astype(np.float32)
    bits = oacc.bf16_bits(rows)  # bf16 logits (truncated), as the kernel reads them
    bits = np.stack([bits, bits])
    p_bf16 = np.exp(oacc.bf16_to_f32(bits[0]).astype(np.float64))
    p_bf16 /= p_bf16.sum()
    rng = np.random.default_rng(kat["seed"])
    trials = kat["trials"]
    counts = np.zeros(5)
    for step in range(trials):
        guess = int(rng.choice(5, p=np.asarray(kat["draft"])))
        out = oacc.sampled_accept(bits, [guess], 1.0, seed=12345, step=step)
        counts[out[0]] += 1
    assert _chi_square(counts, p_bf16, trials) < kat["critical_value"]


def test_philox4x32_10_published_vectors():
    # Random123 kat_vectors, philox4x32 with 10 rounds
    kats = [
        ([0, 0, 0, 0], [0, 0], [0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8]),
        ([0xFFFFFFFF] * 4, [0xFFFFFFFF] * 2, [0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD]),
        ([0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344], [0xA4093822, 0x299F31D0],
         [0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1]),
    ]
    for ctr, key, want in kats:
        assert oacc.philox4x32_10(ctr, key) == want


def test_uniform_takes_the_documented_word_and_24_bits():
    seed, step = 0x0123456789ABCDEF, 0x0000000500000007
    for j in (0, 1, 2, 3, 4, 63):
        words = oacc.philox4x32_10([step & 0xFFFFFFFF, step >> 32, j // 4, 0],
                                   [seed & 0xFFFFFFFF, seed >> 32])
        assert oacc.uniform(seed, step, j) == (words[j % 4] >> 8) * 2.0 ** -24


def test_cephes_exp_is_within_two_ulp_of_exp():
    xs = np.linspace(-85.0, 85.0, 3001, dtype=np.float32)
    for x in xs:
        got = oacc.cephes_exp(float(x))
        want = math.exp(float(x))
        assert abs(got - want) <= 2 * 2.0 ** -23 * want
    assert oacc.cephes_exp(0.0) == 1.0
    assert oacc.cephes_exp(-87.0) == 0.0


def test_top_p_reference_kat():
    kat = KATS["top_p"]
    kept = ov.apply_top_p(torch.tensor(kat["probabilities"]), kat["top_p"])
    assert torch.nonzero(kept).flatten().tolist() == kat["expected_nonzero"]
    assert abs(float(kept.sum()) - 1.0) < 1e-6


def test_contract_top_p_reference_kat():
    """The contract's top-p on the KAT's distribution given as bf16 logits log(p)."""
    kat = KATS["top_p"]
    bits = oacc.bf16_bits(np.log(np.asarray(kat["probabilities"], dtype=np.float32)))
    kept, _, _, _ = oacc.top_p_kept(bits, 1.0, kat["top_p"])
    assert np.nonzero(kept)[0].tolist() == kat["expected_nonzero"]


def test_contract_top_p_closed_forms():
    """top_p >= 1 keeps everything with K = Z; a tiny top_p keeps only the first index of
    the largest logit (ties rank by index); K is the kept tokens' chunked total."""
    rng = np.random.default_rng(5)
    for trial in range(50):
        vocab = int(rng.integers(2, 700))
        vals = (rng.standard_normal(vocab) * 2).astype(np.float32)
        if trial % 3 == 0:  # many exact ties
            vals = np.round(vals).astype(np.float32)
        bits = oacc.bf16_bits(vals)
        temp = float(rng.uniform(0.3, 2.0))
        kept_all, k_all, _, _ = oacc.top_p_kept(bits, temp, 1.0)
        assert kept_all.all()
        kept, _, _, _ = oacc.top_p_kept(bits, temp, 1e-7)
        f = oacc.bf16_to_f32(bits)
        assert np.nonzero(kept)[0].tolist() == [int(np.argmax(f))]
        # K: the chunked sum of the kept exps equals a plain fp64 sum of them to fp32 accuracy
        kept9, k9, _, _ = oacc.top_p_kept(bits, temp, 0.9)
        e = np.exp(f.astype(np.float64) / np.float32(temp) - (f / np.float32(temp)).max())
        assert abs(k9 - e[kept9].sum()) <= 1e-5 * e.sum()
        assert abs(k_all - e.sum()) <= 1e-5 * e.sum()


def test_contract_top_p_matches_a_sorted_scan():
    """Brute force: sort by logit (desc), ties by index, and keep a token while the mass
    before it is below top_p * Z (sampling.py:21-27 with the contract's tie order).  Cases
    where some token's mass-before lies within rounding of the threshold are skipped."""
    rng = np.random.default_rng(6)
    checked = 0
    for trial in range(300):
        vocab = int(rng.integers(2, 200))
        vals = (rng.standard_normal(vocab) * float(rng.uniform(0.5, 4))).astype(np.float32)
        if trial % 2:
            vals = (np.round(vals * 2) / 2).astype(np.float32)  # ties
        bits = oacc.bf16_bits(vals)
        f = oacc.bf16_to_f32(bits)
        temp, top_p = float(rng.uniform(0.3, 2.0)), float(rng.uniform(0.05, 0.99))
        z = f.astype(np.float64) / np.float32(temp)
        e = np.exp(z - z.max())
        order = sorted(range(vocab), key=lambda j: (-float(f[j]) + 0.0, j))
        thr = top_p * e.sum()
        before, want, ambiguous = 0.0, np.zeros(vocab, dtype=bool), False
        for j in order:
            if abs(before - thr) < 1e-4 * e.sum():
                ambiguous = True
            want[j] = before < thr
            before += e[j]
        if ambiguous:
            continue
        kept, _, _, _ = oacc.top_p_kept(bits, temp, top_p)
        assert np.array_equal(kept, want), (trial, np.nonzero(kept ^ want))
        checked += 1
    assert checked > 200


def test_contract_top_p_draws_follow_apply_top_p_chi_square():
    """Bonus draws (no guesses) under the contract follow the reference's apply_top_p
    distribution (oracle restatement of sampling.py:21-38) on the same bf16 logits."""
    logits = np.log(np.array([0.3, 0.05, 0.25, 0.15, 0.1, 0.08, 0.07], dtype=np.float32))
    bits = oacc.bf16_bits(logits)[None, :]
    temp, top_p, trials = 0.9, 0.75, 6000
    probs = ov.compute_token_probabilities(torch.from_numpy(oacc.bf16_to_f32(bits[0]).copy()), temp, top_p)
    probs = probs.double().numpy()
    keep = probs > 0
    counts = np.zeros(7)
    for step in range(trials):
        counts[oacc.sampled_accept_v2(bits, [], temp, top_p, seed=99, step=step)[0]] += 1
    assert counts[~keep].sum() == 0
    critical = {2: 13.82, 3: 16.27, 4: 18.47, 5: 20.52}[int(keep.sum()) - 1]  # 0.999 quantiles
    assert _chi_square(counts[keep], probs[keep], trials) < critical


def test_contract_draft_probabilities_keep_the_target_distribution():
    """fp32 draft probabilities used as given (verifier.py:44-56): with the guess drawn from
    q, the first emitted token follows the target p (chi-square, the reference's test
    distributions) and the acceptance rate is sum min(p, q)."""
    kat = KATS["rejection_sampling_chi_square"]
    target = np.asarray(kat["target"], dtype=np.float64)
    q = np.asarray(kat["draft"], dtype=np.float32)
    bits = oacc.bf16_bits(np.log(target).astype(np.float32))
    bits = np.stack([bits, bits])
    p_bf16 = np.exp(oacc.bf16_to_f32(bits[0]).astype(np.float64))
    p_bf16 /= p_bf16.sum()
    rng = np.random.default_rng(kat["seed"])
    trials, counts, kept = kat["trials"], np.zeros(5), 0
    for step in range(trials):
        guess = int(rng.choice(5, p=q.astype(np.float64) / q.astype(np.float64).sum()))
        out = oacc.sampled_accept_v2(bits, [guess], 1.0, 1.0, seed=777, step=step, draft_probs=q[None, :])
        counts[out[0]] += 1
        kept += len(out) == 2
    assert _chi_square(counts, p_bf16, trials) < kat["critical_value"]
    overlap = float(np.minimum(p_bf16, q).sum())
    assert abs(kept / trials - overlap) < 4 * math.sqrt(overlap * (1 - overlap) / trials)


def test_contract_v2_without_top_p_is_the_previous_contract():
    """With top_p = 1 the generalised contract makes the same draws as the one-hot and the
    draft-logit forms (both pinned above) on random rows."""
    rng = np.random.default_rng(8)
    for _ in range(100):
        vocab, g = int(rng.integers(2, 300)), int(rng.integers(0, 5))
        rows = oacc.bf16_bits((rng.standard_normal((g + 1, vocab)) * 3).astype(np.float32))
        drows = oacc.bf16_bits((rng.standard_normal((max(g, 1), vocab)) * 3).astype(np.float32))
        guesses = [int(x) for x in rng.integers(0, vocab, g)]
        temp, seed, step = float(rng.uniform(0.3, 2)), int(rng.integers(0, 2**62)), int(rng.integers(0, 99))
        assert oacc.sampled_accept_v2(rows, guesses, temp, 1.0, seed, step) == oacc.sampled_accept(
            rows, guesses, temp, seed, step)
        assert oacc.sampled_accept_v2(rows, guesses, temp, 1.0, seed, step, draft_bits=drows) == \
            oacc.sampled_accept_draft(rows, drows, guesses, temp, seed, step)


# ---- the integer-mass contract (one-hot guesses; the GPU's sampled n-gram path)
def test_v3_exp_is_within_two_ulp_of_exp():
    for x in np.linspace(-85.0, 20.0, 3001, dtype=np.float32):
        got, want = oacc.exp3(float(x)), math.exp(float(x))
        assert abs(got - want) <= 2 * 2.0 ** -23 * want, float(x)
    assert oacc.exp3(0.0) == 1.0 and oacc.exp3(-87.0) == 0.0


def test_v3_weights_are_the_scaled_softmax_numerators():
    """E(k) / 2^31 equals exp(val(k) / T - max / T) computed in fp64 (to fp32 accuracy plus
    the 2^-31 truncation), E(kmax) = 2^31, and tokens more than ~21.5 T below the largest
    logit weigh 0 -- a wrong sign, a missing 1/T or a wrong maximum fails."""
    rng = np.random.default_rng(31)
    for trial in range(20):
        vocab = int(rng.integers(5, 400))
        vals = (rng.standard_normal(vocab) * float(rng.uniform(0.5, 8))).astype(np.float32)
        bits = oacc.bf16_bits(vals)
        temp = float(rng.uniform(0.2, 2.0))
        keys = oacc.key16(bits)
        f = oacc.bf16_to_f32(bits).astype(np.float64)
        mx = f.max() / np.float32(temp)
        for j in rng.integers(0, vocab, 10).tolist() + [int(np.argmax(f))]:
            e = oacc.v3_weight(bits, temp, int(keys[j]))
            want = math.exp(f[j] / np.float32(temp) - mx)
            # fp32 rounding of z = logit / T and of z - max (relative 2^-24 each) plus the exp's 2 ulp
            tol = 2.0 ** -23 * (abs(f[j] / temp) + abs(mx) + 4)
            assert abs(e / 2.0 ** 31 - want) <= tol * want + 2.0 ** -31, (trial, j)
        assert oacc.v3_weight(bits, temp, int(keys.max())) == 2 ** 31
    bits = oacc.bf16_bits(np.array([0.0, -30.0, -5.0], dtype=np.float32))
    assert oacc.v3_weight(bits, 1.0, int(oacc.key16(bits)[1])) == 0


def test_v3_top_p_reference_kat():
    """sampling.py:21-27 KAT ([.05, .6, .3, .05] at 0.8 keeps [1, 2]) on bf16 logits log(p)."""
    kat = KATS["top_p"]
    bits = oacc.bf16_bits(np.log(np.asarray(kat["probabilities"], dtype=np.float32)))
    kept, _, _, _, _ = oacc.v3_row(bits, 1.0, kat["top_p"])
    assert np.nonzero(kept)[0].tolist() == kat["expected_nonzero"]


def test_v3_top_p_closed_forms():
    """top_p >= 1 keeps everything with K = Z; a tiny top_p keeps only the first index of
    the largest logit (ties rank by index); K is the exact integer sum of the kept weights
    and the smallest such sum reaching top_p * Z."""
    rng = np.random.default_rng(32)
    for trial in range(50):
        vocab = int(rng.integers(2, 700))
        vals = (rng.standard_normal(vocab) * 2).astype(np.float32)
        if trial % 3 == 0:  # many exact ties
            vals = np.round(vals).astype(np.float32)
        bits = oacc.bf16_bits(vals)
        temp = float(rng.uniform(0.3, 2.0))
        kept, k_all, z, _, _ = oacc.v3_row(bits, temp, 1.0)
        assert kept.all() and k_all == z
        kept, _, _, _, _ = oacc.v3_row(bits, temp, 1e-9)
        f = oacc.bf16_to_f32(bits)
        assert np.nonzero(kept)[0].tolist() == [int(np.argmax(f))]
        kept9, k9, z9, tau, m = oacc.v3_row(bits, temp, 0.9)
        keys = oacc.key16(bits)
        w = np.array([oacc.v3_weight(bits, temp, int(k)) for k in keys], dtype=object)
        assert k9 == sum(w[kept9]) and z9 == sum(w)
        thr = max(1, int(float(z9) * float(np.float32(0.9))))
        assert k9 >= thr and k9 - w[np.nonzero(kept9 & (keys == tau))[0][-1]] < thr
        assert int(((keys == tau) & kept9).sum()) == m


def test_v3_top_p_matches_a_sorted_scan():
    """Brute force in fp64: sort by logit (desc), ties by index, keep a token while the mass
    before it is below top_p * Z.  Cases where some token's mass-before lies within
    rounding of the threshold are skipped."""
    rng = np.random.default_rng(33)
    checked = 0
    for trial in range(300):
        vocab = int(rng.integers(2, 200))
        vals = (rng.standard_normal(vocab) * float(rng.uniform(0.5, 4))).astype(np.float32)
        if trial % 2:
            vals = (np.round(vals * 2) / 2).astype(np.float32)
        bits = oacc.bf16_bits(vals)
        f = oacc.bf16_to_f32(bits)
        temp, top_p = float(rng.uniform(0.3, 2.0)), float(rng.uniform(0.05, 0.99))
        z = f.astype(np.float64) / np.float32(temp)
        e = np.exp(z - z.max())
        order = sorted(range(vocab), key=lambda j: (-float(f[j]) + 0.0, j))
        thr = top_p * e.sum()
        before, want, ambiguous = 0.0, np.zeros(vocab, dtype=bool), False
        for j in order:
            if abs(before - thr) < 1e-4 * e.sum():
                ambiguous = True
            want[j] = before < thr
            before += e[j]
        if ambiguous:
            continue
        kept, _, _, _, _ = oacc.v3_row(bits, temp, top_p)
        assert np.array_equal(kept, want), (trial, np.nonzero(kept ^ want))
        checked += 1
    assert checked > 200


def test_v3_top_p_draws_follow_apply_top_p_chi_square():
    """Bonus draws (no guesses) follow the reference's apply_top_p distribution (the
    oracle's restatement of sampling.py:21-38) on the same bf16 logits."""
    logits = np.log(np.array([0.3, 0.05, 0.25, 0.15, 0.1, 0.08, 0.07], dtype=np.float32))
    bits = oacc.bf16_bits(logits)[None, :]
    temp, top_p, trials = 0.9, 0.75, 6000
    probs = ov.compute_token_probabilities(torch.from_numpy(oacc.bf16_to_f32(bits[0]).copy()), temp, top_p)
    probs = probs.double().numpy()
    keep = probs > 0
    counts = np.zeros(7)
    for step in range(trials):
        counts[oacc.sampled_accept_v3(bits, [], temp, top_p, seed=99, step=step)[0]] += 1
    assert counts[~keep].sum() == 0
    critical = {2: 13.82, 3: 16.27, 4: 18.47, 5: 20.52}[int(keep.sum()) - 1]  # 0.999 quantiles
    assert _chi_square(counts[keep], probs[keep], trials) < critical


def test_v3_keeps_the_target_distribution():
    """The reference's chi-square (test_speculative_decoding.py:58-74) for n-gram guesses:
    a guess drawn from the reversed distribution is kept with probability p[g], else the
    token is drawn from p without it -- the first emitted token follows the target p, and
    the acceptance rate is sum_g q[g] p[g]."""
    kat = KATS["rejection_sampling_chi_square"]
    target = np.asarray(kat["target"], dtype=np.float64)
    bits = oacc.bf16_bits(np.log(target).astype(np.float32))
    bits = np.stack([bits, bits])
    p_bf16 = np.exp(oacc.bf16_to_f32(bits[0]).astype(np.float64))
    p_bf16 /= p_bf16.sum()
    q = np.asarray(kat["draft"], dtype=np.float64)
    rng = np.random.default_rng(kat["seed"])
    trials, counts, kept = kat["trials"], np.zeros(5), 0
    for step in range(trials):
        guess = int(rng.choice(5, p=q))
        out = oacc.sampled_accept_v3(bits, [guess], 1.0, 1.0, seed=4242, step=step)
        counts[out[0]] += 1
        kept += len(out) == 2
    assert _chi_square(counts, p_bf16, trials) < kat["critical_value"]
    rate = float((q * p_bf16).sum())
    assert abs(kept / trials - rate) < 4 * math.sqrt(rate * (1 - rate) / trials)


def test_v3_draw_walks_keys_down_then_indices_up():
    """The inverse CDF orders kept tokens by key (descending) then index: as the draw's
    uniform grows the token moves monotonically along that order, and a token holding
    every kept weight with the guess removed is drawn only through the fallback that
    keeps it."""
    vals = np.array([1.0, 3.0, 1.0, 2.0, 3.0, 0.5], dtype=np.float32)
    bits = oacc.bf16_bits(vals)[None, :]
    order = [1, 4, 3, 0, 2, 5]  # key descending, index ascending
    seen = []
    for step in range(4000):
        u = oacc.uniform(5, step, 63)
        seen.append((u, oacc.sampled_accept_v3(bits, [], 0.7, 1.0, seed=5, step=step)[0]))
    seen.sort()
    ranks = [order.index(t) for _, t in seen]
    assert ranks == sorted(ranks) and set(ranks) == set(range(6))
    one = oacc.bf16_bits(np.array([5.0, -200.0], dtype=np.float32))
    rows = np.stack([one, one])
    outs = {tuple(oacc.sampled_accept_v3(rows, [1], 1.0, 1.0, seed=1, step=s)) for s in range(50)}
    assert outs == {(0,)}  # guess 1 weighs 0: rejected, and the draw without it is token 0
    outs = {tuple(oacc.sampled_accept_v3(rows, [0], 1.0, 1.0, seed=1, step=s)) for s in range(50)}
    assert outs == {(0, 0)}  # guess 0 holds all the weight: always kept


# ------------------------------------------------------------------ A7 / A8 int8
def test_quantize_round_trip_reference_kat():
    torch.manual_seed(0)
    x = torch.randn(*KATS["int8_round_trip"]["shape"])
    q, s = oq.quantize_vectors(x)
    assert q.dtype == torch.int8 and s.shape == (6, 4, 1)
    assert torch.all((q.float() * s - x).abs() <= s / 2 + 1e-6)


def test_quantize_closed_form_half_even_and_clamp():
    # absmax 127 -> scale exactly 1.0: codes are round-half-even of the inputs
    x = torch.tensor([[127.0, 0.5, 1.5, 2.5, -0.5, -1.5, -127.0, 3.49]])
    q, s = oq.quantize_vectors(x)
    assert float(s) == 1.0
    assert q.tolist() == [[127, 0, 2, 2, 0, -2, -127, 3]]
    # an all-zero vector takes the 1e-8 floor and all-zero codes
    q0, s0 = oq.quantize_vectors(torch.zeros(1, 4))
    assert q0.abs().sum() == 0 and math.isclose(float(s0), 1e-8 / 127, rel_tol=1e-6)
    # the stored scale is the fp32 scale cast to the input dtype after quantising
    xb = torch.tensor([[3.0, -1.0, 0.3]], dtype=torch.bfloat16)
    qb, sb = oq.quantize_vectors(xb)
    s32 = torch.tensor(3.0) / 127
    assert sb.dtype == torch.bfloat16 and float(sb) == float(s32.to(torch.bfloat16))
    assert qb.tolist() == [[127, -42, 13]]


def test_int8_linear_reference_kat():
    kat = KATS["int8_linear_relative_error"]
    torch.manual_seed(kat["seed"])
    lin = torch.nn.Linear(kat["in_features"], kat["out_features"], bias=False)
    x = torch.randn(kat["rows"], kat["in_features"])
    w8, sc = oq.quantize_linear(lin.weight)
    y = oq.int8_linear(x, w8, sc)
    ref = lin(x)
    assert float((y - ref).norm() / ref.norm()) < kat["max_relative_error"]
    # closed form: dequantise-then-linear equals scaling each output column
    assert torch.allclose(y, (x @ w8.float().t()) * sc[None, :], atol=1e-5)


def test_kv_bytes_per_token_reference_kat():
    kat = KATS["kv_bytes_per_token"]
    assert opg.count_kv_bytes_per_token(28, 8, 128, 2, True) == kat["int8_fp16"]
    assert opg.count_kv_bytes_per_token(28, 8, 128, 2, False) == kat["fp16"]


# ------------------------------------------------------------------ A3 / A4 paging
def test_paged_allocator_growth_reference_kat():
    kat = KATS["paged_allocator_growth"]
    alloc = opg.PagedSlotAllocator(kat["num_blocks"], kat["block_size"])
    for n in kat["reserve"]:
        alloc.reserve("r", n)
    assert alloc.block_table("r") == kat["expected_table"]
    slots = alloc.build_context_slots(["r"], kat["context_length"])
    assert slots.tolist() == kat["expected_slots"]


def test_interleaved_tables_reference_kat():
    kat = KATS["interleaved_tables"]
    alloc = opg.PagedSlotAllocator(kat["num_blocks"], kat["block_size"])
    lengths = [len(p) for p in kat["prompts"]]
    for i, n in enumerate(lengths):
        alloc.reserve(f"r{i}", n)
    for _ in range(kat["steps"]):
        for i in range(len(lengths)):
            lengths[i] += 1
            alloc.reserve(f"r{i}", lengths[i])
    assert [alloc.block_table(f"r{i}") for i in range(2)] == kat["expected_tables"]


def test_step_inputs_pad_to_scratch_and_mask_closed_form():
    alloc = opg.PagedSlotAllocator(8, 4)
    alloc.reserve("a", 6)
    alloc.reserve("b", 3)
    step = opg.build_step_inputs([[1, 2, 3, 4, 5, 6], [7, 8, 9]], [3, 2], [3, 1],
                                 lambda c: alloc.build_context_slots(["a", "b"], c), scratch_slot=32)
    assert step.token_ids.tolist() == [[4, 5, 6], [9, 0, 0]]
    assert step.positions.tolist() == [[3, 4, 5], [2, 0, 0]]
    assert step.slot_mapping.tolist() == [[3, 4, 5], [10, 32, 32]]  # b's table is [2]
    # query at position p sees keys 0..p, and nothing past the sequence end
    m = step.attention_mask[:, 0]
    assert m[0].tolist()[2] == [True] * 6 and m[0].tolist()[0] == [True] * 4 + [False] * 2
    assert m[1].tolist()[0] == [True, True, True, False, False, False]


# ------------------------------------------------------------------ A5 / A6 model + attention
def test_rotate_half_and_rope_identity_at_zero():
    kat = KATS["rotate_half"]
    assert om.rotate_half(torch.tensor(kat["input"])).tolist() == kat["expected"]
    cos, sin = om.build_rotary_tables(torch.zeros(1, 3, dtype=torch.long), 8, 1e4, torch.float32)
    x = torch.randn(1, 2, 3, 8)
    assert torch.equal(om.apply_rotary_embedding(x, cos, sin), x)


@pytest.mark.parametrize("kv", ["bf16", "int8"])
def test_paged_attention_reference_against_textbook_fp64(kv):
    g = torch.Generator().manual_seed(3)
    bs, blocks, hkv, hq, d = 16, 6, 2, 4, 128
    slots = blocks * bs + 1
    k = torch.randn(slots, hkv, d, generator=g).to(torch.bfloat16)
    v = torch.randn(slots, hkv, d, generator=g).to(torch.bfloat16)
    if kv == "int8":
        kq, ks = oq.quantize_vectors(k)
        vq, vs = oq.quantize_vectors(v)
        kc, vc, ksc, vsc = kq, vq, ks[..., 0], vs[..., 0]
        kd = (kq.to(torch.bfloat16) * ks).float()
        vd = (vq.to(torch.bfloat16) * vs).float()
    else:
        kc, vc, ksc, vsc = k, v, None, None
        kd, vd = k.float(), v.float()
    tables = torch.tensor([[4, 1, 5], [0, 2, 3]], dtype=torch.int32)
    ctx = torch.tensor([37, 20], dtype=torch.int32)
    ql = torch.tensor([3, 2], dtype=torch.int32)
    qs = torch.tensor([0, 3], dtype=torch.int32)
    q = torch.randn(5, hq, d, generator=g).to(torch.bfloat16)
    got = oatt.paged_attention_reference(q, kc, vc, ksc, vsc, tables, bs, ctx, qs, ql)
    for b in range(2):
        pos = torch.arange(int(ctx[b]))
        sl = tables[b][pos // bs].long() * bs + pos % bs
        qpos = int(ctx[b]) - int(ql[b]) + np.arange(int(ql[b]))
        want = oatt.textbook_attention_fp64(q[int(qs[b]):int(qs[b]) + int(ql[b])].float().numpy(),
                                            kd[sl].numpy(), vd[sl].numpy(), qpos, 1 / math.sqrt(d))
        np.testing.assert_allclose(got[int(qs[b]):int(qs[b]) + int(ql[b])].numpy(), want, rtol=1e-4, atol=1e-5)


TINY = om.Qwen3Config(vocab_size=64, hidden_size=32, intermediate_size=64, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2, head_dim=16, rms_norm_eps=1e-6,
                      rope_theta=1e4, tie_word_embeddings=True)


def test_contiguous_allocator_reference_kat():
    """nt/engine/test_memory_allocators.py:34-49: one whole region per sequence, refusals
    for a third sequence and an over-long reservation, reuse after a free, contiguous
    context slots starting at a region boundary."""
    kat = KATS["contiguous_allocator"]
    alloc = opg.ContiguousSlotAllocator(kat["num_regions"], kat["region_length"])
    for rid, n in kat["reserve"]:
        alloc.reserve(rid, n)
    assert alloc.num_reserved_slots == kat["expected_reserved_slots"]
    for rid, n in kat["refused"]:
        assert not alloc.can_reserve(rid, n)
    with pytest.raises(opg.OutOfKVMemoryError):
        alloc.reserve(*kat["refused"][0])
    alloc.free(kat["free"])
    assert alloc.can_reserve(*kat["accepted_after_free"])
    rid, c = kat["context"]
    slots = alloc.build_context_slots([rid], c).tolist()[0]
    assert slots == list(range(slots[0], slots[0] + c))
    assert slots[0] % kat["region_start_multiple"] == 0
    # closed form of the region order (contiguous_allocator.py:17, 36-38): regions are
    # handed out from the low end, so the second sequence holds region 1
    assert slots[0] == kat["region_length"]
    alloc.reserve("c", 1)
    assert alloc.build_context_slots(["c"], 2).tolist() == [[0, 1]]


def test_find_finish_reason_closed_form():
    """sampling.py:54-62: stop on a stop token unless ignore_eos; length at the limit."""
    stops = frozenset({7})
    assert ov.find_finish_reason(7, 1, 12, False, stops) == "stop"
    assert ov.find_finish_reason(7, 1, 12, True, stops) is None
    assert ov.find_finish_reason(7, 12, 12, True, stops) == "length"
    assert ov.find_finish_reason(3, 12, 12, False, stops) == "length"
    assert ov.find_finish_reason(3, 11, 12, False, stops) is None


def _tiny_from_kat(m):
    cfg = om.Qwen3Config(m["vocab_size"], m["hidden_size"], m["intermediate_size"], m["num_hidden_layers"],
                         m["num_attention_heads"], m["num_key_value_heads"], m["head_dim"], m["rms_norm_eps"],
                         m["rope_theta"], True)
    return cfg, om.build_random_model(cfg, seed=m["seed"], std=m["std"])


def test_speculative_stop_token_reference_kat():
    """nt/engine/test_speculative_decoding.py:100-112: on a paged cache, a stop token (the
    4th greedy token of a non-speculative full-recompute decode) ends the speculative
    request with finish reason "stop" after at most 4 events; the tokens up to it equal
    that greedy decode's."""
    kat = KATS["speculative_stop_token"]
    cfg, model = _tiny_from_kat(kat["model"])
    prompt = kat["prompt"]
    ids, greedy = list(prompt), []
    with torch.no_grad():  # NaiveGenerator: full recompute per token
        for _ in range(kat["greedy_reference_new_tokens"]):
            tok = int(torch.argmax(model.compute_logits(model(torch.tensor([ids])))[0, -1]))
            greedy.append(tok)
            ids.append(tok)
    stop = greedy[kat["stop_token_greedy_index"]]
    bs = kat["kv_block_size"]
    runner = ov.ModelRunner(model, om.KVCachePool(cfg, 64, torch.float32), opg.PagedSlotAllocator(64 // bs, bs))
    seq = ov.Sequence("stop", list(prompt), len(prompt), kat["max_new_tokens"], ignore_eos=False)
    stats = ov.SpeculativeStats()
    out = ov.generate_speculative(runner, seq, kat["num_speculative_tokens"], kat["ngram_max_size"],
                                  frozenset({stop}), stats)
    assert stats.finish_reason == kat["expected_finish_reason"] and out[-1] == stop
    assert len(out) <= kat["max_events"]
    assert out == greedy[: greedy.index(stop) + 1]
    assert runner.allocator.num_reserved_slots == 0  # the finished request's blocks are freed


def test_model_matches_transformers_qwen3():
    """An independent Qwen3 (Hugging Face transformers) with the same weights: logits 1e-4
    (the reference's own twin test, nt/models/test_qwen3_model.py:17-49)."""
    transformers = pytest.importorskip("transformers")
    model = om.build_random_model(TINY, seed=7, std=0.5)
    cfg = transformers.Qwen3Config(vocab_size=64, hidden_size=32, intermediate_size=64, num_hidden_layers=2,
                                   num_attention_heads=4, num_key_value_heads=2, head_dim=16,
                                   rms_norm_eps=1e-6, rope_theta=1e4, tie_word_embeddings=True,
                                   max_position_embeddings=128, attention_bias=False)
    hf = transformers.Qwen3ForCausalLM(cfg).eval()
    missing = hf.load_state_dict(model.state_dict(), strict=False)
    assert not [k for k in missing.missing_keys if k != "lm_head.weight"]
    ids = torch.randint(0, 64, (1, 12), generator=torch.Generator().manual_seed(1))
    with torch.no_grad():
        ours = model.compute_logits(model(ids))
        theirs = hf(ids).logits
    assert torch.allclose(ours, theirs, atol=1e-4)


def test_cached_paged_forward_equals_full_recompute():
    """nt/engine/test_kv_cache.py:78-90: logits of a paged, cached forward == recompute."""
    model = om.build_random_model(TINY, seed=7, std=0.5)
    pool = om.KVCachePool(TINY, 64, torch.float32)
    alloc = opg.PagedSlotAllocator(16, 4)
    seq = ov.Sequence("s", [3, 9, 27, 1, 5, 6, 2], 7, 20)
    runner = ov.ModelRunner(model, pool, alloc)
    alloc.reserve("s", 7)
    runner.run_step([seq])
    seq.token_ids += [11, 12, 13]
    alloc.reserve("s", 10)
    cached = runner.score_tokens(seq, 3)  # positions 7..9, the three uncached tokens
    with torch.no_grad():
        full = model.compute_logits(model(torch.tensor([seq.token_ids])))[0, 7:10]
    assert torch.allclose(cached, full, atol=1e-5)


@pytest.mark.parametrize("kv_int8", [False, True])
def test_speculative_output_equals_the_target_alone(kv_int8):
    """nt/engine/test_speculative_decoding.py:77-97 for the n-gram proposer: the serial
    speculative loop emits exactly the non-speculative greedy tokens."""
    model = om.build_random_model(TINY, seed=7, std=0.5)
    prompt = [5, 6, 7, 5, 6, 7, 5, 6]
    pool = om.KVCachePool(TINY, 128, torch.float32, is_int8=kv_int8)
    runner = ov.ModelRunner(model, pool, opg.PagedSlotAllocator(32, 4))
    stats = ov.SpeculativeStats()
    seq = ov.Sequence("s", list(prompt), len(prompt), 16)
    spec = ov.generate_speculative(runner, seq, 3, 2, stats=stats)
    pool2 = om.KVCachePool(TINY, 128, torch.float32, is_int8=kv_int8)
    runner2 = ov.ModelRunner(model, pool2, opg.PagedSlotAllocator(32, 4))
    seq2 = ov.Sequence("t", list(prompt), len(prompt), 16)
    runner2.allocator.reserve("t", len(prompt))
    plain = []
    for _ in range(16):
        tok = runner2.run_step([seq2])[0]
        seq2.token_ids.append(tok)
        plain.append(tok)
        runner2.allocator.reserve("t", len(seq2.token_ids))
    assert spec == plain
    assert 0 <= stats.accepted <= stats.proposed and stats.proposed > 0


def test_draft_proposals_equal_a_cached_greedy_decode():
    """oracle.draft.propose (full forwards) against the oracle's cached ModelRunner path
    (paged KV, one scored token per step) on the same tiny draft model; a shorter
    proposal is a prefix of a longer one (proposers.py:70-88 appends each guess)."""
    from oracle import draft as odr

    cfg = om.Qwen3Config(97, 64, 128, 2, 4, 2, 16, 1e-6, 1e4, True)
    model = om.build_random_model(cfg, seed=11, std=0.3)
    prompt = [5, 17, 3, 88, 41, 5, 17, 3]
    guesses = odr.propose(model, prompt, 6)
    assert odr.propose(model, prompt, 3) == guesses[:3]
    runner = ov.ModelRunner(model, om.KVCachePool(cfg, 64, torch.float32), opg.PagedSlotAllocator(4, 16))
    seq = ov.Sequence("d", list(prompt), len(prompt), 6)
    decoded = []
    for _ in range(6):
        runner.allocator.reserve(seq.request_id, len(seq.token_ids))
        token = runner.run_step([seq])[0]
        seq.token_ids.append(token)
        decoded.append(token)
    assert decoded == guesses
    rows = odr.draft_logits(model, prompt, guesses)
    assert rows.shape == (6, 97)
    assert [int(r.argmax()) for r in rows] == guesses


def test_draft_distribution_rule_keeps_the_target_distribution():
    """nt/engine/test_speculative_decoding.py:58-75 under the explicit-uniform contract
    (C oracle): the guess is drawn from the draft's own distribution q, the rule keeps it
    with min(1, p/q) and otherwise draws from max(p - q, 0); the first token then
    follows the target distribution p."""
    kat = KATS["rejection_sampling_chi_square"]
    target = np.asarray(kat["target"], dtype=np.float64)
    draft = np.asarray(kat["draft"], dtype=np.float64)
    bits = oacc.bf16_bits(np.log(target).astype(np.float32))
    bits = np.stack([bits, bits])
    dbits = oacc.bf16_bits(np.log(draft).astype(np.float32))[None, :]
    p_bf16 = np.exp(oacc.bf16_to_f32(bits[0]).astype(np.float64))
    p_bf16 /= p_bf16.sum()
    q_bf16 = np.exp(oacc.bf16_to_f32(dbits[0]).astype(np.float64))
    q_bf16 /= q_bf16.sum()
    rng = np.random.default_rng(kat["seed"])
    trials = kat["trials"]
    counts = np.zeros(5)
    kept = 0
    for step in range(trials):
        guess = int(rng.choice(5, p=q_bf16))
        out = oacc.sampled_accept_draft(bits, dbits, [guess], 1.0, seed=12345, step=step)
        counts[out[0]] += 1
        kept += len(out) == 2
    assert _chi_square(counts, p_bf16, trials) < kat["critical_value"]
    # acceptance rate sum_g min(p_g, q_g) (the overlap of the two distributions)
    overlap = float(np.minimum(p_bf16, q_bf16).sum())
    assert abs(kept / trials - overlap) < 4 * math.sqrt(overlap * (1 - overlap) / trials)


def test_draft_distribution_rule_equal_distributions_keep_every_guess():
    """q = p: min(1, p/q) = 1 for every guess (no uniform is consulted)."""
    rng = np.random.default_rng(3)
    bits = oacc.bf16_bits(rng.standard_normal((4, 50)).astype(np.float32))
    for trial in range(20):
        guesses = [int(x) for x in rng.integers(0, 50, 3)]
        out = oacc.sampled_accept_draft(bits, bits[:3], guesses, 0.7, seed=trial, step=trial)
        assert out[:3] == guesses and len(out) == 4
