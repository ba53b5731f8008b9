"""Pins the oracle's sampler/acceptance math (sampler.rs, speculative.rs) with the
reference's own KATs plus closed forms."""
import numpy as np
import pytest

import refcpu as R


def test_greedy_is_deterministic():  # sampler.rs:353-359
    s = R.sampler(greedy=True)
    assert R.argmax([0.1, 4.0, 1.0]) == 1
    rng = R.Rng(0)
    p = R.probabilities(s, [0.1, 4.0, 1.0])
    assert R.sample_probabilities(s, rng, p) == 1
    assert rng.pos == 0  # greedy consumes no draws (sampler.rs:157-162)


def test_argmax_takes_last_index_on_ties():  # sampler.rs:217-224 (F9)
    assert R.argmax([1.0, 3.0, 3.0, 2.0]) == 2
    assert R.argmax([0.0] * 7) == 6
    assert R.argmax([-0.0, 0.0, -0.0]) == 1  # total_cmp: -0 < +0
    assert R.argmax([1.0, float("nan"), 2.0]) == 1  # NaN ranks highest under total_cmp


def test_top_k_excludes_lower_ranked_tokens():  # sampler.rs:361-376
    s = R.sampler(temperature=1.0, top_k=2)
    p = R.probabilities(s, [10.0, 9.0, 8.0, 7.0])
    assert p[0] > 0 and p[1] > 0 and p[2] == 0.0 and p[3] == 0.0


def test_temperature_zero_returns_argmax():  # sampler.rs:378-382
    s = R.sampler(temperature=0.0, top_k=1, top_p=0.1)
    assert R.lib().ref_is_deterministic(s)
    assert list(R.probabilities(s, [1.0, 2.0, 3.0])) == [0.0, 0.0, 1.0]


def test_probabilities_match_sampling_filters():  # sampler.rs:396-402
    s = R.sampler(temperature=1.0, top_k=2)
    p = R.probabilities(s, [10.0, 9.0, 8.0])
    assert p[2] == 0.0 and abs(p.sum() - 1.0) < 1e-6


def test_deterministic_probabilities_are_one_hot():  # sampler.rs:404-411
    assert list(R.probabilities(R.sampler(greedy=True), [1.0, 3.0, 2.0])) == [0.0, 1.0, 0.0]


def test_softmax_matches_float64_closed_form():
    rng = np.random.default_rng(0)
    for T in (0.7, 1.0, 1.3):
        logits = rng.normal(0, 3, 4096).astype(np.float32)
        p = R.probabilities(R.sampler(temperature=T), logits)
        z = logits.astype(np.float64) / T
        ref = np.exp(z - z.max())
        ref /= ref.sum()
        assert np.max(np.abs(p - ref)) < 1e-6
        assert abs(float(p.astype(np.float64).sum()) - 1.0) < 1e-5


def test_top_p_keeps_smallest_prefix_reaching_mass():
    s = R.sampler(temperature=1.0, top_p=0.8)
    logits = np.log(np.array([0.5, 0.3, 0.15, 0.05], np.float32))
    p = R.probabilities(s, logits)
    assert p[2] == 0.0 and p[3] == 0.0
    np.testing.assert_allclose(p[:2], [0.625, 0.375], atol=1e-6)


def test_non_finite_logits_are_excluded():
    p = R.probabilities(R.sampler(temperature=1.0), [0.0, float("-inf"), 0.0])
    assert list(p) == [0.5, 0.0, 0.5]
    with pytest.raises(ValueError):
        R.probabilities(R.sampler(temperature=1.0), [float("-inf")] * 3)


def test_residual_is_positive_difference_normalized():  # speculative.rs:906-912
    r = R.residual([0.1, 0.2, 0.7], [0.6, 0.3, 0.1])
    assert r[0] == 0.0 and r[1] == 0.0 and abs(r[2] - 1.0) < 1e-6


def test_residual_zero_mass_is_an_error():  # speculative.rs:784-788
    with pytest.raises(ValueError):
        R.residual([0.25, 0.75], [0.25, 0.75])


def test_deterministic_acceptance_requires_matching_argmax():  # speculative.rs:914-919
    s = R.sampler(greedy=True)
    rng = R.Rng(0)
    assert R.accept_proposal(s, rng, 1, [0.0, 1.0], [0.0, 1.0])
    assert not R.accept_proposal(s, rng, 1, [0.0, 1.0], [1.0, 0.0])


def test_full_rejection_uses_target_residual():  # speculative.rs:952-960
    draft, target = [1.0, 0.0], [0.0, 1.0]
    r = R.residual(target, draft)
    s = R.sampler(temperature=1.0)
    rng = R.Rng(9)
    assert not R.accept_proposal(s, rng, 0, draft, target)
    assert R.sample_probabilities(s, rng, r) == 1


def test_acceptance_draws_only_when_draft_mass_is_positive():  # speculative.rs:764-767
    s = R.sampler(temperature=1.0)
    rng = R.Rng(3)
    assert not R.accept_proposal(s, rng, 0, [0.0, 1.0], [1.0, 0.0])
    assert rng.pos == 0
    R.accept_proposal(s, rng, 1, [0.0, 1.0], [1.0, 0.0])
    assert rng.pos == 1


def test_sampled_speculation_matches_target_distribution():  # speculative.rs:926-950
    target = np.array([0.1, 0.2, 0.7], np.float32)
    draft = np.array([0.6, 0.3, 0.1], np.float32)
    s = R.sampler(temperature=1.0)
    rng = R.Rng(7)
    res = R.residual(target, draft)
    counts = np.zeros(3)
    n = 50000
    for _ in range(n):
        prop = R.sample_probabilities(s, rng, draft)
        tok = prop if R.accept_proposal(s, rng, prop, draft, target) else R.sample_probabilities(s, rng, res)
        counts[tok] += 1
    assert np.max(np.abs(counts / n - target)) < 0.01


def test_inverse_cdf_uses_draw_le_cumulative():  # sampler.rs:337-347
    # Brute force over the 2^24 grid is too big; check the boundary rule on a
    # distribution whose cumulative sums are exact binary fractions.
    s = R.sampler(temperature=1.0)
    p = np.array([0.25, 0.25, 0.5], np.float32)
    seen = set()
    rng = R.Rng(11)
    for _ in range(2000):
        pos = rng.pos
        u = R.Rng(11, pos).next_f32()
        tok = R.sample_probabilities(s, rng, p)
        want = 0 if u <= 0.25 else (1 if u <= 0.5 else 2)
        assert tok == want
        seen.add(tok)
    assert seen == {0, 1, 2}


def test_accept_batch_matches_sequential_functions():
    rng0 = np.random.default_rng(5)
    B, K, V = 6, 3, 50
    tgt = rng0.normal(0, 2, (B, K + 1, V)).astype(np.float32)
    dft = (tgt[:, :K] + rng0.normal(0, 1, (B, K, V))).astype(np.float32)
    toks = rng0.integers(0, V, (B, K)).astype(np.uint32)
    s = R.sampler(temperature=0.8)
    seeds = np.arange(B, dtype=np.uint64) + 100
    out = R.accept_batch(tgt, dft, toks, s, bonus=True, seeds=seeds)
    for b in range(B):
        rng = R.Rng(int(seeds[b]))
        n_acc, token = 0, -1
        for i in range(K):
            p = R.probabilities(s, tgt[b, i])
            q = R.probabilities(s, dft[b, i])
            if R.accept_proposal(s, rng, int(toks[b, i]), q, p):
                n_acc += 1
                continue
            token = R.sample_probabilities(s, rng, R.residual(p, q))
            break
        else:
            token = R.sample_probabilities(s, rng, R.probabilities(s, tgt[b, K]))
        assert out["accept_len"][b] == n_acc and out["token"][b] == token
        assert out["draws"][b] == rng.pos


def test_accept_batch_explicit_uniforms_equal_stream():
    rng0 = np.random.default_rng(6)
    B, K, V = 4, 4, 64
    tgt = rng0.normal(0, 3, (B, K + 1, V)).astype(np.float32)
    dft = (tgt[:, :K] + rng0.normal(0, 1, (B, K, V))).astype(np.float32)
    toks = rng0.integers(0, V, (B, K)).astype(np.uint32)
    s = R.sampler(temperature=0.8)
    seeds = np.arange(B, dtype=np.uint64)
    a = R.accept_batch(tgt, dft, toks, s, bonus=True, seeds=seeds)
    uni = np.array([[R.Rng(int(seeds[b]), i).next_f32() for i in range(K + 1)] for b in range(B)], np.float32)
    b_ = R.accept_batch(tgt, dft, toks, s, bonus=True, uniforms=uni)
    assert np.array_equal(a["accept_len"], b_["accept_len"]) and np.array_equal(a["token"], b_["token"])


def test_top_k_ties_keep_lower_indices():
    """Stable sort (slice::sort_by is stable): equal logits at the boundary keep the
    lower token ids (sampler.rs:238-245)."""
    s = R.sampler(temperature=1.0, top_k=2)
    p, _, gap = R.probabilities(s, [1.0, 3.0, 3.0, 3.0, 2.0], margins=True)
    assert p[1] == p[2] == np.float32(0.5) and p[0] == p[3] == p[4] == 0.0
    assert gap == 0.0  # the 2nd and 3rd ranked logits tie
    s = R.sampler(temperature=1.0, top_k=3)
    p = R.probabilities(s, [float("nan"), 5.0, 4.0, 3.0])
    # NaN ranks highest under total_cmp and takes a top-k slot, but softmax drops it (non-finite)
    assert p[0] == 0.0 and p[3] == 0.0 and p[1] > p[2] > 0.0


def test_top_p_ties_and_exact_boundary():
    """Equal probabilities are ranked by ascending index; the cumulative sum stops at
    the first element with cumulative >= top_p (sampler.rs:268-275)."""
    s = R.sampler(temperature=1.0, top_p=0.5)
    p, margin, _ = R.probabilities(s, np.zeros(4, np.float32), margins=True)
    assert list(p) == [0.5, 0.5, 0.0, 0.0]  # 0.25 + 0.25 == 0.5 exactly
    assert margin == 0.0


def test_top_p_against_stable_sort_brute_force():
    """filtered_probs top-p against numpy's stable argsort and float32 sequential
    cumsum (np.cumsum accumulates left to right in the requested dtype)."""
    rng = np.random.default_rng(3)
    for trial in range(20):
        V = int(rng.integers(2, 3000))
        logits = (rng.normal(0, rng.choice([0.3, 3.0]), V)).astype(np.float32)
        if trial % 4 == 0:
            logits = np.round(logits)  # many exact ties
        top_p = float(rng.choice([0.3, 0.8, 0.9, 0.99]))
        s = R.sampler(temperature=0.7, top_p=top_p)
        p0 = R.probabilities(R.sampler(temperature=0.7), logits)
        order = np.argsort(-p0, kind="stable")
        cum = np.cumsum(p0[order], dtype=np.float32)
        hit = np.nonzero(cum >= np.float32(top_p))[0]
        n_keep = int(hit[0]) + 1 if hit.size else V
        keep = np.zeros(V, bool)
        keep[order[:n_keep]] = True
        kept = np.where(keep, p0, np.float32(0))
        tot = np.float32(0)
        for v in kept:
            tot = np.float32(tot + v)
        want = (kept / tot).astype(np.float32)
        got, margin, _ = R.probabilities(s, logits, margins=True)
        assert np.array_equal(got, want), trial
        if hit.size:
            prev = cum[hit[0] - 1] if hit[0] > 0 else np.float32(0)
            assert margin == min(cum[hit[0]] - np.float32(top_p), np.float32(top_p) - prev)
