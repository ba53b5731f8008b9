"""Pins the oracle's Sampler::top_candidates_from_probabilities (sampler.rs:188-208):
a stable descending sort truncated to n, and the engines' per-token candidate
record (mtp_speculative.rs:247-250, engine.rs:70 top_candidates = 5)."""
import numpy as np

import refcpu as R


def test_reference_kat_sorted():  # sampler.rs:384-394
    p = R.probabilities(R.sampler(temperature=1.0), np.array([1.0, 3.0, 2.0], np.float32))
    ids, probs = R.top_candidates(p, 3)
    assert ids.tolist() == [1, 2, 0]
    assert (np.diff(probs) <= 0).all()
    assert np.allclose(probs, np.exp([3, 2, 1]) / np.exp([1, 2, 3]).sum(), rtol=1e-6)


def test_ties_keep_ascending_token_order():
    ids, probs = R.top_candidates(np.array([0.1, 0.3, 0.3, 0.2, 0.1], np.float32), 5)
    assert ids.tolist() == [1, 2, 3, 0, 4]
    assert probs.tolist() == np.float32([0.3, 0.3, 0.2, 0.1, 0.1]).tolist()


def test_matches_stable_argsort_with_many_ties():
    rng = np.random.default_rng(3)
    for trial in range(20):
        p = (rng.integers(0, 7, 300) / 7.0).astype(np.float32)
        want = np.argsort(-p, kind="stable")[:5]
        ids, probs = R.top_candidates(p, 5)
        assert ids.tolist() == want.tolist()
        assert np.array_equal(probs, p[want])


def test_short_distribution_pads():
    ids, probs = R.top_candidates(np.array([0.25, 0.75], np.float32), 5)
    assert ids[:2].tolist() == [1, 0] and (ids[2:] == 0xFFFFFFFF).all() and (probs[2:] == 0).all()


def test_engine_records_one_hot_candidates_per_committed_token():
    """Greedy distributions are one-hot at the argmax: the committed token leads with
    probability 1, then the four lowest other ids at 0 (stable order)."""
    kw = dict(vocab_size=256, hidden_dim=128, ffn_dim=256, n_layers=1, n_heads=2, n_kv_heads=1, max_seq_len=64,
              num_future_tokens=3)
    rc = R.make_config(**kw)
    m = R.Model(rc)
    for i, (name, r, c, kind) in enumerate(m.tensors()):
        m.set(i, R.synth_fill(4, i, r * c, 0.3) if kind != R.T_NORM else np.ones(r * c, np.float32))
    toks, _, _, _ = m.mtp_generate(np.arange(1, 6, dtype=np.uint32), 12, 3, R.sampler(greedy=True))
    ids, probs = m.last_candidates
    assert len(ids) == len(toks) == 12
    for t, ci, cp in zip(toks, ids, probs):
        assert ci[0] == t and cp.tolist() == [1.0, 0.0, 0.0, 0.0, 0.0]
        assert ci[1:].tolist() == [j for j in range(6) if j != t][:4]
