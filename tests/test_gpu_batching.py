"""Continuous batching with speculative rounds (the serving worker's loop,
serve/src/batching.rs:324-445, with decode_sessions, inference/src/engine.rs:323-355,
replaced by MTP rounds) on the device, against the oracle engine run one request at a
time (mtp_speculative.rs:86-336).  Requests of ragged prompt lengths and token budgets
join free rows between rounds, leave when they finish or are cancelled, and their rows
and KV slots are reused: every completed request must equal the oracle's stand-alone
run of it (tokens, finish reason, statistics, top candidates)."""
import numpy as np
import pytest

import aarambh_hip as A
import refcpu as R
from gpu_util import first_divergent_round, make_pair, prob_margin

pytestmark = pytest.mark.gpu

KW = dict(vocab_size=1024, hidden_dim=256, ffn_dim=512, n_layers=2, n_heads=4, n_kv_heads=2, max_seq_len=128,
          num_future_tokens=3)
STAT_KEYS = ("rounds", "draft_tokens_proposed", "draft_tokens_accepted", "target_decode_forwards",
             "mtp_head_forwards")


def _collect(events):
    deltas, done, failed = {}, {}, {}
    for ev in events:
        if ev[0] == "delta":
            deltas.setdefault(ev[1], []).extend(ev[2])
        elif ev[0] == "completed":
            assert ev[1] not in done
            done[ev[1]] = ev[2]
        else:
            failed[ev[1]] = ev[2]
    return deltas, done, failed


def test_continuous_batching_greedy_matches_oracle():
    ref, hip = make_pair(seed=8, std=0.3, max_batch=3, max_rows=64, **KW)
    g = R.sampler(greedy=True)
    # (prompt length, token budget): ragged; the 100-token prompt runs into the context
    # limit (128 - 100 = 28 < 40)
    shapes = [(5, 20), (17, 8), (9, 35), (30, 14), (12, 25), (3, 40), (21, 11), (100, 40), (7, 30)]
    reqs, want = [], []
    ps = 0
    for plen, budget in shapes:
        while True:  # prompts whose greedy run has no near-tie (top-2 gap above the f32 bar)
            prompt = R.synth_tokens(8, 100 + ps, plen, 1024)
            ps += 1
            w, fin, stats, gap = ref.mtp_generate(prompt, budget, 3, g)
            if gap > 1e-5:
                break
        reqs.append(A.GenerationRequest(prompt, budget, seed=0))
        want.append((list(w), A.FINISH[fin], stats, ref.last_candidates))
    assert want[7][1] == "ContextLimit"
    eng = A.MtpSpeculativeEngine(hip, A.SpeculativeConfig(3))
    bat = A.SpeculativeBatcher(eng, A.BatcherConfig(max_batch_size=3, queue_capacity=16, prefill_chunk_size=8),
                               A.Sampler.greedy_sampler())
    ids = [bat.submit(r) for r in reqs[:4]]
    # a prompt at the context limit fails at admission and takes no row (admit_job)
    bad = bat.submit(A.GenerationRequest(np.ones(128, np.uint32), 4))
    events = bat.step() + bat.step()
    assert len(bat.active) == 3
    ids += [bat.submit(r) for r in reqs[4:]]
    # a cancelled request leaves at the next step; its row is reused
    victim = bat.submit(A.GenerationRequest(R.synth_tokens(8, 999, 10, 1024), 60))
    for _ in range(200):
        if any(e[0] == "delta" and e[1] == victim for e in events):
            break
        events += bat.step()
    bat.cancel(victim)
    events += bat.run()
    deltas, done, failed = _collect(events)
    assert set(failed) == {bad} and "max_seq_len" in failed[bad]
    assert victim not in done and victim in deltas
    assert set(done) == set(ids)
    for rid, (w, fin, stats, (ci, cp)) in zip(ids, want):
        out = done[rid]
        assert [int(t) for t in out.token_ids] == w, rid
        assert deltas.get(rid, []) == w
        assert out.finish_reason == fin, (rid, out.finish_reason, fin)
        for k in STAT_KEYS:
            assert getattr(out.speculative_stats, k) == stats[k], (rid, k)
        assert [[i for i, _ in c] for c in out.candidates] == ci.tolist()
        np.testing.assert_allclose([[p for _, p in c] for c in out.candidates], cp, rtol=0, atol=1e-6)
    assert not bat.active and (bat.session.rows() == A.ContinuousSession.FREE).all()
    bat.close()
    hip.close()


def test_continuous_batching_sampled_matches_oracle():
    """Sampled rounds (reference CLI default sampler T 0.7, top-k 50, top-p 0.9) with a
    seed per request: a request admitted into a reused row starts its own keystream.
    Each completed request equals the oracle's run of it, or departs from it first in a
    round the oracle marks as a near-tie."""
    ref, hip = make_pair(seed=31, std=0.3, max_batch=2, max_rows=64, **KW)
    s_ref = R.sampler(temperature=0.7, top_k=50, top_p=0.9)
    s_dev = A.Sampler.top_k_top_p(0.7, top_k=50, top_p=0.9)
    shapes = [(12, 30), (5, 18), (20, 26), (9, 12), (15, 34)]
    reqs = [A.GenerationRequest(R.synth_tokens(31, 50 + i, p, 1024), n, seed=1000 + 17 * i)
            for i, (p, n) in enumerate(shapes)]
    tol_p = prob_margin([(ref, hip)], reqs[0].prompt_ids, 0.7)
    assert tol_p < 5e-3, tol_p
    eng = A.MtpSpeculativeEngine(hip, A.SpeculativeConfig(3))
    bat = A.SpeculativeBatcher(eng, A.BatcherConfig(max_batch_size=2), s_dev)
    ids = [bat.submit(r) for r in reqs]
    _, done, failed = _collect(bat.run())
    assert not failed and set(done) == set(ids)
    same = 0
    for rid, r in zip(ids, reqs):
        w, fin, stats, _ = ref.mtp_generate(r.prompt_ids, r.max_new_tokens, 3, s_ref, seed=r.seed)
        got = [int(t) for t in done[rid].token_ids]
        d = first_divergent_round(ref.last_rounds, w, got)
        if d is None:
            same += 1
            assert done[rid].finish_reason == A.FINISH[fin]
            for k in STAT_KEYS:
                assert getattr(done[rid].speculative_stats, k) == stats[k], (rid, k)
            continue
        rd = ref.last_rounds[d]
        assert rd["prob_margin"] < tol_p or rd["logit_gap"] < 1e-4, (rid, d, rd)
    assert same >= 4, same
    bat.close()
    hip.close()


def test_session_rows_admit_retire_validation():
    ref, hip = make_pair(seed=3, max_batch=2, max_rows=64, **KW)
    eng = A.MtpSpeculativeEngine(hip, A.SpeculativeConfig(3))
    with pytest.raises(A.ConfigError):
        A.SpeculativeBatcher(eng, A.BatcherConfig(max_batch_size=0), A.Sampler.greedy_sampler())
    bat = A.SpeculativeBatcher(eng, A.BatcherConfig(max_batch_size=2, queue_capacity=2),
                               A.Sampler.greedy_sampler())
    bat.submit(A.GenerationRequest([1, 2, 3], 4))
    bat.submit(A.GenerationRequest([1, 2, 3], 4))
    with pytest.raises(A.QueueFull):
        bat.submit(A.GenerationRequest([1, 2, 3], 4))
    bat.close()
    s = A.ContinuousSession(eng, 2, A.Sampler.greedy_sampler())
    assert list(s.rows()) == [0, 0]
    assert s.step(4)  # nothing to run
    with pytest.raises(A.ConfigError):
        s.admit(0, [1, 2, 3], 4, prefill_chunk=0)
    with pytest.raises(A.ShapeError):
        s.admit(2, [1, 2, 3], 4)
    with pytest.raises(A.ShapeError):
        s.admit(0, [], 4)
    s.admit(1, [5, 6, 7, 8], 6)
    assert list(s.rows()) == [0, 1]
    with pytest.raises(A.ConfigError):
        s.admit(1, [1, 2], 4)  # occupied until retired
    s.admit(0, [9, 10], 0)  # no budget: finished at admission (prepare_session, ContextLimit)
    assert list(s.rows()) == [2, 1]
    while not s.step(1):
        pass
    outs = s.results()
    assert outs[0].token_ids == [] and outs[0].finish_reason == "ContextLimit"
    w, fin, stats, _ = ref.mtp_generate(np.array([5, 6, 7, 8], np.uint32), 6, 3, R.sampler(greedy=True))
    assert [int(t) for t in outs[1].token_ids] == list(w)
    s.retire(1)
    assert list(s.rows()) == [2, 0] and hip.kv_len(1) == 0
    assert s.results()[1].token_ids == []
    s.close()
    hip.close()


def test_continuous_batching_int4_int8kv_matches_oracle_per_round():
    """The same loop over INT4 g128 weights, a bf16 LM head and an INT8 KV cache: every
    completed request equals the oracle's stand-alone run up to its first round that
    the oracle marks as a near-tie (top-2 logit gap below the INT4 logit tolerance),
    and most rounds compare equal."""
    kw = dict(vocab_size=2048, hidden_dim=512, ffn_dim=1024, n_layers=2, n_heads=4, n_kv_heads=2, max_seq_len=160,
              num_future_tokens=4, weight_format=A.W_INT4_G128, lm_head_format=1, kv_format=A.KV_INT8)
    ref, hip = make_pair(seed=6, std=0.05, max_batch=4, max_rows=64, **kw)
    g = R.sampler(greedy=True)
    shapes = [(16, 30), (7, 12), (25, 40), (11, 22), (3, 35), (19, 18)]
    reqs = [A.GenerationRequest(R.synth_tokens(6, 40 + i, p, 2048), n) for i, (p, n) in enumerate(shapes)]
    eng = A.MtpSpeculativeEngine(hip, A.SpeculativeConfig(4))
    bat = A.SpeculativeBatcher(eng, A.BatcherConfig(max_batch_size=4, prefill_chunk_size=16),
                               A.Sampler.greedy_sampler())
    ids = [bat.submit(r) for r in reqs]
    _, done, failed = _collect(bat.run())
    assert not failed and set(done) == set(ids)
    tol_l = 4e-3  # |logit error| of the INT4 path
    same = total = 0
    for rid, r in zip(ids, reqs):
        w, fin, stats, _ = ref.mtp_generate(r.prompt_ids, r.max_new_tokens, 4, g)
        rounds = ref.last_rounds
        total += len(rounds)
        d = first_divergent_round(rounds, w, [int(t) for t in done[rid].token_ids])
        if d is None:
            same += len(rounds)
            assert done[rid].finish_reason == A.FINISH[fin]
            continue
        assert rounds[d]["logit_gap"] < tol_l, (rid, d, rounds[d])
        same += d
    assert total >= 20 and same >= 0.7 * total, (same, total)
    bat.close()
    hip.close()
