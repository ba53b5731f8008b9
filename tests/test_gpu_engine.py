"""End-to-end MTP speculative generation on the device against the oracle engine
(mtp_speculative.rs:86-336).  Greedy token ids are bit-exact; sampled runs are
compared round by round from the oracle's state (committed tokens, keystream
position).  A round may differ only where the oracle marks one of its decisions as
a near-tie (a top-2 / top-k logit gap below the logit tolerance, or a sampled
decision within the probability tolerance of its boundary), and a minimum number
of rounds must compare equal."""
import numpy as np
import pytest

import aarambh_hip as A
import refcpu as R
from gpu_util import (first_divergent_round, make_pair, mtp_rounds_vs_oracle, prob_margin, rel_rows,
                      spec_rounds_vs_oracle)

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("replay", ["replacement", "reference"])
def test_c1_config_greedy_mtp_bit_exact(replay):
    # Config 1: 4 layers, d 256, 8q/2kv (hd 32), ffn 704, vocab 4096, 1 MTP head,
    # greedy k=1 (SpeculativeConfig(2)), prompt 64 ids, 128 new tokens.
    kw = dict(vocab_size=4096, hidden_dim=256, ffn_dim=704, n_layers=4, n_heads=8, n_kv_heads=2, max_seq_len=256,
              num_future_tokens=2)
    ref, hip = make_pair(seed=0, max_batch=1, max_rows=64, **kw)
    hip.set_replay_schedule(A.REPLAY_REFERENCE if replay == "reference" else A.REPLAY_REPLACEMENT)
    prompt = R.synth_tokens(0, 0xC1, 64, 4096)
    want, fin, stats, gap = ref.mtp_generate(prompt, 128, 2, R.sampler(greedy=True))
    eng = A.MtpSpeculativeEngine(hip, A.SpeculativeConfig(2))
    out = eng.generate(prompt, 128, A.Sampler.greedy_sampler())
    # the f32 path matches the oracle to ~1e-6 relative (|logit| < 2): a top-2 gap
    # above 1e-5 cannot flip an argmax, so the ids must be identical.
    assert gap > 1e-5, f"oracle near-tie {gap}: parity would be flagged"
    assert out.token_ids == list(want)
    assert out.finish_reason == "MaxTokens" and fin == R.FINISH_MAX_TOKENS
    got = out.speculative_stats
    for k in ("rounds", "draft_tokens_proposed", "draft_tokens_accepted", "target_decode_forwards",
              "mtp_head_forwards"):
        assert getattr(got, k) == stats[k], (k, getattr(got, k), stats[k])
    hip.close()


def test_greedy_mtp_with_untied_head_and_yarn_rope():
    """The MTP engine over a model with an untied LM head (model.rs:239-262, shared by the
    MTP heads) and YaRN RoPE scaling (rope_scaling.rs:62-92): token ids and statistics
    bit-exact against the oracle engine on the same model (f32, C1 widths, 3 heads)."""
    kw = dict(vocab_size=4096, hidden_dim=256, ffn_dim=704, n_layers=2, n_heads=8, n_kv_heads=2, max_seq_len=256,
              num_future_tokens=4)
    ref, hip = make_pair(seed=3, std=0.05, max_batch=1, max_rows=64, tie_embeddings=False, **kw)
    rs = dict(method="yarn", factor=4.0, original_max_seq_len=64, beta_fast=16.0, beta_slow=1.0, attn_factor=1.1)
    ref.set_rope_scaling(rs)
    hip.set_rope_scaling(A.RopeScaling(**rs))
    prompt = R.synth_tokens(3, 0xC1, 48, 4096)
    want, fin, stats, gap = ref.mtp_generate(prompt, 96, 4, R.sampler(greedy=True))
    assert gap > 1e-5, f"oracle near-tie {gap}: parity would be flagged"
    out = A.MtpSpeculativeEngine(hip, A.SpeculativeConfig(4)).generate(prompt, 96, A.Sampler.greedy_sampler())
    assert out.token_ids == list(want)
    got = out.speculative_stats
    for k in ("rounds", "draft_tokens_proposed", "draft_tokens_accepted", "target_decode_forwards",
              "mtp_head_forwards"):
        assert getattr(got, k) == stats[k], (k, getattr(got, k), stats[k])
    hip.close()


def test_int4_batched_greedy_mtp_matches_oracle_per_round():
    """Four requests in lock-step: each request's committed tokens equal the oracle's
    up to its first near-tie round (top-2 gap below the INT4 logit tolerance); past it
    the request is replayed round by round from the oracle's state."""
    kw = dict(vocab_size=2048, hidden_dim=512, ffn_dim=1024, n_layers=2, n_heads=4, n_kv_heads=2, max_seq_len=128,
              num_future_tokens=4, weight_format=A.W_INT4_G128, lm_head_format=1, kv_format=A.KV_INT8)
    ref, hip = make_pair(seed=6, std=0.05, max_batch=4, max_rows=64, **kw)
    prompts = R.synth_tokens(6, 3, 4 * 16, 2048).reshape(4, 16)
    eng = A.MtpSpeculativeEngine(hip, A.SpeculativeConfig(4))
    outs = eng.generate_batch(prompts, 40, A.Sampler.greedy_sampler())
    tol_l = 4e-3  # |logit error| of the INT4 path (2e-3 relative of |logits| <= 2)
    same = total = 0
    for b in range(4):
        want, fin, stats, gap = ref.mtp_generate(prompts[b], 40, 4, R.sampler(greedy=True))
        rounds = ref.last_rounds
        total += len(rounds)
        r = first_divergent_round(rounds, want, outs[b].token_ids)
        if r is None:
            same += len(rounds)
            assert outs[b].speculative_stats.target_decode_forwards == stats["target_decode_forwards"]
            continue
        assert rounds[r]["logit_gap"] < tol_l, (b, r, rounds[r])
        s2, _, _ = mtp_rounds_vs_oracle(ref, hip, prompts[b], 40, 4, R.sampler(greedy=True),
                                        A.Sampler.greedy_sampler(), 0, 0.0, tol_l, start=r + 1, want=want,
                                        rounds=rounds)
        same += r + s2
    assert total >= 20 and same >= 0.8 * total, (same, total)
    hip.close()


@pytest.mark.parametrize("cfg,replay", [("c1_t08", "replacement"), ("k3_cli_default", "replacement"),
                                        ("k3_cli_default", "reference")])
def test_sampled_mtp_engine_round_by_round(cfg, replay):
    """Sampled MTP speculation (draw order: K proposal draws, one acceptance draw per
    tested proposal with q > 0, one residual draw on rejection) on the device, every
    round compared with the oracle's: committed tokens, proposed / accepted counts and
    the keystream position after the round.  C1 model at T 0.8 (k = 1), and a 3-head
    model with the reference CLI's default sampler (T 0.7, top-k 50, top-p 0.9), under
    both rejection replay schedules (the oracle always runs the reference's,
    mtp_speculative.rs:302-313)."""
    if cfg == "c1_t08":
        kw = dict(vocab_size=4096, hidden_dim=256, ffn_dim=704, n_layers=4, n_heads=8, n_kv_heads=2,
                  max_seq_len=256, num_future_tokens=2)
        ref, hip = make_pair(seed=0, max_batch=1, max_rows=64, **kw)
        prompt, K, n_new, seed = R.synth_tokens(0, 0xC1, 64, 4096), 2, 128, 42
        s_ref, s_dev = R.sampler(temperature=0.8), A.Sampler.top_k_top_p(0.8, seed=seed)
        T = 0.8
    else:
        kw = dict(vocab_size=1024, hidden_dim=256, ffn_dim=512, n_layers=2, n_heads=4, n_kv_heads=2,
                  max_seq_len=192, num_future_tokens=4)
        ref, hip = make_pair(seed=31, std=0.3, max_batch=1, max_rows=64, **kw)
        prompt, K, n_new, seed = R.synth_tokens(31, 1, 12, 1024), 4, 120, 7
        s_ref = R.sampler(temperature=0.7, top_k=50, top_p=0.9)
        s_dev = A.Sampler.top_k_top_p(0.7, top_k=50, top_p=0.9, seed=seed)
        T = 0.7
    tol_p = prob_margin([(ref, hip)], prompt, T)
    assert tol_p < 5e-3, tol_p
    hip.set_replay_schedule(A.REPLAY_REFERENCE if replay == "reference" else A.REPLAY_REPLACEMENT)
    want, fin, stats, _ = ref.mtp_generate(prompt, n_new, K, s_ref, seed=seed)
    rounds = ref.last_rounds
    assert stats["draft_tokens_accepted"] > 0 and stats["draft_tokens_rejected"] > 0
    same, flagged, total = mtp_rounds_vs_oracle(ref, hip, prompt, n_new, K, s_ref, s_dev, seed, tol_p, 1e-4,
                                                want=want, rounds=rounds)
    assert total >= 20 and same >= 0.9 * total, (same, flagged, total)
    if flagged == 0:
        # nothing diverged: the one-call engine reproduces the whole run and its statistics
        out = A.MtpSpeculativeEngine(hip, A.SpeculativeConfig(K)).generate_batch(
            prompt[None], n_new, s_dev, seeds=np.array([seed], np.uint64))[0]
        assert [int(t) for t in out.token_ids] == [int(t) for t in want]
        for k in ("rounds", "draft_tokens_proposed", "draft_tokens_accepted", "target_decode_forwards",
                  "mtp_head_forwards"):
            assert getattr(out.speculative_stats, k) == stats[k], k
    hip.close()


def test_mtp_session_top_candidates_match_oracle():
    """Per committed token, the session records the top-5 candidates of the target
    distribution at its position (mtp_speculative.rs:247-250): identical to the
    oracle engine's, accepted, rejected-replacement and bonus-free rounds alike."""
    kw = dict(vocab_size=1024, hidden_dim=256, ffn_dim=512, n_layers=2, n_heads=4, n_kv_heads=2, max_seq_len=128,
              num_future_tokens=3)
    ref, hip = make_pair(seed=8, std=0.3, max_batch=2, max_rows=64, **kw)
    prompts = R.synth_tokens(8, 2, 2 * 9, 1024).reshape(2, 9)
    eng = A.MtpSpeculativeEngine(hip, A.SpeculativeConfig(3))
    sess = eng.session(prompts, 30, A.Sampler.greedy_sampler())
    while not sess.step(4):
        pass
    outs = sess.result()
    sess.close()
    for b in range(2):
        want, fin, stats, gap = ref.mtp_generate(prompts[b], 30, 3, R.sampler(greedy=True))
        assert gap > 1e-5
        assert outs[b].token_ids == list(want)
        ci, cp = ref.last_candidates
        assert [[i for i, _ in c] for c in outs[b].candidates] == ci.tolist()
        assert [[p for _, p in c] for c in outs[b].candidates] == cp.tolist()
    hip.close()


def test_invalid_sampled_proposal_fails_at_the_proposal():
    """An MTP head whose logits are all NaN makes its proposal distribution invalid
    (sample_probabilities, sampler.rs:142-152, 314-335): the round fails with the
    reference's message, and the session is left as the proposal step found it (the
    reference fails before the verify forward, mtp_speculative.rs:169-209), so the cache
    length, the statistics and the keystream position are those of the previous round."""
    kw = dict(vocab_size=1024, hidden_dim=256, ffn_dim=704, n_layers=2, n_heads=8, n_kv_heads=2, max_seq_len=96,
              num_future_tokens=3)
    ref, hip = make_pair(seed=41, std=0.05, **kw)
    names = [t[0] for t in hip.tensors()]
    eng = A.MtpSpeculativeEngine(hip, A.SpeculativeConfig(3))
    prompt = R.synth_tokens(41, 1, 12, 1024)
    s = A.Sampler(greedy=False, temperature=0.8, seed=5)
    sess = eng.session(prompt[None], 20, s, seeds=np.array([5], np.uint64))
    sess.step(1)  # one good round
    out = sess.result()[0]
    st0, off0, kv0, n0 = out.speculative_stats, int(sess.rng_offsets()[0]), hip.kv_len(0), len(out.token_ids)
    assert st0.rounds == 1 and kv0 == len(prompt) + n0
    hip.load_f32(names.index("mtp.heads.1.output_norm.weight"), np.full(256, np.nan, np.float32))
    with pytest.raises(A.ConfigError, match="proposal distribution is invalid"):
        sess.step(1)
    st1 = sess.result()[0].speculative_stats
    assert (st1.rounds, st1.target_decode_forwards, st1.draft_tokens_proposed, st1.mtp_head_forwards) == \
        (st0.rounds, st0.target_decode_forwards, st0.draft_tokens_proposed, st0.mtp_head_forwards)
    assert int(sess.rng_offsets()[0]) == off0 and hip.kv_len(0) == kv0
    assert len(sess.result()[0].token_ids) == n0
    sess.close()
    hip.close()


def test_context_limit_and_engine_validation():
    kw = dict(vocab_size=1024, hidden_dim=256, ffn_dim=512, n_layers=1, n_heads=2, n_kv_heads=1, max_seq_len=16,
              num_future_tokens=3)
    ref, hip = make_pair(seed=7, **kw)
    with pytest.raises(A.ConfigError):
        A.MtpSpeculativeEngine(hip, A.SpeculativeConfig(4))
    with pytest.raises(A.ConfigError):
        A.MtpSpeculativeEngine(hip, A.SpeculativeConfig(1))
    eng = A.MtpSpeculativeEngine(hip, A.SpeculativeConfig(3))
    out = eng.generate(np.arange(1, 6, dtype=np.uint32), 20, A.Sampler.greedy_sampler())
    want, fin, _, _ = ref.mtp_generate(np.arange(1, 6, dtype=np.uint32), 20, 3, R.sampler(greedy=True))
    assert len(out.token_ids) == 11 and out.finish_reason == "ContextLimit"
    assert out.token_ids == list(want)
    hip.close()


def test_ragged_finish_keeps_every_slot_cache():
    """A sequence that finishes rounds before the others (EOS) keeps its cache: its slot
    holds the reference's cache state (prompt + committed tokens, restored to the round's
    base when the replacement is EOS, mtp_speculative.rs:284-288) and a follow-up forward
    from the cached length matches the oracle's forward of the same tokens."""
    kw = dict(vocab_size=512, hidden_dim=128, ffn_dim=256, n_layers=1, n_heads=2, n_kv_heads=1, max_seq_len=96,
              num_future_tokens=3)
    ref, hip = make_pair(seed=21, max_batch=2, **kw)
    emb = ref.get(0).copy()
    emb[0] *= 6.0  # make EOS (id 0) a frequent greedy choice
    ref.set(0, emb)
    hip.load_f32(0, emb)
    g = R.sampler(greedy=True)
    runs = []
    for ps in range(60):
        prompt = R.synth_tokens(21, ps, 12, 512)
        want, fin, stats, gap = ref.mtp_generate(prompt, 24, 3, g)
        if gap > 1e-4:
            runs.append((stats["rounds"], fin, prompt, list(want)))
    early = [r for r in runs if r[1] == R.FINISH_EOS and len(r[3]) > 0]
    late = [r for r in runs if r[1] == R.FINISH_MAX_TOKENS]
    assert early and late, "no ragged pair among the candidate prompts"
    pair = [min(early, key=lambda r: r[0]), late[0]]
    assert pair[0][0] < pair[1][0]
    eng = A.MtpSpeculativeEngine(hip, A.SpeculativeConfig(3))
    outs = eng.generate_batch(np.stack([pair[0][2], pair[1][2]]), 24, A.Sampler.greedy_sampler())
    for b, (rounds, fin, prompt, want) in enumerate(pair):
        assert outs[b].token_ids == want
        seq = np.concatenate([prompt, np.asarray(want, np.uint32)])
        n = hip.kv_len(b)
        # an accepted EOS proposal leaves the whole verify in the cache (no restore)
        assert len(prompt) <= n <= len(seq) + 3, (b, n, len(seq))
        # forward the last cached committed token again at its own position: reads positions < m
        m = min(n, len(seq)) - 1
        got, _ = hip.forward_with_cache_output(seq[None, m:m + 1], [m], slots=[b])
        wl, _ = ref.kv(96).forward(seq[:m + 1], 0)
        assert rel_rows(got[0], wl[-1:]).max() < 1e-4
    hip.close()


def _draft_pair(target_seed, noise, max_batch, max_rows, **kw):
    """Oracle + device draft models whose weights are the target's synthetic weights
    (synth_fill(target_seed, i)) plus N(0, noise^2): a draft that often agrees."""
    rc = R.make_config(**kw)
    ref = R.Model(rc)
    hip = A.HipModel(A.ModelConfig(**kw), max_batch=max_batch, max_rows=max_rows)
    rng = np.random.default_rng(target_seed + 1000)
    for i, (name, r, c, kind) in enumerate(ref.tensors()):
        if kind == R.T_NORM:
            raw = np.ones(r * c, np.float32)
        else:
            raw = R.synth_fill(target_seed, i, r * c, 0.3) + rng.normal(0, noise, r * c).astype(np.float32)
        ref.set(i, raw)
        hip.load_f32(i, raw)
    return ref, hip


@pytest.mark.parametrize("k", [1, 3])
def test_external_draft_greedy_matches_oracle(k):
    """SpeculativeEngine (speculative.rs:175-516) on the device, f32 target and a
    perturbed f32 draft, 3 requests in lock-step: token ids and every
    SpeculativeStats counter equal the oracle engine's per request, and equal the
    target's plain greedy decode."""
    kw = dict(vocab_size=512, hidden_dim=256, ffn_dim=512, n_layers=2, n_heads=4, n_kv_heads=2, max_seq_len=96)
    ref_t, hip_t = make_pair(seed=21, std=0.3, max_batch=3, max_rows=64, **kw)
    ref_d, hip_d = _draft_pair(21, 0.05, 3, 64, **kw)
    prompts = R.synth_tokens(21, 1, 3 * 7, 512).reshape(3, 7)
    eng = A.SpeculativeEngine(hip_t, hip_d, A.SpeculativeConfig(k))
    outs = eng.generate_batch(prompts, 40, A.Sampler.greedy_sampler())
    n_acc = 0
    for b in range(3):
        want, fin, stats, gap = ref_t.spec_generate(ref_d, prompts[b], 40, k, R.sampler(greedy=True))
        plain, _ = ref_t.plain_generate(prompts[b], 40, R.sampler(greedy=True))
        assert list(want) == list(plain)
        assert gap > 1e-5, f"oracle near-tie {gap}"
        assert outs[b].token_ids == list(want), b
        assert outs[b].finish_reason == A.FINISH[fin]
        got = outs[b].speculative_stats
        for key, v in stats.items():
            assert getattr(got, key) == v, (b, key, getattr(got, key), v)
        n_acc += stats["draft_tokens_accepted"]
        # top candidates of every committed token (sampler.rs:188-208): one-hot at the token
        ci, cp = ref_t.last_candidates
        assert [[i for i, _ in c] for c in outs[b].candidates] == ci.tolist()
        assert [[p for _, p in c] for c in outs[b].candidates] == cp.tolist()
    assert n_acc > 0  # acceptance, rejection and bonus paths all ran
    for m in (hip_t, hip_d):
        m.close()


def test_external_draft_int4_batched_matches_oracle():
    """External-draft engine, INT4 target and draft, 4 requests in lock-step: each
    request equals the oracle up to its first near-tie round (top-2 gap below the INT4
    logit tolerance), with its statistics when there is none; past it the request is
    replayed round by round from the oracle's state (teacher forcing)."""
    kw = dict(vocab_size=2048, hidden_dim=512, ffn_dim=1024, n_heads=4, n_kv_heads=2, max_seq_len=128,
              weight_format=A.W_INT4_G128, lm_head_format=1, kv_format=A.KV_INT8)
    ref_t, hip_t = make_pair(seed=22, std=0.05, max_batch=4, max_rows=64, n_layers=2, **kw)
    ref_d, hip_d = make_pair(seed=22, std=0.05, max_batch=4, max_rows=64, n_layers=1, **kw)
    prompts = R.synth_tokens(22, 3, 4 * 12, 2048).reshape(4, 12)
    eng = A.SpeculativeEngine(hip_t, hip_d, A.SpeculativeConfig(4))
    outs = eng.generate_batch(prompts, 32, A.Sampler.greedy_sampler())
    tol_l = 4e-3
    same = total = 0
    for b in range(4):
        want, fin, stats, gap = ref_t.spec_generate(ref_d, prompts[b], 32, 4, R.sampler(greedy=True))
        rounds = ref_t.last_rounds
        total += len(rounds)
        r = first_divergent_round(rounds, want, outs[b].token_ids)
        if r is None:
            same += len(rounds)
            assert outs[b].speculative_stats.target_decode_forwards == stats["target_decode_forwards"]
            assert outs[b].speculative_stats.draft_decode_forwards == stats["draft_decode_forwards"]
            continue
        assert rounds[r]["logit_gap"] < tol_l, (b, r, rounds[r])
        s2, _, _ = spec_rounds_vs_oracle(ref_t, ref_d, eng, prompts[b], 32, 4, R.sampler(greedy=True),
                                         A.Sampler.greedy_sampler(), 0, 0.0, tol_l, start=r + 1, want=want,
                                         rounds=rounds)
        same += r + s2
    assert total >= 16 and same >= 0.9 * total, (same, total)
    for m in (hip_t, hip_d):
        m.close()


def test_external_draft_context_limit_and_validation():
    kw = dict(vocab_size=1024, hidden_dim=256, ffn_dim=512, n_layers=1, n_heads=2, n_kv_heads=1)
    ref_t, hip_t = make_pair(seed=23, max_seq_len=16, **kw)
    ref_d, hip_d = make_pair(seed=24, max_seq_len=12, **kw)
    with pytest.raises(A.ConfigError):
        A.SpeculativeEngine(hip_t, hip_d, A.SpeculativeConfig(0))
    eng = A.SpeculativeEngine(hip_t, hip_d, A.SpeculativeConfig(4))
    p = np.arange(1, 6, dtype=np.uint32)
    out = eng.generate(p, 20, A.Sampler.greedy_sampler())
    want, fin, _, _ = ref_t.spec_generate(ref_d, p, 20, 4, R.sampler(greedy=True))
    assert len(out.token_ids) == 7 and out.finish_reason == "ContextLimit" and fin == R.FINISH_CONTEXT_LIMIT
    assert out.token_ids == list(want)
    with pytest.raises(A.ShapeError):
        eng.generate(np.arange(1, 14, dtype=np.uint32), 4, A.Sampler.greedy_sampler())
    for m in (hip_t, hip_d):
        m.close()


@pytest.mark.parametrize("sampler", ["t09", "cli_default"])
def test_external_draft_sampled_round_by_round(sampler):
    """Sampled external-draft speculation (draw order: one draw per proposal, one
    acceptance draw per tested proposal with q > 0, a residual draw on rejection, a bonus
    draw when everything is accepted, speculative.rs:251-501): the whole run is
    reproducible with consistent statistics, and every round, started from the oracle's
    state (teacher forcing), commits the oracle's tokens with its counts and keystream
    position, unless the oracle marks the round as a near-tie within the margin the
    measured logit error allows (prob_margin)."""
    kw = dict(vocab_size=512, hidden_dim=256, ffn_dim=512, n_layers=1, n_heads=4, n_kv_heads=2, max_seq_len=96)
    ref_t, hip_t = make_pair(seed=25, std=0.3, max_batch=2, max_rows=64, **kw)
    ref_d, hip_d = _draft_pair(25, 0.1, 2, 64, **kw)
    prompts = R.synth_tokens(25, 1, 2 * 6, 512).reshape(2, 6)
    eng = A.SpeculativeEngine(hip_t, hip_d, A.SpeculativeConfig(3))
    if sampler == "t09":
        T, s_dev, s_ref = 0.9, A.Sampler.top_k_top_p(0.9, seed=11), R.sampler(temperature=0.9)
    else:
        T = 0.7
        s_dev = A.Sampler.top_k_top_p(0.7, top_k=50, top_p=0.9, seed=11)
        s_ref = R.sampler(temperature=0.7, top_k=50, top_p=0.9)
    seeds = np.array([11, 12], np.uint64)
    a = eng.generate_batch(prompts, 60, s_dev, seeds=seeds)
    b = eng.generate_batch(prompts, 60, s_dev, seeds=seeds)
    tol_p = prob_margin([(ref_t, hip_t), (ref_d, hip_d)], prompts[0], T)
    assert tol_p < 5e-3, tol_p
    same = total = flagged = 0
    for j, (x, y) in enumerate(zip(a, b)):
        assert x.token_ids == y.token_ids
        st = x.speculative_stats
        assert st.draft_tokens_proposed == st.draft_tokens_accepted + st.draft_tokens_rejected
        want, fin, stats, _ = ref_t.spec_generate(ref_d, prompts[j], 60, 3, s_ref, seed=int(seeds[j]))
        rounds = ref_t.last_rounds
        if first_divergent_round(rounds, want, x.token_ids) is None:
            for k, v in stats.items():
                assert getattr(st, k) == v, (j, k, getattr(st, k), v)
        s2, f2, t2 = spec_rounds_vs_oracle(ref_t, ref_d, eng, prompts[j], 60, 3, s_ref, s_dev, int(seeds[j]), tol_p,
                                           1e-4, want=want, rounds=rounds)
        same, flagged, total = same + s2, flagged + f2, total + t2
    assert total >= 20 and same >= 0.9 * total, (same, flagged, total)
    for m in (hip_t, hip_d):
        m.close()
