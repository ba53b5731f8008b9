"""Shared helpers for the GPU parity tests: build matching oracle / HIP models."""
import numpy as np

import aarambh_hip as A
import refcpu as R


def rel_rows(got, want):
    """Norm-wise relative error per row: max|d| / max|ref| (the logit tolerance rule)."""
    got = np.asarray(got, np.float64).reshape(-1, got.shape[-1])
    want = np.asarray(want, np.float64).reshape(-1, want.shape[-1])
    return np.max(np.abs(got - want), axis=1) / np.maximum(np.max(np.abs(want), axis=1), 1e-30)


def make_pair(seed=0, std=0.02, max_batch=1, max_rows=64, **kw):
    """Identical random-init weights in the oracle and on the device (f32 host values,
    quantised by each side's own codec)."""
    tie = kw.pop("tie_embeddings", True)
    rc = R.make_config(untied_lm_head=0 if tie else 1, **kw)
    ref = R.Model(rc)
    mc = A.ModelConfig(tie_embeddings=tie, **kw)
    hip = A.HipModel(mc, max_batch=max_batch, max_rows=max_rows)
    assert [t[0] for t in hip.tensors()] == [t[0] for t in ref.tensors()]
    for i, (name, r, c, kind) in enumerate(ref.tensors()):
        raw = R.synth_fill(seed, i, r * c, std) if kind != R.T_NORM else np.ones(r * c, np.float32)
        ref.set(i, raw)
        hip.load_f32(i, raw)
    return ref, hip


def mtp_rounds_vs_oracle(ref, hip, prompt, max_new, K, s_ref, s_dev, seed, tol_p, tol_l, start=0, want=None,
                         rounds=None):
    """MtpSpeculativeEngine (mtp_speculative.rs:161-322) on the device, round by round
    against the oracle engine's trace, with teacher forcing: the device starts from the
    oracle's state at round `start` (prompt + committed tokens, sampler keystream
    position) and runs one round at a time; a round must commit the oracle's tokens with
    the same proposed / accepted counts and end at the same keystream position.  A round
    that differs must be one the oracle marks as a near-tie (a sampled decision within
    tol_p of its boundary, or a greedy / top-k logit gap below tol_l); the device then
    restarts from the oracle's state after that round.
    Returns (rounds equal, flagged divergences, oracle rounds from `start`)."""
    prompt = np.asarray(prompt, np.uint32)
    if want is None:
        want, _, _, _ = ref.mtp_generate(prompt, max_new, K, s_ref, seed=seed)
        rounds = ref.last_rounds
    eng = A.MtpSpeculativeEngine(hip, A.SpeculativeConfig(K))
    r, same, flagged = start, 0, 0
    while r < len(rounds):
        rd = rounds[r]
        c0 = rd["committed_before"]
        p = np.concatenate([prompt, np.asarray(want[:c0], np.uint32)])
        sess = eng.session(p[None], max_new - c0, s_dev, seeds=np.array([seed], np.uint64))
        sess.set_rng_offsets([rd["rng_pos_before"]])
        n_prev, prop_prev, acc_prev = 0, 0, 0
        try:
            while r < len(rounds):
                rd = rounds[r]
                sess.step(1)
                out = sess.result()[0]
                st = out.speculative_stats
                got = [int(t) for t in out.token_ids[n_prev:]]
                exp = [int(t) for t in want[rd["committed_before"]:rd["committed_after"]]]
                ok = (got == exp and st.draft_tokens_proposed - prop_prev == rd["proposed"]
                      and st.draft_tokens_accepted - acc_prev == rd["accepted"]
                      and int(sess.rng_offsets()[0]) == rd["rng_pos_after"])
                r += 1
                if ok:
                    same += 1
                    n_prev, prop_prev, acc_prev = len(out.token_ids), st.draft_tokens_proposed, st.draft_tokens_accepted
                    continue
                assert rd["prob_margin"] < tol_p or rd["logit_gap"] < tol_l, \
                    f"round {r - 1} differs without a near-tie: device {got} oracle {exp} ({rd})"
                flagged += 1
                break
        finally:
            sess.close()
    return same, flagged, len(rounds) - start


def first_divergent_round(rounds, want, got):
    """Index of the oracle round holding the first token where `got` departs from
    `want` (None when they are equal)."""
    n = min(len(want), len(got))
    diff = [i for i in range(n) if int(want[i]) != int(got[i])]
    t = diff[0] if diff else (n if len(want) != len(got) else None)
    if t is None:
        return None
    for i, rd in enumerate(rounds):
        if rd["committed_before"] <= t < max(rd["committed_after"], rd["committed_before"] + 1):
            return i
    return len(rounds) - 1


def spec_rounds_vs_oracle(ref_t, ref_d, eng, prompt, max_new, K, s_ref, s_dev, seed, tol_p, tol_l, start=0,
                          want=None, rounds=None):
    """SpeculativeEngine (speculative.rs:251-508) on the device, round by round against
    the oracle engine's trace with teacher forcing, as mtp_rounds_vs_oracle does for the
    MTP engine: the device starts from the oracle's state at round `start` (prompt +
    committed tokens prefilled into both models, sampler keystream position) and runs one
    round at a time; a round must commit the oracle's tokens with the same proposed /
    accepted counts and draft forwards and end at the same keystream position.  From a
    later round the reference carries the last committed token as its pending verify row
    (:305-310); the restarted device forwards it in the prefill instead, which gives the
    same distributions.  A differing round must be one the oracle marks as a near-tie;
    the device then restarts from the oracle's state after it.
    Returns (rounds equal, flagged divergences, oracle rounds from `start`)."""
    prompt = np.asarray(prompt, np.uint32)
    if want is None:
        want, _, _, _ = ref_t.spec_generate(ref_d, prompt, max_new, K, s_ref, seed=seed)
        rounds = ref_t.last_rounds
    r, same, flagged = start, 0, 0
    while r < len(rounds):
        rd = rounds[r]
        c0 = rd["committed_before"]
        p = np.concatenate([prompt, np.asarray(want[:c0], np.uint32)])
        sess = eng.session(p[None], max_new - c0, s_dev, seeds=np.array([seed], np.uint64))
        sess.set_rng_offsets([rd["rng_pos_before"]])
        n_prev, prop_prev, acc_prev = 0, 0, 0
        try:
            while r < len(rounds):
                rd = rounds[r]
                sess.step(1)
                out = sess.result()[0]
                st = out.speculative_stats
                got = [int(t) for t in out.token_ids[n_prev:]]
                exp = [int(t) for t in want[rd["committed_before"]:rd["committed_after"]]]
                ok = (got == exp and st.draft_tokens_proposed - prop_prev == rd["proposed"]
                      and st.draft_tokens_accepted - acc_prev == rd["accepted"]
                      and int(sess.rng_offsets()[0]) == rd["rng_pos_after"])
                r += 1
                if ok:
                    same += 1
                    n_prev, prop_prev, acc_prev = len(out.token_ids), st.draft_tokens_proposed, st.draft_tokens_accepted
                    continue
                assert rd["prob_margin"] < tol_p or rd["logit_gap"] < tol_l, \
                    f"round {r - 1} differs without a near-tie: device {got} oracle {exp} ({rd})"
                flagged += 1
                break
        finally:
            sess.close()
    return same, flagged, len(rounds) - start


def prob_margin(pairs, prompt, temperature):
    """Near-tie margin for sampled engine comparisons, from the measured logit error:
    the largest |device - oracle| logit over a forward of `prompt` through each
    (oracle, device) model pair, e.  Softmax at T moves each probability by a relative
    factor of at most exp(2 e / T) - 1 (about 2 e / T), and a ratio p / q by twice
    that; the margin is twice the ratio bound (at least 1e-5, the acceptance flag's
    own width).  Decisions closer than this to their boundary may flip."""
    prompt = np.asarray(prompt, np.uint32)
    e = 0.0
    for ref, hip in pairs:
        want, _ = ref.kv(len(prompt) + 8).forward(prompt, 0)
        got, _ = hip.forward_with_cache_output(prompt[None], [0], slots=[0])
        e = max(e, float(np.max(np.abs(got[0].astype(np.float64) - want))))
        hip.restore(0, slot=0)
    print(f"prob_margin: max logit error {e:.3e} at T {temperature}")
    return max(1e-5, 2.0 * 2.0 * float(np.expm1(2.0 * e / temperature)))
