"""Pins the oracle forward and MTP engine (model.rs, nn/src, mtp_speculative.rs)."""
import numpy as np
import pytest

import npref
import refcpu as R


def tiny_cfg(**kw):
    base = dict(vocab_size=97, hidden_dim=64, ffn_dim=96, n_layers=2, n_heads=4, n_kv_heads=2,
                max_seq_len=48, num_future_tokens=3)
    base.update(kw)
    return R.make_config(**base)


def rel(a, b):
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


def test_cached_forward_matches_float64_full_forward():  # model_tests.rs:178-203
    cfg = tiny_cfg()
    m = R.Model(cfg, seed=0, std=0.05)
    W = npref.weights(m)
    ids = R.synth_tokens(0, 99, 13, cfg.vocab_size)
    kv = m.kv(cfg.max_seq_len)
    l1, h1 = kv.forward(ids[:9], 0)
    l2, h2 = kv.forward(ids[9:], 9)
    want, hwant = npref.forward(W, cfg, ids)
    got = np.concatenate([l1, l2])
    assert rel(got, want) < 1e-5
    assert rel(np.concatenate([h1, h2]), hwant) < 1e-5


def test_gqa_head_map_is_interleaved():
    # With h % n_kv the result matches; a grouped map (h // rep) would not.
    cfg = tiny_cfg(n_heads=4, n_kv_heads=2, n_layers=1)
    m = R.Model(cfg, seed=3, std=0.2)
    W = npref.weights(m)
    ids = R.synth_tokens(1, 1, 10, cfg.vocab_size)
    got, _ = m.kv(cfg.max_seq_len).forward(ids, 0)
    want, _ = npref.forward(W, cfg, ids)
    assert rel(got, want) < 1e-5


def test_rollback_by_index_overwrites_suffix():  # nn/src/kvcache.rs:380-414
    cfg = tiny_cfg()
    m = R.Model(cfg, seed=1, std=0.05)
    ids = R.synth_tokens(2, 1, 12, cfg.vocab_size)
    kv = m.kv(cfg.max_seq_len)
    kv.forward(ids[:8], 0)
    kv.forward(ids[8:12], 8)
    assert len(kv) == 12
    a, _ = kv.forward(ids[10:12], 10)  # rewind to 10 and replay
    kv2 = m.kv(cfg.max_seq_len)
    b, _ = kv2.forward(ids[:12], 0)
    assert rel(a, b[10:]) < 1e-5
    kv.truncate(4)
    assert len(kv) == 4
    with pytest.raises(ValueError):
        kv.truncate(5)


def test_mtp_head_matches_float64():  # mtp.rs:104-114, model.rs:783-817
    cfg = tiny_cfg()
    m = R.Model(cfg, seed=2, std=0.05)
    W = npref.weights(m)
    anchor = np.random.default_rng(0).normal(0, 1, cfg.hidden_dim).astype(np.float32)
    for head in (0, 1):
        ids = R.synth_tokens(3, head, head + 1, cfg.vocab_size)
        got = m.mtp_head(head, anchor, ids)
        want = npref.mtp_head(W, cfg, head, anchor, ids)
        assert rel(got, want) < 1e-5
    with pytest.raises(ValueError):
        m.mtp_head(0, anchor, np.array([1, 2], np.uint32))


def test_zero_weight_model_picks_last_index():  # F9; speculative.rs:878-904
    cfg = tiny_cfg()
    m = R.Model(cfg)  # all linears zero, norms 1
    prompt = np.array([5, 6, 7], np.uint32)
    toks, fin, stats, _ = m.mtp_generate(prompt, 6, 3, R.sampler(greedy=True))
    assert list(toks) == [cfg.vocab_size - 1] * 6 and fin == R.FINISH_MAX_TOKENS
    assert stats["target_decode_forwards"] == 2 and stats["draft_tokens_accepted"] == 6


def test_greedy_mtp_matches_plain_greedy():  # mtp_speculative.rs:438-454
    cfg = tiny_cfg(vocab_size=64, max_seq_len=64)
    m = R.Model(cfg, seed=4, std=0.3)
    prompt = R.synth_tokens(4, 2, 9, cfg.vocab_size)
    s = R.sampler(greedy=True)
    plain, fin_p = m.plain_generate(prompt, 30, s)
    for nd in (2, 3):
        spec, fin_s, stats, _ = m.mtp_generate(prompt, 30, nd, s)
        assert list(spec) == list(plain) and fin_s == fin_p
        assert stats["mtp_head_forwards"] > 0
        assert stats["draft_tokens_proposed"] == stats["draft_tokens_accepted"] + stats["draft_tokens_rejected"]
        assert stats["rounds"] <= stats["target_decode_forwards"]


def test_context_limit_is_reported():  # speculative.rs:1030-1043
    cfg = tiny_cfg(max_seq_len=16)
    m = R.Model(cfg)
    toks, fin, _, _ = m.mtp_generate(np.array([1, 2, 3, 4, 5], np.uint32), 20, 3, R.sampler(greedy=True))
    assert len(toks) == 11 and fin == R.FINISH_CONTEXT_LIMIT


def test_quantised_weights_only_change_weights():
    cfg4 = tiny_cfg(hidden_dim=128, ffn_dim=256, n_heads=4, n_kv_heads=2, weight_format=R.W_INT4_G128,
                    lm_head_format=1)
    m4 = R.Model(cfg4, seed=5, std=0.02)
    cfg32 = tiny_cfg(hidden_dim=128, ffn_dim=256, n_heads=4, n_kv_heads=2)
    m32 = R.Model(cfg32)
    for i in range(len(m4.tensors())):
        m32.set(i, m4.get(i))
    ids = R.synth_tokens(5, 5, 10, cfg4.vocab_size)
    a, _ = m4.kv(48).forward(ids, 0)
    b, _ = m32.kv(48).forward(ids, 0)
    assert np.array_equal(a, b)
    # the INT4 weights really are the g128 codec applied to the raw synthetic weights
    raw = R.synth_fill(5, 2, 128 * 128, 0.02)
    p, sh, zh = R.quantise_i4_f16(raw, 128)
    assert np.array_equal(m4.get(2).ravel(), R.dequantise_i4_f16(p, raw.size, 128, sh, zh))


def test_int8_kv_cache_stays_close_to_f32():
    kw = dict(hidden_dim=128, ffn_dim=256, n_heads=2, n_kv_heads=1)
    m8 = R.Model(tiny_cfg(kv_format=R.KV_INT8, **kw), seed=6, std=0.05)
    m32 = R.Model(tiny_cfg(**kw), seed=6, std=0.05)
    ids = R.synth_tokens(6, 6, 20, 97)
    a, _ = m8.kv(48).forward(ids, 0)
    b, _ = m32.kv(48).forward(ids, 0)
    assert 0 < rel(a, b) < 2e-2


def test_external_draft_greedy_equal_models_one_round():  # speculative.rs:962-982
    cfg = tiny_cfg(vocab_size=64, max_seq_len=64)
    t = R.Model(cfg, seed=6, std=0.3)
    d = R.Model(cfg, seed=6, std=0.3)  # draft identical to the target
    prompt = R.synth_tokens(6, 1, 5, cfg.vocab_size)
    s = R.sampler(greedy=True)
    plain, _ = t.plain_generate(prompt, 4, s)
    spec, fin, stats, _ = t.spec_generate(d, prompt, 4, 4, s)
    assert list(spec) == list(plain) and fin == R.FINISH_MAX_TOKENS
    assert stats["target_decode_forwards"] == 1 and stats["draft_tokens_accepted"] == 4


@pytest.mark.parametrize("k", [1, 2, 4])
def test_external_draft_greedy_matches_target_only(k):
    """Any draft model: greedy speculation commits exactly the target's greedy
    tokens (speculative.rs:962-982 with a disagreeing draft: rejections, replay,
    pending tokens and bonus tokens all exercised)."""
    cfg = tiny_cfg(vocab_size=64, max_seq_len=64)
    t = R.Model(cfg, seed=7, std=0.3)
    d = R.Model(cfg)  # the target's weights plus noise: a draft that agrees often, not always
    rng = np.random.default_rng(7)
    for i, (name, r, c, kind) in enumerate(t.tensors()):
        w = t.get(i)
        d.set(i, w + (rng.normal(0, 0.12, w.shape).astype(np.float32) if kind != R.T_NORM else 0))
    prompt = R.synth_tokens(7, 2, 9, cfg.vocab_size)
    s = R.sampler(greedy=True)
    plain, fin_p = t.plain_generate(prompt, 30, s)
    spec, fin_s, stats, _ = t.spec_generate(d, prompt, 30, k, s)
    assert list(spec) == list(plain) and fin_s == fin_p
    assert stats["rounds"] == stats["target_decode_forwards"]
    assert stats["draft_tokens_proposed"] == stats["draft_tokens_accepted"] + stats["draft_tokens_rejected"]
    assert stats["draft_tokens_rejected"] > 0 and stats["draft_tokens_accepted"] > 0
    # a draft forward per proposal (EOS aside) plus one per rejection or bonus, plus accepted-prefix replays
    assert stats["draft_decode_forwards"] >= stats["draft_tokens_proposed"]


def test_external_draft_shared_context_limit():  # speculative.rs:1030-1043, :203-212
    t = R.Model(tiny_cfg(max_seq_len=16))
    d = R.Model(tiny_cfg(max_seq_len=16))
    toks, fin, _, _ = t.spec_generate(d, np.array([1, 2, 3, 4, 5], np.uint32), 20, 4, R.sampler(greedy=True))
    assert len(toks) == 11 and fin == R.FINISH_CONTEXT_LIMIT
    d2 = R.Model(tiny_cfg(max_seq_len=12))  # the shorter of the two limits applies
    toks, fin, _, _ = t.spec_generate(d2, np.array([1, 2, 3, 4, 5], np.uint32), 20, 4, R.sampler(greedy=True))
    assert len(toks) == 7 and fin == R.FINISH_CONTEXT_LIMIT


def test_external_draft_sampled_stream_is_seeded():
    """Sampled external speculation: reproducible per seed, and different seeds
    give different streams (the draws come from the request's StdRng)."""
    cfg = tiny_cfg(vocab_size=64, max_seq_len=64)
    t = R.Model(cfg, seed=9, std=0.3)
    d = R.Model(cfg, seed=10, std=0.3)
    prompt = R.synth_tokens(9, 2, 6, cfg.vocab_size)
    s = R.sampler(temperature=0.9)
    a = t.spec_generate(d, prompt, 24, 3, s, seed=5)
    b = t.spec_generate(d, prompt, 24, 3, s, seed=5)
    c = t.spec_generate(d, prompt, 24, 3, s, seed=6)
    assert list(a[0]) == list(b[0]) and a[2] == b[2]
    assert list(a[0]) != list(c[0])


def test_mtp_invalid_head_after_eos_proposal_is_not_sampled():
    """mtp_speculative.rs:196-203: proposing stops after an EOS proposal, so a later
    head with an invalid (NaN) distribution raises nothing; when that head's proposal
    counts, sample_probabilities fails (sampler.rs:142-152, 286-288) and so does the run."""
    kw = dict(vocab_size=512, hidden_dim=128, ffn_dim=256, n_layers=1, n_heads=2, n_kv_heads=1, max_seq_len=96,
              num_future_tokens=3)
    ref = R.Model(R.make_config(**kw))
    for i, (name, r, c, kind) in enumerate(ref.tensors()):
        ref.set(i, R.synth_fill(21, i, r * c, 0.02) if kind != R.T_NORM else np.ones(r * c, np.float32))
    emb = ref.get(0).copy()
    emb[0] *= 10.0
    ref.set(0, emb)
    for i, (name, r, c, kind) in enumerate(ref.tensors()):
        if name.startswith("mtp.heads.1.") and kind == R.T_NORM:
            ref.set(i, np.full(r * c, np.nan, np.float32))
    ok = failed = 0
    for seed in range(60):
        prompt = R.synth_tokens(21, seed % 7, 10, 512)
        try:
            want, fin, stats, _ = ref.mtp_generate(prompt, 12, 3, R.sampler(temperature=0.8), seed=seed)
        except ValueError:
            failed += 1
            continue
        ok += 1
        # three proposals a round (target_next, head 0, head 1): a run that never samples the
        # NaN head ends in its first round on an EOS proposed by target_next or head 0
        assert fin == R.FINISH_EOS and stats["rounds"] == 1 and stats["draft_tokens_proposed"] in (1, 2)
    assert ok >= 3 and failed >= 10
