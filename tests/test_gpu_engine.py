"""End-to-end MTP speculative generation on the device against the oracle engine
(mtp_speculative.rs:86-336).  Greedy token ids are bit-exact; any divergence is
allowed only where the oracle's top-2 logit gap is below the logit tolerance."""
import numpy as np
import pytest

import aarambh_hip as A
import refcpu as R
from gpu_util import make_pair

pytestmark = pytest.mark.gpu


def test_c1_config_greedy_mtp_bit_exact():
    # 4 layers, d 256, 8q/2kv (hd 32), ffn 704, vocab 4096, 1 MTP head,
    # greedy k=1 (SpeculativeConfig(2)), prompt 64 ids, 128 new tokens.
    kw = dict(vocab_size=4096, hidden_dim=256, ffn_dim=704, n_layers=4, n_heads=8, n_kv_heads=2, max_seq_len=256,
              num_future_tokens=2)
    ref, hip = make_pair(seed=0, max_batch=1, max_rows=64, **kw)
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


def test_int4_batched_greedy_mtp_matches_oracle_per_sequence():
    kw = dict(vocab_size=2048, hidden_dim=512, ffn_dim=1024, n_layers=2, n_heads=4, n_kv_heads=2, max_seq_len=128,
              num_future_tokens=4, weight_format=A.W_INT4_G128, lm_head_format=1, kv_format=A.KV_INT8)
    ref, hip = make_pair(seed=6, std=0.05, max_batch=4, max_rows=64, **kw)
    prompts = R.synth_tokens(6, 3, 4 * 16, 2048).reshape(4, 16)
    eng = A.MtpSpeculativeEngine(hip, A.SpeculativeConfig(4))
    outs = eng.generate_batch(prompts, 40, A.Sampler.greedy_sampler())
    for b in range(4):
        want, fin, stats, gap = ref.mtp_generate(prompts[b], 40, 4, R.sampler(greedy=True))
        if gap < 2e-3:
            continue  # flagged near-tie in this request
        assert outs[b].token_ids == list(want), b
        assert outs[b].speculative_stats.target_decode_forwards == stats["target_decode_forwards"]
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
