"""Parity of the fused acceptance kernel against the oracle (accept_proposal,
residual_distribution, sample_probabilities: speculative.rs:755-793,
sampler.rs:102-347).  Bar: accepted lengths and tokens bit-identical except on
draws either side flags as near-ties (|p/q - u| < 1e-5, |cdf - u| < 1e-6)."""
import numpy as np
import pytest
import torch

import aarambh_hip as A
import refcpu as R

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


@pytest.fixture(scope="module")
def ctx():
    m = A.HipModel(A.ModelConfig(vocab_size=128, hidden_dim=128, ffn_dim=128, n_layers=1, n_heads=1,
                                 n_kv_heads=1, max_seq_len=16), max_batch=1, max_rows=16)
    yield m
    m.close()


def c2_inputs(B=32, K=4, V=32000, T=0.8, seed=0):
    """benchmark config 2: target ~ N(0, 3^2), draft = target + N(0, 1), draft tokens
    sampled from the draft distribution with the oracle's sequential CDF."""
    rng = np.random.default_rng(seed)
    tgt = rng.normal(0, 3, (B, K + 1, V)).astype(np.float32)
    drf = (tgt[:, :K] + rng.normal(0, 1, (B, K, V))).astype(np.float32)
    s = R.sampler(temperature=T)
    toks = np.zeros((B, K), np.uint32)
    for b in range(B):
        r = R.Rng(10_000 + b)
        for i in range(K):
            toks[b, i] = R.sample_probabilities(s, r, R.probabilities(s, drf[b, i]))
    return tgt, drf, toks


def run_both(ctx, tgt, drf, toks, T, bonus, seeds=None, offsets=None, uniforms=None, nprop=None, greedy=False,
             top_k=0, top_p=0.0):
    s_dev = A.Sampler.greedy_sampler() if greedy else A.Sampler.top_k_top_p(T, top_k=top_k, top_p=top_p)
    s_ref = R.sampler(greedy=True) if greedy else R.sampler(temperature=T, top_k=top_k, top_p=top_p)
    t = lambda a, dt: None if a is None else torch.from_numpy(np.ascontiguousarray(a).astype(dt)).to(DEV)
    out = ctx.accept_sample(t(tgt, np.float32), t(drf, np.float32), t(toks, np.int32), s_dev, bonus,
                            seeds=t(seeds, np.int64), word_offsets=t(offsets, np.int64),
                            uniforms=t(uniforms, np.float32), n_proposals=t(nprop, np.int32))
    out = {k: v.cpu().numpy() for k, v in out.items()}
    ref = R.accept_batch(tgt, drf, toks, s_ref, bonus, seeds=seeds, word_offsets=offsets, uniforms=uniforms,
                         n_proposals=nprop)
    return out, ref


def assert_parity(out, ref, max_flag_frac=0.05):
    B = len(ref["accept_len"])
    flagged = (ref["flags"] != 0) | (out["flags"] != 0)
    ok = (out["accept_len"] == ref["accept_len"]) & (out["token"] == ref["token"])
    bad = np.nonzero(~ok & ~flagged)[0]
    assert bad.size == 0, f"mismatch on unflagged sequences {bad}: gpu {out['accept_len'][bad]}/{out['token'][bad]} " \
                          f"oracle {ref['accept_len'][bad]}/{ref['token'][bad]}"
    assert flagged.mean() <= max_flag_frac
    assert np.all(out["status"] == 0)
    return flagged


def test_c2_config_bit_exact_against_oracle(ctx):
    tgt, drf, toks = c2_inputs()
    B = tgt.shape[0]
    out, ref = run_both(ctx, tgt, drf, toks, 0.8, True, seeds=np.arange(B, dtype=np.uint64) + 7)
    assert_parity(out, ref)
    assert np.array_equal(out["draws"], ref["draws"])
    # acceptance is exercised: some sequences reject, some accept everything
    assert (ref["accept_len"] < 4).any() and (ref["accept_len"] > 0).any()


def test_c2_with_explicit_uniforms_and_stream_offsets(ctx):
    tgt, drf, toks = c2_inputs(B=16, seed=1)
    B, K = toks.shape
    offs = (np.arange(B, dtype=np.uint64) * 13) % 50
    out, ref = run_both(ctx, tgt, drf, toks, 0.8, True, seeds=np.full(B, 3, np.uint64), offsets=offs)
    assert_parity(out, ref)
    uni = np.random.default_rng(4).random((B, K + 1)).astype(np.float32)
    out, ref = run_both(ctx, tgt, drf, toks, 0.8, True, uniforms=uni)
    assert_parity(out, ref)


def test_greedy_acceptance_exact(ctx):
    tgt, drf, toks = c2_inputs(B=16, V=4096, seed=2)
    # plant argmax agreement on some positions
    for b in range(0, 16, 3):
        drf[b, :2] = tgt[b, :2]
    out, ref = run_both(ctx, tgt, drf, toks, 0.0, True, greedy=True)
    assert np.array_equal(out["accept_len"], ref["accept_len"])
    assert np.array_equal(out["token"], ref["token"])
    assert np.all(out["draws"] == 0)


def test_argmax_ties_take_last_index(ctx):
    V = 256
    tgt = np.zeros((1, 2, V), np.float32)
    drf = np.zeros((1, 1, V), np.float32)
    tgt[0, 0, [3, 200]] = 5.0
    drf[0, 0, [3, 200]] = 5.0
    out, ref = run_both(ctx, tgt, drf, np.array([[7]], np.uint32), 0.0, True, greedy=True)
    assert out["accept_len"][0] == 1 and out["token"][0] == ref["token"][0] == 255  # bonus row all zeros


def test_ragged_proposals_and_mtp_round(ctx):
    tgt, drf, toks = c2_inputs(B=12, K=4, V=2048, seed=3)
    nprop = np.array([0, 1, 2, 3, 4, 4, 3, 2, 1, 0, 4, 2], np.int32)
    for bonus in (False, True):
        out, ref = run_both(ctx, tgt, drf, toks, 0.7, bonus, seeds=np.arange(12, dtype=np.uint64), nprop=nprop)
        assert_parity(out, ref)
        assert np.all(out["accept_len"] <= nprop)


def test_sampling_only_launch_is_inverse_cdf(ctx):
    # K = 0 with bonus: plain sample_probabilities(probabilities(logits)) per sequence
    rng = np.random.default_rng(5)
    B, V = 64, 32000
    tgt = rng.normal(0, 3, (B, 1, V)).astype(np.float32)
    out, ref = run_both(ctx, tgt, np.zeros((B, 0, V), np.float32), np.zeros((B, 0), np.uint32), 0.8, True,
                        seeds=np.arange(B, dtype=np.uint64))
    assert_parity(out, ref)
    assert np.all(out["draws"] == 1)


def test_exact_sums_over_rounding_ties_and_wide_ranges(ctx):
    """Rows built to stress the exact sequential f32 sums: logits on a 1/16 grid (a few
    hundred distinct terms, each repeated, so a term that lands exactly halfway between
    two floats of the running sum does so again and again and rounds by parity), and
    logits spread over [-110, 0] (terms from 1 down
    to subnormals, so the running sum crosses many binades with terms far below its
    ulp).  Normalisers, residual masses and CDF walks must equal the oracle's
    sequential loops: accepted lengths, tokens and draws identical except flagged."""
    rng = np.random.default_rng(21)
    B, K, V = 16, 4, 32000
    tgt = np.empty((B, K + 1, V), np.float32)
    tgt[:8] = np.round(rng.normal(0, 3, (8, K + 1, V)) * 16) / 16
    tgt[8:] = -rng.uniform(0, 110, (8, K + 1, V))
    drf = tgt[:, :K].copy()
    drf[:, :, ::3] += np.round(rng.normal(0, 1, (B, K, (V + 2) // 3)) * 16).astype(np.float32) / 16
    s = R.sampler(temperature=1.0)
    toks = np.zeros((B, K), np.uint32)
    for b in range(B):
        r = R.Rng(500 + b)
        for i in range(K):
            toks[b, i] = R.sample_probabilities(s, r, R.probabilities(s, drf[b, i]))
    out, ref = run_both(ctx, tgt, drf, toks, 1.0, True, seeds=np.arange(B, dtype=np.uint64) + 40)
    assert_parity(out, ref, max_flag_frac=0.25)
    assert np.array_equal(out["draws"], ref["draws"])
    assert (ref["accept_len"] < K).any()
    # sampling-only launches over the same target rows (the CDF walk over exact sums)
    out, ref = run_both(ctx, tgt[:, :1], np.zeros((B, 0, V), np.float32), np.zeros((B, 0), np.uint32), 1.0, True,
                        seeds=np.arange(B, dtype=np.uint64) + 90)
    assert_parity(out, ref, max_flag_frac=0.25)


def test_out_of_vocab_draft_token_rejects(ctx):
    tgt, drf, toks = c2_inputs(B=4, K=2, V=1024, seed=6)
    toks[:, 0] = 5000  # q = 0 -> rejected without a draw (speculative.rs:764-767)
    out, ref = run_both(ctx, tgt, drf, toks, 0.8, True, seeds=np.arange(4, dtype=np.uint64))
    assert np.all(out["accept_len"] == 0) and np.array_equal(out["token"], ref["token"])
    assert np.all(out["draws"] == 1)


def test_zero_mass_residual_reports_error(ctx):
    # A draft token with q[x] = 0 is rejected without a draw; if p == q the residual
    # max(0, p - q) has no mass: the reference returns Err (speculative.rs:784-788).
    V = 512
    l = np.random.default_rng(7).normal(0, 1, V).astype(np.float32)
    l[5] = -np.inf
    tgt = np.stack([l, l])[None]
    drf = l[None, None]
    toks = np.array([[5]], np.uint32)
    t = lambda a, dt: torch.from_numpy(np.ascontiguousarray(a).astype(dt)).to(DEV)
    out = ctx.accept_sample(t(tgt, np.float32), t(drf, np.float32), t(toks, np.int32), A.Sampler.top_k_top_p(1.0),
                            True, seeds=t(np.array([1]), np.int64))
    assert int(out["accept_len"][0]) == 0 and int(out["status"][0]) == 1
    with pytest.raises(ValueError):
        R.accept_batch(tgt, drf, toks, R.sampler(temperature=1.0), True, seeds=np.array([1], np.uint64))


def test_speculative_sampling_preserves_target_distribution(ctx):
    # speculative.rs:926-950 on the device: 50k independent sequences, one round each.
    target = np.array([0.1, 0.2, 0.7], np.float32)
    draft = np.array([0.6, 0.3, 0.1], np.float32)
    B = 50000
    tl = np.broadcast_to(np.log(target), (B, 2, 3)).astype(np.float32)
    dl = np.broadcast_to(np.log(draft), (B, 1, 3)).astype(np.float32)
    rng = np.random.default_rng(8)
    props = rng.choice(3, size=(B, 1), p=draft / draft.sum()).astype(np.int32)
    t = lambda a, dt: torch.from_numpy(np.ascontiguousarray(a).astype(dt)).to(DEV)
    out = ctx.accept_sample(t(tl, np.float32), t(dl, np.float32), t(props, np.int32), A.Sampler.top_k_top_p(1.0),
                            False, seeds=t(np.arange(B), np.int64))
    acc = out["accept_len"].cpu().numpy()
    tok = np.where(acc == 1, props[:, 0], out["token"].cpu().numpy())
    freq = np.bincount(tok, minlength=3) / B
    assert np.max(np.abs(freq - target)) < 0.01


@pytest.mark.parametrize("greedy", [False, True])
def test_top_candidates_bit_exact(ctx, greedy):
    """Sampler::top_candidates_from_probabilities (sampler.rs:188-208) of C2 target rows
    (N(0, 3^2) logits, T = 0.8) and of rows with many exact ties: ids identical to the
    oracle's and probabilities within 2 ulps (the device's exp is correctly rounded,
    the host libm expf the oracle calls is within 1 ulp); greedy rows are exact."""
    tgt, _, _ = c2_inputs(B=8, K=4, V=32000)
    rows = tgt.reshape(-1, 32000)
    tied = np.round(np.random.default_rng(5).normal(0, 1, (4, 32000)) * 2).astype(np.float32) / 2
    rows = np.concatenate([rows, tied])
    s_ref = R.sampler(greedy=True) if greedy else R.sampler(temperature=0.8)
    s_dev = A.Sampler.greedy_sampler() if greedy else A.Sampler.top_k_top_p(0.8)
    ids, probs = ctx.top_candidates(torch.from_numpy(rows).to(DEV), s_dev, 5)
    ids, probs = ids.cpu().numpy().astype(np.uint32), probs.cpu().numpy()
    for r in range(rows.shape[0]):
        wi, wp = R.top_candidates(R.probabilities(s_ref, rows[r]), 5)
        if greedy:
            assert ids[r].tolist() == wi.tolist() and np.array_equal(probs[r], wp), r
            continue
        ulps = np.abs(probs[r].view(np.int32).astype(np.int64) - wp.view(np.int32).astype(np.int64))
        assert ulps.max() <= 2, (r, ulps)
        # an id swap is only possible between candidates the rounding cannot order
        for k in range(5):
            if ids[r][k] != wi[k]:
                assert abs(int(wp[k].view(np.int32)) - int(probs[r][k].view(np.int32))) <= 2, (r, k)


# ---------------------------------------------------------------------------
# top-k / top-p (filtered_probs, sampler.rs:226-278) and long vocabularies
# ---------------------------------------------------------------------------
def test_cli_default_sampler_on_c2_shapes(ctx):
    """The reference CLI's sampled speculation (infer.rs:72-77: T 0.7, top_k 50,
    top_p 0.9) on C2 shapes: accepted lengths, tokens and draws bit-identical to the
    oracle except on flagged draws (including a top-p cumulative within 1e-6 of p)."""
    tgt, drf, toks = c2_inputs(B=32, K=4, V=32000, T=0.7, seed=11)
    B = tgt.shape[0]
    # draft tokens from the filtered draft distribution, as the engine proposes them
    s = R.sampler(temperature=0.7, top_k=50, top_p=0.9)
    for b in range(B):
        r = R.Rng(20_000 + b)
        for i in range(4):
            toks[b, i] = R.sample_probabilities(s, r, R.probabilities(s, drf[b, i]))
    out, ref = run_both(ctx, tgt, drf, toks, 0.7, True, seeds=np.arange(B, dtype=np.uint64) + 3, top_k=50,
                        top_p=0.9)
    flagged = assert_parity(out, ref)
    assert np.array_equal(out["draws"][~flagged], ref["draws"][~flagged])
    assert (ref["accept_len"] < 4).any() and (ref["accept_len"] > 0).any()


@pytest.mark.parametrize("top_k,top_p", [(50, 0.0), (0, 0.9), (1, 0.0), (700, 0.95), (1024, 0.9), (1025, 0.0),
                                         (31999, 0.5)])
def test_top_k_top_p_variants_match_oracle(ctx, top_k, top_p):
    """top-k alone, top-p alone (several top-p pages of 4096 sorted candidates on
    the flat rows), k = 1, and both, on peaked N(0, 3^2) and flat N(0, 0.3^2) rows."""
    rng = np.random.default_rng(12 + top_k)
    B, K, V = 8, 3, 32000
    sc = np.where(np.arange(B) % 2 == 0, 3.0, 0.3).astype(np.float32)[:, None, None]
    tgt = (rng.normal(0, 1, (B, K + 1, V)) * sc).astype(np.float32)
    drf = (tgt[:, :K] + rng.normal(0, 0.5, (B, K, V)) * sc).astype(np.float32)
    s = R.sampler(temperature=0.9, top_k=top_k, top_p=top_p)
    toks = np.zeros((B, K), np.uint32)
    for b in range(B):
        r = R.Rng(30_000 + b)
        for i in range(K):
            toks[b, i] = R.sample_probabilities(s, r, R.probabilities(s, drf[b, i]))
    for bonus in (True, False):
        out, ref = run_both(ctx, tgt, drf, toks, 0.9, bonus, seeds=np.arange(B, dtype=np.uint64), top_k=top_k,
                            top_p=top_p)
        # flat rows keep ~28k tokens whose increments near the top-p cut are ~1e-5, so
        # a cut within 1e-6 of p (flagged) is common there; flagged or not, the
        # outcomes must still agree on nearly every sequence
        assert_parity(out, ref, max_flag_frac=0.6)
        same = (out["accept_len"] == ref["accept_len"]) & (out["token"] == ref["token"])
        assert same.mean() >= 0.85


@pytest.mark.parametrize("n_out", [1, 3, 49, 60])
@pytest.mark.parametrize("top_p", [0.0, 0.9])
def test_top_k_rows_with_outlier_logits(ctx, n_out, top_p):
    """Rows where n_out logits sit far above a N(0, 0.7^2) bulk, as an MTP head scores
    the token it was fed: with fewer than k = 50 outliers the top quarter of the range
    holds fewer than k logits and the top-k cut lies in the bulk (the selection's second
    banding level), with 60 it lies among the outliers.  Proposal draws (K = 0) and
    acceptance with bonus bit-identical to the oracle except flagged draws."""
    rng = np.random.default_rng(70 + n_out)
    B, K, V = 8, 3, 32000
    tgt = rng.normal(0, 0.7, (B, K + 1, V)).astype(np.float32)
    drf = (tgt[:, :K] + rng.normal(0, 0.3, (B, K, V))).astype(np.float32)
    for a in (tgt, drf):
        for b in range(B):
            for i in range(a.shape[1]):
                idx = rng.choice(V, n_out, replace=False)
                a[b, i, idx] = rng.uniform(12.0, 16.0, n_out).astype(np.float32)
    s = R.sampler(temperature=0.7, top_k=50, top_p=top_p)
    toks = np.zeros((B, K), np.uint32)
    for b in range(B):
        r = R.Rng(40_000 + b)
        for i in range(K):
            toks[b, i] = R.sample_probabilities(s, r, R.probabilities(s, drf[b, i]))
    out, ref = run_both(ctx, tgt, drf, toks, 0.7, True, seeds=np.arange(B, dtype=np.uint64) + 9, top_k=50,
                        top_p=top_p)
    assert_parity(out, ref, max_flag_frac=0.25)
    # proposal draws: one row per sequence, sampling only
    out, ref = run_both(ctx, drf[:, :1], np.zeros((B, 0, V), np.float32), np.zeros((B, 0), np.uint32), 0.7, True,
                        seeds=np.arange(B, dtype=np.uint64) + 19, top_k=50, top_p=top_p)
    assert_parity(out, ref, max_flag_frac=0.25)


@pytest.mark.parametrize("offset", [300.0, 1.0e4, -2.0e4])
def test_top_k_rows_far_from_zero(ctx, offset):
    """Logits offset far from zero with a range small against their magnitude: the band
    thresholds round at the logits' own ulp, and the selection must still keep exactly
    the top k (bit-identical draws to the oracle except flagged ones)."""
    rng = np.random.default_rng(90)
    B, K, V = 8, 3, 32000
    tgt = (offset + rng.normal(0, 1.0, (B, K + 1, V))).astype(np.float32)
    drf = (tgt[:, :K] + rng.normal(0, 0.3, (B, K, V))).astype(np.float32)
    s = R.sampler(temperature=0.7, top_k=50, top_p=0.9)
    toks = np.zeros((B, K), np.uint32)
    for b in range(B):
        r = R.Rng(50_000 + b)
        for i in range(K):
            toks[b, i] = R.sample_probabilities(s, r, R.probabilities(s, drf[b, i]))
    out, ref = run_both(ctx, tgt, drf, toks, 0.7, True, seeds=np.arange(B, dtype=np.uint64) + 29, top_k=50,
                        top_p=0.9)
    assert_parity(out, ref, max_flag_frac=0.25)


def test_top_k_keeps_lower_index_among_ties(ctx):
    """Stable total_cmp ranking: among equal logits at the top-k boundary the lower
    token ids are kept (sampler.rs:238-245), so the bonus draw can only land on them."""
    V = 1024
    l = np.full(V, -5.0, np.float32)
    l[[10, 20, 30, 40, 50]] = 2.0  # five-way tie, top_k = 3 keeps 10, 20, 30
    tgt = np.broadcast_to(l, (256, 1, V)).copy()
    out, ref = run_both(ctx, tgt, np.zeros((256, 0, V), np.float32), np.zeros((256, 0), np.uint32), 1.0, True,
                        seeds=np.arange(256, dtype=np.uint64), top_k=3)
    assert_parity(out, ref)
    assert set(out["token"].tolist()) == {10, 20, 30}


def test_long_vocabulary_rows_are_scanned_in_chunks(ctx):
    """V = 128 000 (beyond one LDS chunk of 32 768): softmax normaliser, residual
    mass and CDF carried across chunks, bit-identical to the oracle."""
    tgt, drf, toks = c2_inputs(B=6, K=3, V=128000, T=0.8, seed=13)
    out, ref = run_both(ctx, tgt, drf, toks, 0.8, True, seeds=np.arange(6, dtype=np.uint64) + 50)
    assert_parity(out, ref)
    assert np.array_equal(out["draws"], ref["draws"])
    out, ref = run_both(ctx, tgt, drf, toks, 0.8, False, seeds=np.arange(6, dtype=np.uint64) + 50, top_k=40,
                        top_p=0.9)
    assert_parity(out, ref, max_flag_frac=0.34)


@pytest.mark.parametrize("top_k,top_p", [(50, 0.9), (0, 0.8), (3, 0.0)])
def test_top_candidates_of_filtered_distributions(ctx, top_k, top_p):
    """Candidates of the filtered distribution (mtp_speculative.rs:247-250 pass the
    target distribution, i.e. after top-k / top-p): dropped tokens carry probability 0
    and ids equal the oracle's up to 2-ulp rounding swaps."""
    rng = np.random.default_rng(14)
    rows = np.concatenate([rng.normal(0, 3, (6, 32000)), rng.normal(0, 0.3, (2, 32000))]).astype(np.float32)
    s_ref = R.sampler(temperature=0.7, top_k=top_k, top_p=top_p)
    s_dev = A.Sampler.top_k_top_p(0.7, top_k=top_k, top_p=top_p)
    ids, probs = ctx.top_candidates(torch.from_numpy(rows).to(DEV), s_dev, 5)
    ids, probs = ids.cpu().numpy().astype(np.uint32), probs.cpu().numpy()
    for r in range(rows.shape[0]):
        p, tm, _ = R.probabilities(s_ref, rows[r], margins=True)
        if tm < 1e-6:
            continue  # top-p cut within rounding of p: the kept sets may differ
        wi, wp = R.top_candidates(p, 5)
        ulps = np.abs(probs[r].view(np.int32).astype(np.int64) - wp.view(np.int32).astype(np.int64))
        assert ulps.max() <= 2, (r, ulps, probs[r], wp)
        for k in range(5):
            if ids[r][k] != wi[k]:
                assert wp[k] == 0.0 or ulps[k] <= 2, (r, k)
