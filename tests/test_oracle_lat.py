"""Pins the latent-attention MoE oracle (benchmark config 5): MLA (mla.rs:300-489)
and fine-grained MoE with shared experts (moe.rs:127-406)."""
import numpy as np
import pytest

import npref
import refcpu as R


def tiny_lat(**kw):
    base = dict(vocab_size=97, hidden_dim=64, n_layers=2, n_heads=2, max_seq_len=48, latent_dim=32, rope_dim=8,
                nope_dim=16, v_dim=12, n_experts=6, top_k=2, expert_dim=24, n_shared=2)
    base.update(kw)
    return R.make_lat_config(**base)


def synth(m, seed, std=0.2):
    for i, (name, r, c, kind) in enumerate(m.tensors()):
        if kind == R.T_NORM:
            m.set(i, 1.0 + 0.1 * R.synth_fill(seed, 1000 + i, r * c, 1.0))
        else:
            m.set(i, R.synth_fill(seed, i, r * c, std))


def rel(a, b):
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


def test_top_k_gating_kat():  # moe.rs:441-463
    idx, w = R.topk_gating(np.array([[0, 3, 1, 2], [9, 8, 7, 6]], np.float32), 2)
    assert idx.tolist() == [[1, 3], [0, 1]]
    e = np.e
    assert np.allclose(w, [[e / (e + 1), 1 / (e + 1)]] * 2, atol=1e-7)
    assert np.allclose(w.sum(-1), 1.0, atol=1e-6)
    # ties keep the lower index first (stable descending order)
    idx, _ = R.topk_gating(np.array([[1, 5, 5, 0, 5]], np.float32), 3)
    assert idx.tolist() == [[1, 2, 4]]


def test_lat_forward_matches_float64_dense_moe_and_reconstructed_mla():
    cfg = tiny_lat()
    m = R.LatModel(cfg)
    synth(m, 3)
    ids = R.synth_tokens(3, 1, 11, cfg.vocab_size)
    got, gh = m.kv(48).forward(ids, 0)
    W = npref.weights(m)
    want, wh = npref.lat_forward(W, cfg, ids)
    assert rel(got, want) < 1e-4 and rel(gh, wh) < 1e-4


def test_mla_absorption_equals_reconstruction():
    """The device path scores q_lat = up_k^T q_nope against the latent cache and
    projects P c through up_v: the same numbers as the reference's
    reconstructed K / V, up to rounding."""
    cfg = tiny_lat(n_layers=1)
    m = R.LatModel(cfg)
    synth(m, 4)
    W = npref.weights(m)
    ids = R.synth_tokens(4, 2, 9, cfg.vocab_size)
    a, _ = npref.lat_forward(W, cfg, ids, absorbed=False)
    b, _ = npref.lat_forward(W, cfg, ids, absorbed=True)
    assert rel(a, b) < 1e-12


def test_cached_prefix_equals_full_forward():  # model_tests.rs:178-203 for the latent cache
    cfg = tiny_lat()
    m = R.LatModel(cfg)
    synth(m, 5)
    ids = R.synth_tokens(5, 3, 14, cfg.vocab_size)
    full, _ = m.kv(48).forward(ids, 0)
    kv = m.kv(48)
    a, _ = kv.forward(ids[:9], 0)
    b, _ = kv.forward(ids[9:], 9)
    assert rel(np.concatenate([a, b]), full) < 1e-5
    # rollback by index then a different suffix (mtp_speculative.rs:284-313)
    kv.truncate(9)
    c, _ = kv.forward(ids[9:12], 9)
    assert rel(c, b[:3]) < 1e-6


def test_shared_experts_are_added_for_every_token():  # moe.rs:544-572
    cfg0 = tiny_lat(n_layers=1, n_shared=0)
    cfg1 = tiny_lat(n_layers=1, n_shared=1)
    m0, m1 = R.LatModel(cfg0), R.LatModel(cfg1)
    synth(m1, 6)
    names1 = [t[0] for t in m1.tensors()]
    for i, (name, r, c, kind) in enumerate(m0.tensors()):
        m0.set(i, m1.get(names1.index(name)))
    W1 = npref.weights(m1)
    ids = R.synth_tokens(6, 4, 5, cfg0.vocab_size)
    # with vs without the shared expert differ by exactly that expert's FFN output
    pre = "blocks.0."
    x = W1["embedding.weight"][ids.astype(np.int64)]
    pos = np.arange(len(ids), dtype=np.float64)
    y0 = npref.lat_block(W1, pre, x, cfg0, pos)
    y1 = npref.lat_block(W1, pre, x, cfg1, pos)
    a, _ = m0.kv(48).forward(ids, 0)
    b, _ = m1.kv(48).forward(ids, 0)
    assert not np.allclose(a, b)
    assert np.max(np.abs(y1 - y0)) > 1e-3


def test_synthetic_latent_cache_is_deterministic():
    cfg = tiny_lat(kv_format=R.KV_F16)
    m = R.LatModel(cfg)
    synth(m, 7)
    ids = np.array([3, 4], np.uint32)
    k1, k2 = m.kv(48), m.kv(48)
    k1.fill_synthetic(9, 20)
    k2.fill_synthetic(9, 20)
    a, _ = k1.forward(ids, 20)
    b, _ = k2.forward(ids, 20)
    assert np.array_equal(a, b)


def test_untied_head_reads_lm_head():
    """tie_embeddings false (LmHead::untied_with_qat, model.rs:239-248): lm_head.weight is the
    tensor after final_norm and the logits are the final normed hidden state times it; the
    embedding still feeds the input rows (same hidden state as the tied model)."""
    tied = R.LatModel(tiny_lat())
    untied = R.LatModel(tiny_lat(untied_lm_head=1))
    names = [t[0] for t in untied.tensors()]
    assert names[:-1] == [t[0] for t in tied.tensors()] and names[-1] == "lm_head.weight"
    assert untied.tensors()[-1][1:3] == (97, 64)
    synth(tied, 3)
    synth(untied, 3)
    kv_t, kv_u = tied.kv(48), untied.kv(48)
    ids = np.array([5, 17, 96, 0, 41], np.uint32)
    lt, ht = kv_t.forward(ids, 0)
    lu, hu = kv_u.forward(ids, 0)
    assert np.array_equal(ht, hu)  # everything before the head is shared
    head = untied.get(len(names) - 1).astype(np.float64)
    emb = untied.get(0).astype(np.float64)
    assert rel(lu, hu.astype(np.float64) @ head.T) < 1e-5
    assert rel(lt, ht.astype(np.float64) @ emb.T) < 1e-5
    assert rel(lu, lt) > 0.1
    tied.close()
    untied.close()
