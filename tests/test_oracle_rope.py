"""Pins the oracle's RoPE scaling (nn/src/rope_scaling.rs, core/src/config.rs:22-96, nn/src/rope.rs:17-72).

The frequencies are checked against the reference's own tests (rope_scaling.rs:142-168) and
against what the definitions fix independently of the formulas' code:
  * linear: every frequency is the base one divided by factor;
  * NTK: theta' = theta * factor^(hd / (hd - 2)) makes the LAST frequency theta^(-(hd-2)/hd) / factor
    (the first stays 1), so an exponent mistake moves it;
  * YaRN: dimension i keeps its base frequency when it turns at least beta_fast times over the
    original context (L * f_i / 2pi >= beta_fast), takes base / factor when it turns at most
    beta_slow times, and lies strictly between in the ramp (the YaRN paper's definition of the
    correction range by rotation counts, computed here from counted rotations, not from the
    closed-form dimension);
and at the model level: a scaled model equals the float64 numpy forward given the same
frequencies, and attn_factor a equals scaling the q and k projections by a (RoPE is linear).
"""
import math

import numpy as np
import pytest

import npref
import refcpu as R


def yarn(**kw):
    d = dict(method="yarn", factor=4.0, original_max_seq_len=4096, beta_fast=32.0, beta_slow=1.0,
             attn_factor=1.138629436)
    d.update(kw)
    return d


def test_reference_yarn_boundary_kat():  # rope_scaling.rs:148-168
    base, a0 = R.rope_frequencies(64, 500000.0, 8192, None)
    y, a = R.rope_frequencies(64, 500000.0, 8192, yarn())
    assert a0 == 1.0 and a == np.float32(1.138629436)
    assert abs(base[0] - y[0]) < 1e-6
    assert abs(base[-1] / np.float32(4.0) - y[-1]) < 1e-8
    assert np.all(y[:-1] >= y[1:])


def test_base_frequencies_closed_form():
    inv, _ = R.rope_frequencies(64, 10000.0, 16, None)
    want = np.array([10000.0 ** (-2.0 * i / 64) for i in range(32)])
    assert inv[0] == 1.0
    np.testing.assert_allclose(inv, want, rtol=1e-7)


def test_linear_divides_every_frequency():
    base, _ = R.rope_frequencies(64, 10000.0, 64, None)
    lin, a = R.rope_frequencies(64, 10000.0, 64, dict(method="linear", factor=2.5, original_max_seq_len=16,
                                                      attn_factor=0.75))
    assert a == np.float32(0.75)
    assert np.array_equal(lin, base / np.float32(2.5))


@pytest.mark.parametrize("hd,factor", [(64, 4.0), (32, 2.0), (128, 8.0)])
def test_ntk_endpoints(hd, factor):  # rope_scaling.rs:14-22, 143-146
    theta = 10000.0
    ntk, _ = R.rope_frequencies(hd, theta, 64, dict(method="ntk", factor=factor, original_max_seq_len=16))
    base, _ = R.rope_frequencies(hd, theta, 64, None)
    assert ntk[0] == 1.0
    last = theta ** (-(hd - 2) / hd) / factor
    assert abs(ntk[-1] - last) <= 2e-7 * last
    assert np.all(ntk[1:] < base[1:])


@pytest.mark.parametrize("theta,hd,L,bf,bs,factor", [(500000.0, 64, 4096, 32.0, 1.0, 4.0),
                                                      (10000.0, 128, 2048, 32.0, 1.0, 8.0),
                                                      (10000.0, 32, 512, 16.0, 2.0, 2.0)])
def test_yarn_ramp_by_rotation_counts(theta, hd, L, bf, bs, factor):
    y, _ = R.rope_frequencies(hd, theta, L, yarn(factor=factor, original_max_seq_len=L, beta_fast=bf,
                                                 beta_slow=bs))
    base = np.array([theta ** (-2.0 * i / hd) for i in range(hd // 2)])
    turns = L * base / (2 * math.pi)
    fast, slow = turns >= bf, turns <= bs
    assert fast.any() and slow.any()
    np.testing.assert_allclose(y[fast], base[fast], rtol=1e-7)
    np.testing.assert_allclose(y[slow], base[slow] / factor, rtol=1e-7)
    mid = ~(fast | slow)
    assert mid.any()
    assert np.all(y[mid] < base[mid]) and np.all(y[mid] > base[mid] / factor)


def test_yarn_degenerate_range_uses_epsilon_ramp():  # linear_ramp, rope_scaling.rs:132-139
    # hd = 4 has a single ramp dimension (max_dim = 1): both corrections clamp to 1, and the
    # +0.001 widening makes dimension 1 fully interpolated rather than a 0/0.
    y, _ = R.rope_frequencies(4, 10000.0, 4096, yarn(original_max_seq_len=4096))
    assert y[0] == 1.0
    assert np.isfinite(y).all()


@pytest.mark.parametrize("bad,msg", [
    (dict(factor=1.0), "rope_scaling.factor must be finite and greater than 1.0"),
    (dict(factor=float("inf")), "rope_scaling.factor must be finite and greater than 1.0"),
    (dict(original_max_seq_len=0), "rope_scaling.original_max_seq_len must be non-zero"),
    (dict(original_max_seq_len=9000), "max_seq_len 8192 must be >= rope_scaling.original_max_seq_len 9000"),
    (dict(attn_factor=0.0), "rope_scaling.attn_factor must be finite and positive"),
    (dict(beta_slow=-1.0), "rope_scaling beta values must be finite and positive"),
    (dict(beta_fast=1.0), "rope_scaling.beta_fast must be greater than beta_slow"),
])
def test_validation_messages(bad, msg):  # config.rs:52-96
    with pytest.raises(ValueError, match="^" + msg.replace(".", r"\.") + "$"):
        R.rope_frequencies(64, 10000.0, 8192, yarn(**bad))


def test_ntk_ignores_beta_and_head_dim_two_rejected():
    R.rope_frequencies(64, 10000.0, 64, dict(method="ntk", factor=2.0, original_max_seq_len=8, beta_fast=1.0))
    with pytest.raises(ValueError, match="head_dim must be greater than 2"):
        R.rope_frequencies(2, 10000.0, 64, dict(method="linear", factor=2.0, original_max_seq_len=8))


def tiny_cfg(**kw):
    base = dict(vocab_size=97, hidden_dim=64, ffn_dim=96, n_layers=2, n_heads=4, n_kv_heads=2,
                max_seq_len=48, num_future_tokens=0)
    base.update(kw)
    return R.make_config(**base)


def rel(a, b):
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


@pytest.mark.parametrize("scaling", [
    yarn(original_max_seq_len=16, beta_fast=8.0, beta_slow=1.0, attn_factor=1.2),
    dict(method="ntk", factor=3.0, original_max_seq_len=16),
    dict(method="linear", factor=2.0, original_max_seq_len=8, attn_factor=0.9),  # model_tests.rs:37-50
])
def test_scaled_model_matches_float64_forward(scaling):
    cfg = tiny_cfg()
    m = R.Model(cfg, seed=5, std=0.08)
    m.set_rope_scaling(scaling)
    W = npref.weights(m)
    ids = R.synth_tokens(4, 2, 30, cfg.vocab_size)
    got, _ = m.kv(cfg.max_seq_len).forward(ids, 0)
    rs = R.rope_frequencies(16, cfg.rope_theta, cfg.max_seq_len, scaling)
    want, _ = npref.forward(W, cfg, ids, rs)
    assert rel(got, want) < 1e-5
    base, _ = npref.forward(W, cfg, ids)
    assert rel(got, base) > 1e-3  # the scaling is visible in the logits
    m.set_rope_scaling(None)
    again, _ = m.kv(cfg.max_seq_len).forward(ids, 0)
    assert rel(again, base) < 1e-5


def test_attn_factor_equals_scaled_qk_projections():
    cfg = tiny_cfg(n_layers=1)
    s = dict(method="linear", factor=2.0, original_max_seq_len=8, attn_factor=1.5)
    m1 = R.Model(cfg, seed=9, std=0.08)
    m1.set_rope_scaling(s)
    m2 = R.Model(cfg, seed=9, std=0.08)
    m2.set_rope_scaling(dict(s, attn_factor=1.0))
    names = {t[0]: i for i, t in enumerate(m2.tensors())}
    for n in ("blocks.0.attn.wq.weight", "blocks.0.attn.wk.weight"):
        m2.set(names[n], m2.get(names[n]) * np.float32(1.5))
    ids = R.synth_tokens(6, 1, 20, cfg.vocab_size)
    a, _ = m1.kv(cfg.max_seq_len).forward(ids, 0)
    b, _ = m2.kv(cfg.max_seq_len).forward(ids, 0)
    assert rel(a, b) < 1e-5


def test_bad_scaling_leaves_tables_unchanged():
    cfg = tiny_cfg(n_layers=1)
    m = R.Model(cfg, seed=2, std=0.08)
    ids = R.synth_tokens(1, 1, 12, cfg.vocab_size)
    before, _ = m.kv(cfg.max_seq_len).forward(ids, 0)
    with pytest.raises(ValueError, match="max_seq_len 48 must be"):
        m.set_rope_scaling(dict(method="linear", factor=2.0, original_max_seq_len=64))
    after, _ = m.kv(cfg.max_seq_len).forward(ids, 0)
    assert np.array_equal(before, after)
