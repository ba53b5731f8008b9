"""RoPE scaling (aarh_set_rope_scaling, rope_scaling.rs:24-92 via RopeCache::from_config,
rope.rs:17-72) and the untied LM head (LmHead::untied_with_qat, model.rs:239-262) on the
device against the oracle on identical random-init weights, plus both read from a GGUF
checkpoint's config.  Bars as the other forward tests: f32 contexts 1e-4 relative per
row, quantised contexts 2e-3; a scaled table must move the logits well beyond that."""
import numpy as np
import pytest

import aarambh_hip as A
import refcpu as R
import refgguf as G
from gpu_util import make_pair, rel_rows

pytestmark = pytest.mark.gpu

KW = dict(vocab_size=1024, hidden_dim=256, ffn_dim=704, n_layers=2, n_heads=8, n_kv_heads=2, max_seq_len=96,
          num_future_tokens=3)
SCALINGS = [
    A.RopeScaling("yarn", factor=4.0, original_max_seq_len=24, beta_fast=8.0, beta_slow=1.0, attn_factor=1.1),
    A.RopeScaling("ntk", factor=3.0, original_max_seq_len=32),
    A.RopeScaling("linear", factor=2.0, original_max_seq_len=48, attn_factor=0.9),
]


def as_dict(s):
    return None if s is None else dict(method=s.method, factor=s.factor, original_max_seq_len=s.original_max_seq_len,
                                       beta_fast=s.beta_fast, beta_slow=s.beta_slow, attn_factor=s.attn_factor)


def prefill_verify_mtp(ref, hip, tol, seed=3):
    """Prefill 20 tokens, verify 4 at offset 20, one MTP head call: device vs oracle."""
    ids = R.synth_tokens(seed, 1, 24, hip.cfg.vocab_size)
    hip.kv_reset(0)
    kv = ref.kv(hip.cfg.max_seq_len)
    wl, wh = kv.forward(ids[:20], 0)
    gl, gh = hip.forward_with_cache_output(ids[None, :20], [0])
    assert rel_rows(gl[0], wl).max() < tol and rel_rows(gh[0], wh).max() < tol
    wl2, _ = kv.forward(ids[20:], 20)
    gl2, _ = hip.forward_with_cache_output(ids[None, 20:], [20])
    assert rel_rows(gl2[0], wl2).max() < tol
    anchor = gh[0, -1]
    got = hip.forward_mtp_head(1, anchor[None], ids[None, 20:22])
    want = ref.mtp_head(1, anchor, ids[20:22])
    assert rel_rows(got, want[None]).max() < tol
    return wl


@pytest.mark.parametrize("scaling", SCALINGS, ids=lambda s: s.method)
def test_scaled_rope_matches_oracle(scaling):
    ref, hip = make_pair(seed=11, std=0.05, **KW)
    base = prefill_verify_mtp(ref, hip, 1e-4)
    ref.set_rope_scaling(as_dict(scaling))
    hip.set_rope_scaling(scaling)
    scaled = prefill_verify_mtp(ref, hip, 1e-4)
    assert rel_rows(scaled, base).max() > 1e-2  # the tables changed the result
    ref.set_rope_scaling(None)
    hip.set_rope_scaling(None)
    again = prefill_verify_mtp(ref, hip, 1e-4)
    assert np.array_equal(again, base)
    hip.close()


def test_rope_scaling_errors_match_oracle_and_keep_tables():
    ref, hip = make_pair(seed=12, std=0.05, **dict(KW, num_future_tokens=0))
    ids = R.synth_tokens(5, 1, 16, 1024)
    before, _ = hip.forward_with_cache_output(ids[None], [0])
    for bad in (A.RopeScaling("yarn", factor=0.5, original_max_seq_len=16),
                A.RopeScaling("linear", factor=2.0, original_max_seq_len=200),
                A.RopeScaling("yarn", factor=2.0, original_max_seq_len=16, beta_fast=1.0, beta_slow=2.0),
                A.RopeScaling("ntk", factor=2.0, original_max_seq_len=16, attn_factor=float("nan"))):
        with pytest.raises(ValueError) as want:
            ref.set_rope_scaling(as_dict(bad))
        with pytest.raises(A.ConfigError) as got:
            hip.set_rope_scaling(bad)
        assert str(got.value) == str(want.value)
    after, _ = hip.forward_with_cache_output(ids[None], [0])
    assert np.array_equal(before, after)
    hip.close()


def test_rope_scaling_reaches_captured_graphs():
    # Verify-shaped forwards replay captured graphs; the setter rewrites the tables those
    # graphs read, so a replay after it uses the new frequencies.
    ref, hip = make_pair(seed=13, std=0.05, **dict(KW, num_future_tokens=0))
    ids = R.synth_tokens(6, 1, 28, 1024)
    hip.forward_with_cache_output(ids[None, :24], [0])
    for _ in range(3):
        hip.forward_with_cache_output(ids[None, 24:], [24])
    s = SCALINGS[0]
    ref.set_rope_scaling(as_dict(s))
    hip.set_rope_scaling(s)
    kv = ref.kv(96)
    kv.forward(ids[:24], 0)
    hip.kv_reset(0)
    hip.forward_with_cache_output(ids[None, :24], [0])
    for _ in range(2):
        gl, _ = hip.forward_with_cache_output(ids[None, 24:], [24])
        wl, _ = kv.forward(ids[24:], 24)
        assert rel_rows(gl[0], wl).max() < 1e-4
    hip.close()


@pytest.mark.parametrize("wfmt,lmfmt,kvfmt,tol", [(A.W_F32, 0, A.KV_F32, 1e-4), (A.W_F32, 1, A.KV_F32, 1e-4),
                                                   (A.W_INT4_G128, 1, A.KV_F16, 2e-3)])
def test_untied_lm_head_matches_oracle(wfmt, lmfmt, kvfmt, tol):
    kw = dict(KW, ffn_dim=768, weight_format=wfmt, lm_head_format=lmfmt, kv_format=kvfmt, tie_embeddings=False)
    ref, hip = make_pair(seed=14, std=0.05, **kw)
    names = [t[0] for t in hip.tensors()]
    assert names[-1] == "lm_head.weight" and hip.tensors()[-1][1:3] == (1024, 256)
    prefill_verify_mtp(ref, hip, tol)
    # the head really is separate: changing lm_head.weight moves the logits, the embedding stays
    ids = R.synth_tokens(8, 1, 12, 1024)
    hip.kv_reset(0)
    l0, h0 = hip.forward_with_cache_output(ids[None], [0])
    w = R.synth_fill(99, 0, 1024 * 256, 0.05)
    hip.load_f32(len(names) - 1, w)
    ref.set(len(names) - 1, w)
    hip.kv_reset(0)
    l1, h1 = hip.forward_with_cache_output(ids[None], [0])
    wl, _ = ref.kv(96).forward(ids, 0)
    assert np.array_equal(h0, h1) and rel_rows(l1[0], l0[0]).max() > 0.1
    assert rel_rows(l1[0], wl).max() < tol
    hip.close()


def checkpoint_tensors(ref, seed):
    rng = np.random.default_rng(seed)
    out = {}
    for name, r, c, kind in ref.tensors():
        if kind == R.T_NORM:
            out[name] = (1 + 0.1 * rng.normal(size=c)).astype(np.float32)
        else:
            out[name] = rng.normal(0, 0.03, (r, c)).astype(np.float32)
    return out


def test_gguf_with_untied_head_and_rope_scaling(tmp_path):
    shape = {k: KW[k] for k in KW}
    rs = dict(method="yarn", factor=4.0, original_max_seq_len=24, beta_fast=8.0, beta_slow=1.0, attn_factor=1.2)
    ref = R.Model(R.make_config(untied_lm_head=1, **shape))
    vals = checkpoint_tensors(ref, 21)
    path = str(tmp_path / "m.gguf")
    G.save_gguf(path, G.model_config_json(**shape, tie_embeddings=False, rope_scaling=rs), "Q80", vals)
    cfg = A.ModelConfig.from_gguf(path)
    assert cfg.tie_embeddings is False
    assert cfg.rope_scaling == A.RopeScaling(**rs)
    hip = A.HipModel(cfg, max_batch=1, max_rows=64)
    assert hip.load_gguf(path) == len(hip.tensors()) == len(ref.tensors())
    _, dec = G.load_gguf_tensors(path)
    for i, (name, *_rest) in enumerate(ref.tensors()):
        ref.set(i, dec[name])
    ref.set_rope_scaling(rs)
    prefill_verify_mtp(ref, hip, 1e-4)
    # a context created without scaling takes the checkpoint's tables at load
    plain = A.HipModel(A.ModelConfig(**shape, tie_embeddings=False), max_batch=1, max_rows=64)
    plain.load_gguf(path)
    prefill_verify_mtp(ref, plain, 1e-4)
    plain.close()
    # a checkpoint without rope_scaling restores the unscaled tables
    p2 = str(tmp_path / "n.gguf")
    G.save_gguf(p2, G.model_config_json(**shape, tie_embeddings=False), "Q80", vals)
    hip.load_gguf(p2)
    ref.set_rope_scaling(None)
    prefill_verify_mtp(ref, hip, 1e-4)
    # tie mismatch and an invalid scaling are refused
    tied = A.HipModel(A.ModelConfig(**shape), max_batch=1, max_rows=64)
    with pytest.raises(A.ConfigError, match="tie_embeddings false"):
        tied.load_gguf(path)
    p3 = str(tmp_path / "o.gguf")
    G.save_gguf(p3, G.model_config_json(**shape, tie_embeddings=False, rope_scaling=dict(rs, factor=1.0)), "Q80",
                vals)
    with pytest.raises(A.ConfigError, match="rope_scaling.factor must be finite and greater than 1.0"):
        hip.load_gguf(p3)
    p4 = str(tmp_path / "p.gguf")
    G.save_gguf(p4, G.model_config_json(**shape, tie_embeddings=False, rope_scaling=dict(rs, method="dynamic")),
                "Q80", vals)
    with pytest.raises(A.CheckpointError, match="method"):
        hip.load_gguf(p4)
    tied.close()
    hip.close()
    ref.close()
