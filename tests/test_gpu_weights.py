"""Checkpoints into a device context (aarh_load_gguf / aarh_load_safetensors): the
device forward and MTP head of a context loaded from a file equal the oracle's with
the tensors the oracle decodes from the same file (decode rules of gguf.rs:143-241 and
load_model_with_dtype, weights/src/lib.rs:68-79).  Bars: f32 contexts within 1e-4
relative per row (same f32 weights on both sides), quantised contexts within 2e-3
(each side quantises the decoded f32 values with its own codec); error kinds as the
reference reports them."""
import json
import os
import struct

import numpy as np
import pytest

import aarambh_hip as A
import refcpu as R
import refgguf as G
from gpu_util import rel_rows

pytestmark = pytest.mark.gpu

KW = dict(vocab_size=1024, hidden_dim=256, ffn_dim=704, n_layers=2, n_heads=8, n_kv_heads=2, max_seq_len=96,
          num_future_tokens=2)


def checkpoint_tensors(seed=7, **kw):
    """Named f32 tensors in the reference's checkpoint shapes (1-D norms)."""
    rc = R.make_config(**kw)
    ref = R.Model(rc)
    rng = np.random.default_rng(seed)
    out = {}
    for name, r, c, kind in ref.tensors():
        if kind == R.T_NORM:
            out[name] = (1 + 0.1 * rng.normal(size=c)).astype(np.float32)
        else:
            out[name] = rng.normal(0, 0.03, (r, c)).astype(np.float32)
    ref.close()
    return out


def oracle_with(values, **kw):
    ref = R.Model(R.make_config(**kw))
    for i, (name, r, c, kind) in enumerate(ref.tensors()):
        ref.set(i, values[name])
    return ref


def compare(ref, hip, tol, seed=3):
    ids = R.synth_tokens(seed, 1, 24, hip.cfg.vocab_size)
    kv = ref.kv(hip.cfg.max_seq_len)
    wl, wh = kv.forward(ids[:20], 0)
    gl, gh = hip.forward_with_cache_output(ids[None, :20], [0])
    assert rel_rows(gl[0], wl).max() < tol and rel_rows(gh[0], wh).max() < tol
    wl, _ = kv.forward(ids[20:], 20)
    gl, _ = hip.forward_with_cache_output(ids[None, 20:], [20])
    assert rel_rows(gl[0], wl).max() < tol
    anchor = gh[0, -1]
    got = hip.forward_mtp_head(0, anchor[None], ids[None, 20:21])
    want = ref.mtp_head(0, anchor, ids[20:21])
    assert rel_rows(got, want[None]).max() < tol


@pytest.mark.parametrize("fmt", ["Q4KM", "Q80"])
def test_gguf_into_f32_context(tmp_path, fmt):
    vals = checkpoint_tensors(**KW)
    vals["blocks.0.attn.extra_conv.weight"] = np.ones((3, 5), np.float32)  # not a context tensor: ignored
    path = str(tmp_path / "m.gguf")
    G.save_gguf(path, G.model_config_json(**{k: KW[k] for k in KW}), fmt, vals)
    _, dec = G.load_gguf_tensors(path)
    cfg = A.ModelConfig.from_gguf(path)
    want = A.ModelConfig(**KW)
    for f in ("vocab_size", "hidden_dim", "ffn_dim", "n_layers", "n_heads", "n_kv_heads", "max_seq_len",
              "num_future_tokens"):
        assert getattr(cfg, f) == getattr(want, f), f
    hip = A.HipModel(cfg, max_batch=1, max_rows=64)
    assert hip.load_gguf(path) == len(hip.tensors())
    ref = oracle_with(dec, **KW)
    compare(ref, hip, 1e-4)
    hip.close()
    ref.close()


def test_gguf_into_int4_context(tmp_path):
    shape = dict(KW, ffn_dim=768)  # quantised contexts take ffn_dim in whole 128-groups
    kw = dict(shape, weight_format=A.W_INT4_G128, lm_head_format=1, kv_format=A.KV_INT8)
    vals = checkpoint_tensors(seed=8, **shape)
    path = str(tmp_path / "m.gguf")
    G.save_gguf(path, G.model_config_json(**shape), "Q4KM", vals)
    _, dec = G.load_gguf_tensors(path)
    hip = A.HipModel(A.ModelConfig.from_gguf(path, weight_format=A.W_INT4_G128, lm_head_format=1,
                                             kv_format=A.KV_INT8), max_batch=1, max_rows=64)
    hip.load_gguf(path)
    ref = oracle_with(dec, **kw)
    compare(ref, hip, 2e-3)
    hip.close()
    ref.close()


@pytest.mark.parametrize("dtype", ["F32", "BF16", "F16"])
def test_safetensors_into_f32_context(tmp_path, dtype):
    vals = checkpoint_tensors(seed=9, **KW)
    path = str(tmp_path / "m.safetensors")
    G.save_safetensors(path, vals, dtype)
    hip = A.HipModel(A.ModelConfig(**KW), max_batch=1, max_rows=64)
    assert hip.load_safetensors(path) == len(hip.tensors())
    ref = oracle_with(G.safetensors_values(vals, dtype), **KW)
    compare(ref, hip, 1e-4)
    hip.close()
    ref.close()


def test_checkpoint_errors(tmp_path):
    kw = dict(KW, n_layers=1)
    vals = checkpoint_tensors(seed=10, **kw)
    hip = A.HipModel(A.ModelConfig(**kw), max_batch=1, max_rows=64)

    def gguf(config, tensors, name):
        p = str(tmp_path / name)
        G.save_gguf(p, config, "Q80", tensors)
        return p

    base = G.model_config_json(**kw)
    with pytest.raises(A.ConfigError):  # a different model shape
        hip.load_gguf(gguf(dict(base, ffn_dim=768), vals, "a.gguf"))
    with pytest.raises(A.ConfigError, match="tie_embeddings"):  # an untied head into a tied context
        hip.load_gguf(gguf(dict(base, tie_embeddings=False), vals, "b.gguf"))
    with pytest.raises(A.CheckpointError, match="tie_embeddings"):  # serde requires the field
        hip.load_gguf(gguf({k: v for k, v in base.items() if k != "tie_embeddings"}, vals, "b2.gguf"))
    with pytest.raises(A.UnsupportedError):  # a layer variant the device does not run
        hip.load_gguf(gguf(dict(base, moe={"num_experts": 4}), vals, "c.gguf"))
    short = {k: v for k, v in vals.items() if k != "blocks.0.ffn.w_up.weight"}
    with pytest.raises(A.CheckpointError, match="w_up"):
        hip.load_gguf(gguf(base, short, "d.gguf"))
    bad = dict(vals, **{"blocks.0.attn.wo.weight": np.zeros((256, 128), np.float32)})
    with pytest.raises(A.ShapeError):
        hip.load_gguf(gguf(base, bad, "e.gguf"))
    with pytest.raises(A.IoError):
        hip.load_safetensors(str(tmp_path / "missing.safetensors"))
    p = str(tmp_path / "f.safetensors")
    G.save_safetensors(p, short)
    with pytest.raises(A.CheckpointError, match="w_up"):
        hip.load_safetensors(p)
    # the context still works after failed loads
    G.save_safetensors(p, vals)
    hip.load_safetensors(p)
    ref = oracle_with(vals, **kw)
    ids = R.synth_tokens(4, 1, 8, kw["vocab_size"])
    wl, _ = ref.kv(96).forward(ids, 0)
    gl, _ = hip.forward_with_cache_output(ids[None], [0])
    assert rel_rows(gl[0], wl).max() < 1e-4
    hip.close()
    ref.close()
