"""Parity of the latent-attention MoE decoder on the device (benchmark config 5:
MLA mla.rs:300-489 with the latent cache, fine-grained top-k MoE with shared
experts moe.rs:127-406) against the oracle on identical random-init weights.
Bar: logits and final hidden states within 2e-3 relative (max|d|/max|ref| per
row).  The device evaluates attention in the latent space (absorbed up_k /
up_v) where the oracle reconstructs K and V, and routes only the selected rows
through each expert where the reference runs every expert densely; both are
the same function up to rounding.  A row whose k-th and (k+1)-th router logits
are within GAP_FLAG of each other in some layer can pick a different expert
than an f32 CPU path (the analogue of the flagged near-tie draws of the
acceptance test); sequences holding such a row are reported, not compared."""
import numpy as np
import pytest

import aarambh_hip as A
import refcpu as R
from gpu_util import rel_rows

pytestmark = pytest.mark.gpu
TOL = 2e-3
GAP_FLAG = 1e-4


def small_kw(**over):
    kw = dict(vocab_size=1024, hidden_dim=256, n_layers=2, n_heads=4, max_seq_len=128, latent_dim=128, rope_dim=32,
              nope_dim=32, v_dim=32, n_experts=8, top_k=2, expert_dim=128, n_shared=1, expert_format=A.W_INT4_G128,
              attn_format=A.W_INT8_ROW, lm_head_format=1, kv_format=A.KV_F16)
    kw.update(over)
    return kw


def lat_pair(seed, std, max_batch, max_rows, **kw):
    rc = R.make_lat_config(**kw)
    ref = R.LatModel(rc)
    ref.init_synthetic(seed, std)
    hip = A.HipLatModel(A.LatConfig(**kw), max_batch=max_batch, max_rows=max_rows)
    hip.init_synthetic(seed, std)
    return ref, hip


def compare(gl, gh, want, gaps, S):
    """gl/gh [B, S, *]; want = [(logits, hidden)] per sequence; gaps [B*S].
    Returns the number of sequences compared."""
    checked = 0
    for b, (wl, wh) in enumerate(want):
        if np.min(gaps[b * S:(b + 1) * S]) < GAP_FLAG:
            print(f"sequence {b}: router near-tie (gap {np.min(gaps[b * S:(b + 1) * S]):.2e}), not compared")
            continue
        el, eh = rel_rows(gl[b], wl).max(), rel_rows(gh[b], wh).max()
        assert el < TOL and eh < TOL, (b, el, eh)
        checked += 1
    return checked


FORMATS = [(A.W_INT4_G128, A.W_INT8_ROW, 1), (A.W_INT8_ROW, A.W_BF16, 0), (A.W_BF16, A.W_F32, 1),
           (A.W_INT4_G128, A.W_INT4_G128, 1)]


@pytest.mark.parametrize("efmt,afmt,lmfmt", FORMATS)
def test_lat_prefill_verify_rollback(efmt, afmt, lmfmt):
    kw = small_kw(expert_format=efmt, attn_format=afmt, lm_head_format=lmfmt)
    print("lat small", kw, flush=True)
    ref, hip = lat_pair(5, 0.05, 3, 128, **kw)
    B, P, K = 3, 37, 4
    ids = R.synth_tokens(5, 3, B * (P + K), kw["vocab_size"]).reshape(B, P + K)
    kvs = [ref.kv(128) for _ in range(B)]
    # prefill (many-row GEMM path), verify K tokens (GEMV path), rollback + shorter replay
    steps = [(0, P), (P, P + K), (P, P + 2)]
    total = 0
    for lo, hi in steps:
        gl, gh = hip.forward_with_cache_output(ids[:, lo:hi], [lo] * B)
        gaps = hip.router_gaps()
        want = []
        for b in range(B):
            kvs[b].truncate(lo)
            want.append(kvs[b].forward(ids[b, lo:hi], lo))
        total += compare(gl, gh, want, gaps, hi - lo)
    assert total >= 2 * len(steps)
    assert hip.kv_len(2) == P + 2
    counts = hip.expert_counts()
    assert (counts[:, :kw["n_experts"]].sum(1) == B * 2 * kw["top_k"]).all()
    assert (counts[:, kw["n_experts"]:] == B * 2).all()
    hip.close()


def test_lat_ragged_offsets_and_host_loaded_weights():
    """Per-sequence offsets (different cache lengths in one batch) and weights
    loaded from host f32 values with non-unit norm weights."""
    kw = small_kw(n_layers=1, n_experts=6, top_k=3, n_shared=2)
    rc = R.make_lat_config(**kw)
    ref = R.LatModel(rc)
    hip = A.HipLatModel(A.LatConfig(**kw), max_batch=2, max_rows=64)
    for i, (name, r, c, kind) in enumerate(ref.tensors()):
        if kind == R.T_NORM:
            raw = 1.0 + 0.2 * R.synth_fill(7, 500 + i, r * c, 1.0)
        else:
            raw = R.synth_fill(7, i, r * c, 1.0 / np.sqrt(c) if name.endswith("router.weight") else 0.05)
        ref.set(i, raw)
        hip.load_f32(i, raw)
    ids = R.synth_tokens(7, 1, 40, kw["vocab_size"])
    kvs = [ref.kv(128), ref.kv(128)]
    # sequence 0 holds 20 tokens, sequence 1 holds 9
    hip.forward_with_cache_output(ids[None, :20], [0], slots=[0])
    hip.forward_with_cache_output(ids[None, 20:29], [0], slots=[1])
    kvs[0].forward(ids[:20], 0)
    kvs[1].forward(ids[20:29], 0)
    nxt = np.stack([ids[29:32], ids[32:35]])
    gl, gh = hip.forward_with_cache_output(nxt, [20, 9], slots=[0, 1])
    gaps = hip.router_gaps()
    want = [kvs[0].forward(nxt[0], 20), kvs[1].forward(nxt[1], 9)]
    assert compare(gl, gh, want, gaps, 3) >= 1
    hip.close()


def test_lat_c5_shape_one_layer():
    """benchmark config 5 widths (d_model 2048, latent 512 + rope 64, 16 heads,
    64 experts top-6 of width 1408 + 2 shared, INT4 experts, vocab 32000) at one
    layer over a 1000-token synthetic latent cache; batch 4 x 5 rows (GEMM path)
    and batch 1 x 5 rows (GEMV path)."""
    kw = dict(vocab_size=32000, hidden_dim=2048, n_layers=1, n_heads=16, max_seq_len=1056, latent_dim=512,
              rope_dim=64, nope_dim=128, v_dim=128, n_experts=64, top_k=6, expert_dim=1408, n_shared=2,
              expert_format=A.W_INT4_G128, attn_format=A.W_INT4_G128, lm_head_format=1, kv_format=A.KV_F16)
    print("lat c5 one layer: building models", flush=True)
    ref, hip = lat_pair(11, 0.02, 5, 64, **kw)
    T, S, B = 1000, 5, 4
    kvs = []
    for b in range(B + 1):
        hip.kv_fill_synthetic(b, T, seed=100 + b)
        kv = ref.kv(1056)
        kv.fill_synthetic(100 + b, T)
        kvs.append(kv)
    ids = R.synth_tokens(11, 5, (B + 1) * S, kw["vocab_size"]).reshape(B + 1, S)
    print("lat c5 one layer: batch 4", flush=True)
    gl, gh = hip.forward_with_cache_output(ids[:B], [T] * B, slots=list(range(B)))
    gaps = hip.router_gaps()
    want = [kvs[b].forward(ids[b], T, nthreads=16) for b in range(B)]
    n4 = compare(gl, gh, want, gaps, S)
    print("lat c5 one layer: batch 1", flush=True)
    gl, gh = hip.forward_with_cache_output(ids[B:], [T], slots=[B])
    gaps = hip.router_gaps()
    n1 = compare(gl, gh, [kvs[B].forward(ids[B], T, nthreads=16)], gaps, S)
    assert n4 + n1 >= 3
    hip.close()


def test_lat_bench_shape_properties():
    """The bench batch (32 sequences x 5 rows = 160 rows over a 4096-token cache)
    at reduced depth: routed-count invariants, bit-identical repeat, and rollback
    + replay giving the same logits (the cache rows past the rollback point are
    rewritten, not appended)."""
    kw = dict(vocab_size=32000, hidden_dim=2048, n_layers=2, n_heads=16, max_seq_len=4160, latent_dim=512,
              rope_dim=64, nope_dim=128, v_dim=128, n_experts=64, top_k=6, expert_dim=1408, n_shared=2,
              expert_format=A.W_INT4_G128, attn_format=A.W_INT4_G128, lm_head_format=1, kv_format=A.KV_F16)
    hip = A.HipLatModel(A.LatConfig(**kw), max_batch=32, max_rows=160)
    hip.init_synthetic(12, 0.02)
    B, S, T = 32, 5, 4096
    for b in range(B):
        hip.kv_fill_synthetic(b, T, seed=200 + b)
    ids = R.synth_tokens(12, 9, B * S, kw["vocab_size"]).reshape(B, S)
    a, ah = hip.forward_with_cache_output(ids, [T] * B)
    assert np.isfinite(a).all() and np.isfinite(ah).all()
    counts = hip.expert_counts()
    assert (counts[:, :64].sum(1) == B * S * 6).all() and (counts[:, 64:] == B * S).all()
    for b in range(B):
        hip.restore(T, slot=b)
    b2, _ = hip.forward_with_cache_output(ids, [T] * B)
    assert np.array_equal(a, b2)
    # one sequence alone (GEMV path) agrees with its row of the batch within the bar
    for b in range(B):
        hip.restore(T, slot=b)
    c, _ = hip.forward_with_cache_output(ids[3:4], [T], slots=[3])
    assert rel_rows(c[0], a[3]).max() < TOL
    hip.close()


def test_lat_c5_bench_shape_vs_oracle():
    """The config-5 bench batch against the oracle: one C5-width layer (INT4 experts
    and MLA projections, latent 512 + rope 64, 16 heads, 64 experts top-6 + 2 shared),
    32 sequences x 5 verify rows over synthetic latent caches of about 4096 tokens.
    At this shape the latent attention streams about 32 blocks per chunk (a few long
    chunks per sequence) and the projections and experts take the many-row (160-row)
    GEMM path.  Odd sequences hold ragged cache lengths, so their chunks end inside a
    32-token block.  A final batch-1 forward covers the GEMV path at the same cache
    length.  Every sequence without a router near-tie must match the oracle
    (mla.rs:402-489, moe.rs:212-340) within 2e-3."""
    kw = dict(vocab_size=32000, hidden_dim=2048, n_layers=1, n_heads=16, max_seq_len=4160, latent_dim=512,
              rope_dim=64, nope_dim=128, v_dim=128, n_experts=64, top_k=6, expert_dim=1408, n_shared=2,
              expert_format=A.W_INT4_G128, attn_format=A.W_INT4_G128, lm_head_format=1, kv_format=A.KV_F16)
    B, S = 32, 5
    print("lat c5 bench shape: building models", flush=True)
    ref, hip = lat_pair(13, 0.02, B + 1, B * S, **kw)
    lens = [4096 if b % 2 == 0 else 4096 - 3 - 13 * b for b in range(B)] + [4096]
    assert any((t + S) % 32 for t in lens)
    kvs = []
    for b, t in enumerate(lens):
        hip.kv_fill_synthetic(b, t, seed=300 + b)
        kv = ref.kv(4160)
        kv.fill_synthetic(300 + b, t)
        kvs.append(kv)
    ids = R.synth_tokens(13, 5, (B + 1) * S, kw["vocab_size"]).reshape(B + 1, S)
    print("lat c5 bench shape: batch 32 x 5 rows", flush=True)
    gl, gh = hip.forward_with_cache_output(ids[:B], lens[:B], slots=list(range(B)))
    gaps = hip.router_gaps()
    counts = hip.expert_counts()
    assert (counts[:, :64].sum(1) == B * S * 6).all() and (counts[:, 64:] == B * S).all()
    want = []
    for b in range(B):
        want.append(kvs[b].forward(ids[b], lens[b], nthreads=16))
        if b % 8 == 7:
            print(f"lat c5 bench shape: oracle {b + 1}/{B}", flush=True)
    n32 = compare(gl, gh, want, gaps, S)
    print(f"lat c5 bench shape: {n32} of {B} sequences compared; batch 1", flush=True)
    gl, gh = hip.forward_with_cache_output(ids[B:], [lens[B]], slots=[B])
    gaps = hip.router_gaps()
    n1 = compare(gl, gh, [kvs[B].forward(ids[B], lens[B], nthreads=16)], gaps, S)
    assert n32 >= B - 4 and n32 + n1 >= B - 3
    hip.close()


def test_lat_packed_int4_tensors_equal_device_quantisation():
    """Every INT4 tensor of the latent decoder (MLA projections incl. up_k / up_v, the
    router, routed and shared experts) loaded as a PackedInt4Tensor with the quant
    crate's group-128 codes and f32 scales holds exactly what the device quantiser makes
    of the same f32 weights: logits and hidden states bit-identical; a group-256 load
    matches the oracle within the bar."""
    kw = small_kw(n_layers=1, attn_format=A.W_INT4_G128)
    a = A.HipLatModel(A.LatConfig(**kw), max_batch=1, max_rows=64)
    b = A.HipLatModel(A.LatConfig(**kw), max_batch=1, max_rows=64)
    c = A.HipLatModel(A.LatConfig(**kw), max_batch=1, max_rows=64)
    ref = R.LatModel(R.make_lat_config(**dict(kw, attn_format=A.W_F32, expert_format=A.W_F32)))
    n_packed = 0
    for i, (name, r, cc, kind) in enumerate(a.tensors()):
        raw = R.synth_fill(19, i, r * cc, 0.05) if kind != R.T_NORM else np.ones(r * cc, np.float32)
        a.load_f32(i, raw)
        if kind == R.T_LINEAR:
            data, sc, zz = R.quantise_i4(raw, 128)
            b.load_packed_i4(i, A.PackedInt4Tensor((r, cc), 128, data, sc, zz))
            d2, s2, z2 = R.quantise_i4(raw, 256)
            c.load_packed_i4(i, A.PackedInt4Tensor((r, cc), 256, d2, s2, z2))
            # the oracle holds the device's stored function: fp16 scales of the group-256 codes
            ref.set(i, R.dequantise_i4(d2, r * cc, 256, s2.astype(np.float16).astype(np.float32), z2))
            n_packed += 1
        else:
            b.load_f32(i, raw)
            c.load_f32(i, raw)
            ref.set(i, raw)
    assert n_packed > 10
    ids = R.synth_tokens(19, 1, 7, kw["vocab_size"])
    la, ha = a.forward_with_cache_output(ids[None], [0])
    lb, hb = b.forward_with_cache_output(ids[None], [0])
    assert np.array_equal(la, lb) and np.array_equal(ha, hb)
    lc, hc = c.forward_with_cache_output(ids[None], [0])
    gaps = c.router_gaps()
    assert compare(lc, hc, [ref.kv(128).forward(ids, 0)], gaps, 7) == 1
    for m in (a, b, c):
        m.close()


def lat_checkpoint(ref, seed):
    """Named f32 tensors in the reference's checkpoint shapes (1-D norms) for a latent model."""
    rng = np.random.default_rng(seed)
    out = {}
    for name, r, c, kind in ref.tensors():
        if kind == R.T_NORM:
            out[name] = (1 + 0.1 * rng.normal(size=c)).astype(np.float32)
        else:
            out[name] = rng.normal(0, 0.05, (r, c)).astype(np.float32)
    return out


@pytest.mark.parametrize("kind", ["gguf-Q4KM", "gguf-Q80", "safetensors-BF16"])
def test_lat_checkpoint_into_context(tmp_path, kind):
    """An MLA + MoE checkpoint (model.rs:161-210 names, config resolved by
    aarh_lat_gguf_config) loaded by aarh_lat_load_gguf / aarh_lat_load_safetensors equals
    the oracle holding the values the oracle's reader decodes from the same file."""
    import refgguf as G
    kw = small_kw()
    fmts = {k: kw[k] for k in ("expert_format", "attn_format", "lm_head_format", "kv_format")}
    ref = R.LatModel(R.make_lat_config(**kw))
    vals = lat_checkpoint(ref, 31)
    vals["mtp.heads.0.trunk_norm.weight"] = np.ones(256, np.float32)  # not a latent-context tensor: ignored
    if kind.startswith("gguf"):
        path = str(tmp_path / "m.gguf")
        G.save_gguf(path, G.lat_model_config_json(**kw, fine_grained_factor=2), kind[5:], vals)
        cfg = A.LatConfig.from_gguf(path, **fmts)
        want = A.LatConfig(**kw)
        assert np.float32(cfg.norm_eps) == np.float32(want.norm_eps)
        assert cfg == A.LatConfig(**dict(kw, norm_eps=cfg.norm_eps))
        _, dec = G.load_gguf_tensors(path)
    else:
        path = str(tmp_path / "m.safetensors")
        G.save_safetensors(path, vals, "BF16")
        cfg = A.LatConfig(**kw)
        dec = G.safetensors_values(vals, "BF16")
    hip = A.HipLatModel(cfg, max_batch=3, max_rows=96)
    load = hip.load_gguf if kind.startswith("gguf") else hip.load_safetensors
    assert load(path) == len(hip.tensors()) == len(ref.tensors())
    for i, (name, *_r) in enumerate(ref.tensors()):
        ref.set(i, dec[name])
    B, P, K = 3, 20, 4
    ids = R.synth_tokens(32, 1, B * (P + K), kw["vocab_size"]).reshape(B, P + K)
    kvs = [ref.kv(128) for _ in range(B)]
    gl, gh = hip.forward_with_cache_output(ids[:, :P], [0] * B)
    checked = compare(gl, gh, [kvs[b].forward(ids[b, :P], 0) for b in range(B)], hip.router_gaps(), P)
    gl, gh = hip.forward_with_cache_output(ids[:, P:], [P] * B)
    checked += compare(gl, gh, [kvs[b].forward(ids[b, P:], P) for b in range(B)], hip.router_gaps(), K)
    assert checked >= 3
    if kind == "gguf-Q80":
        other = A.HipLatModel(A.LatConfig(**dict(kw, n_experts=16)), max_batch=1, max_rows=32)
        with pytest.raises(A.ConfigError, match="routed experts 8 does not match the context's 16"):
            other.load_gguf(path)
        other.close()
        short = {k: v for k, v in vals.items() if k != "blocks.1.ffn.experts.3.w_up.weight"}
        p2 = str(tmp_path / "short.gguf")
        G.save_gguf(p2, G.lat_model_config_json(**kw), "Q80", short)
        with pytest.raises(A.CheckpointError, match="experts.3.w_up"):
            hip.load_gguf(p2)
        p3 = str(tmp_path / "dense.gguf")
        G.save_gguf(p3, G.model_config_json(vocab_size=1024, hidden_dim=256, ffn_dim=512, n_layers=2, n_heads=4,
                                            n_kv_heads=4, max_seq_len=128), "Q80", vals)
        with pytest.raises(A.UnsupportedError, match="no moe"):
            hip.load_gguf(p3)
    hip.close()
    ref.close()


def test_lat_untied_head_checkpoint(tmp_path):
    """tie_embeddings false (LmHead::untied_with_qat, model.rs:239-248): the latent context
    holds lm_head.weight after final_norm and reads it from a GGUF checkpoint.  Logits equal
    the oracle's, and equal the final normed hidden state times the stored head (not the
    embedding); a tied context rejects the file."""
    import refgguf as G
    kw = small_kw()
    fmts = {k: kw[k] for k in ("expert_format", "attn_format", "lm_head_format", "kv_format")}
    ref = R.LatModel(R.make_lat_config(**kw, untied_lm_head=1))
    names = [t[0] for t in ref.tensors()]
    assert names[-2:] == ["final_norm.weight", "lm_head.weight"]
    vals = lat_checkpoint(ref, 37)
    path = str(tmp_path / "untied.gguf")
    G.save_gguf(path, G.lat_model_config_json(**kw, tie_embeddings=False), "Q80", vals)
    cfg = A.LatConfig.from_gguf(path, **fmts)
    assert cfg.tie_embeddings is False
    hip = A.HipLatModel(cfg, max_batch=2, max_rows=64)
    assert [t[0] for t in hip.tensors()] == names
    assert hip.load_gguf(path) == len(names)
    _, dec = G.load_gguf_tensors(path)
    for i, name in enumerate(names):
        ref.set(i, dec[name])
    B, P = 2, 24
    ids = R.synth_tokens(33, 1, B * P, kw["vocab_size"]).reshape(B, P)
    kvs = [ref.kv(128) for _ in range(B)]
    gl, gh = hip.forward_with_cache_output(ids, [0] * B)
    assert compare(gl, gh, [kvs[b].forward(ids[b], 0) for b in range(B)], hip.router_gaps(), P) >= 1
    head, emb = ref.get(len(names) - 1), ref.get(0)  # stored (bf16-rounded) values
    for b in range(B):
        via_head = gh[b].astype(np.float64) @ head.astype(np.float64).T
        via_emb = gh[b].astype(np.float64) @ emb.astype(np.float64).T
        assert rel_rows(gl[b], via_head).max() < TOL
        assert rel_rows(gl[b], via_emb).max() > 0.5
    tied = A.HipLatModel(A.LatConfig(**kw), max_batch=1, max_rows=32)
    with pytest.raises(A.ConfigError, match=r"tie_embeddings false does not match the context's LM head \(tied\)"):
        tied.load_gguf(path)
    tied.close()
    hip.close()
    ref.close()


def test_lat_untied_head_synthetic():
    """Random init of an untied latent model (the head is the last tensor id on both sides)
    against the oracle, bf16 and f32 heads."""
    for lmfmt in (1, 0):
        kw = small_kw(lm_head_format=lmfmt)
        ref = R.LatModel(R.make_lat_config(**kw, untied_lm_head=1))
        ref.init_synthetic(41, 0.05)
        hip = A.HipLatModel(A.LatConfig(**kw, tie_embeddings=False), max_batch=2, max_rows=64)
        hip.init_synthetic(41, 0.05)
        B, P = 2, 16
        ids = R.synth_tokens(43, 1, B * P, kw["vocab_size"]).reshape(B, P)
        kvs = [ref.kv(128) for _ in range(B)]
        gl, gh = hip.forward_with_cache_output(ids, [0] * B)
        assert compare(gl, gh, [kvs[b].forward(ids[b], 0) for b in range(B)], hip.router_gaps(), P) >= 1
        hip.close()
        ref.close()
