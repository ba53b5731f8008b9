"""Parity of the device verify forward (model.rs:529-587) and MTP head
(model.rs:783-817) against the oracle on identical random-init weights.
Bar: logits within 2e-3 relative (max|d|/max|ref| per row), hidden states likewise."""
import numpy as np
import pytest

import aarambh_hip as A
import refcpu as R
from gpu_util import make_pair, rel_rows

pytestmark = pytest.mark.gpu
TOL = 2e-3


def test_f32_model_prefill_and_verify():
    # C1 shape family (head_dim 32, ffn 704 not a multiple of 128) at reduced depth.
    kw = dict(vocab_size=1024, hidden_dim=256, ffn_dim=704, n_layers=2, n_heads=8, n_kv_heads=2, max_seq_len=96,
              num_future_tokens=2)
    ref, hip = make_pair(seed=1, **kw)
    ids = R.synth_tokens(1, 1, 24, 1024)
    kv = ref.kv(96)
    wl, wh = kv.forward(ids[:20], 0)
    gl, gh = hip.forward_with_cache_output(ids[None, :20], [0])
    assert rel_rows(gl[0], wl).max() < 1e-4 and rel_rows(gh[0], wh).max() < 1e-4
    wl2, _ = kv.forward(ids[20:], 20)
    gl2, _ = hip.forward_with_cache_output(ids[None, 20:], [20])
    assert rel_rows(gl2[0], wl2).max() < 1e-4
    assert hip.kv_len(0) == 24
    hip.close()


@pytest.mark.parametrize("wfmt,kvfmt,lmfmt", [(A.W_INT8_ROW, A.KV_F16, 1), (A.W_INT4_G128, A.KV_INT8, 1),
                                              (A.W_BF16, A.KV_F32, 0)])
def test_quantised_verify_matches_oracle(wfmt, kvfmt, lmfmt):
    kw = dict(vocab_size=2048, hidden_dim=512, ffn_dim=1024, n_layers=2, n_heads=4, n_kv_heads=2, max_seq_len=160,
              num_future_tokens=3, weight_format=wfmt, kv_format=kvfmt, lm_head_format=lmfmt)
    ref, hip = make_pair(seed=2, max_batch=3, max_rows=128, **kw)
    B, P, K = 3, 37, 4
    prompts = R.synth_tokens(2, 7, B * (P + K), 2048).reshape(B, P + K)
    kvs = [ref.kv(160) for _ in range(B)]
    # batched prefill of different lengths via per-sequence offsets: run P tokens for all
    gl, gh = hip.forward_with_cache_output(prompts[:, :P], [0, 0, 0])
    for b in range(B):
        wl, wh = kvs[b].forward(prompts[b, :P], 0)
        assert rel_rows(gl[b], wl).max() < TOL, (b, rel_rows(gl[b], wl).max())
        assert rel_rows(gh[b], wh).max() < TOL
    # verify K tokens at offset P (the hot call)
    gl, gh = hip.forward_with_cache_output(prompts[:, P:], [P, P, P])
    for b in range(B):
        wl, wh = kvs[b].forward(prompts[b, P:], P)
        assert rel_rows(gl[b], wl).max() < TOL
    # rollback by index and replay a shorter suffix (mtp_speculative.rs:284-313)
    gl, _ = hip.forward_with_cache_output(prompts[:, P:P + 2], [P, P, P])
    for b in range(B):
        kvs[b].truncate(P)
        wl, _ = kvs[b].forward(prompts[b, P:P + 2], P)
        assert rel_rows(gl[b], wl).max() < TOL
    assert hip.kv_len(1) == P + 2
    hip.close()


def test_int4_preloaded_codes_equal_device_quantisation():
    """aarh_load_tensor_int4 with the oracle's codes (int4.rs layout) and
    aarh_load_tensor_f32 (device quantiser) must give bit-identical logits."""
    kw = dict(vocab_size=1024, hidden_dim=256, ffn_dim=512, n_layers=1, n_heads=2, n_kv_heads=1, max_seq_len=64,
              weight_format=A.W_INT4_G128, lm_head_format=1, kv_format=A.KV_INT8)
    ref, hip = make_pair(seed=3, **kw)
    hip2 = A.HipModel(A.ModelConfig(**kw), max_batch=1, max_rows=64)
    for i, (name, r, c, kind) in enumerate(ref.tensors()):
        raw = R.synth_fill(3, i, r * c, 0.02) if kind != R.T_NORM else np.ones(r * c, np.float32)
        if kind == R.T_LINEAR:
            p, sh, zh = R.quantise_i4_f16(raw, 128)
            hip2.load_int4(i, p, sh, zh, r, c, 128)
        else:
            hip2.load_f32(i, raw)
    ids = R.synth_tokens(3, 1, 9, 1024)
    a, _ = hip.forward_with_cache_output(ids[None], [0])
    b, _ = hip2.forward_with_cache_output(ids[None], [0])
    assert np.array_equal(a, b)
    hip.close()
    hip2.close()


def test_int8_preloaded_codes_equal_device_quantisation():
    kw = dict(vocab_size=1024, hidden_dim=256, ffn_dim=512, n_layers=1, n_heads=2, n_kv_heads=1, max_seq_len=64,
              weight_format=A.W_INT8_ROW, lm_head_format=1, kv_format=A.KV_F16)
    ref, hip = make_pair(seed=4, **kw)
    hip2 = A.HipModel(A.ModelConfig(**kw), max_batch=1, max_rows=64)
    for i, (name, r, c, kind) in enumerate(ref.tensors()):
        raw = R.synth_fill(4, i, r * c, 0.02) if kind != R.T_NORM else np.ones(r * c, np.float32)
        if kind == R.T_LINEAR:
            q, sc = R.quantise_i8_rows(raw.reshape(r, c))
            hip2.load_int8(i, q, sc, r, c)
        else:
            hip2.load_f32(i, raw)
    ids = R.synth_tokens(4, 1, 9, 1024)
    a, _ = hip.forward_with_cache_output(ids[None], [0])
    b, _ = hip2.forward_with_cache_output(ids[None], [0])
    assert np.array_equal(a, b)
    hip.close()
    hip2.close()


def test_mtp_heads_match_oracle():
    kw = dict(vocab_size=2048, hidden_dim=512, ffn_dim=1024, n_layers=1, n_heads=4, n_kv_heads=2, max_seq_len=64,
              num_future_tokens=4, weight_format=A.W_INT4_G128, lm_head_format=1, kv_format=A.KV_INT8)
    ref, hip = make_pair(seed=5, max_batch=2, **kw)
    anchors = np.random.default_rng(5).normal(0, 1, (2, 512)).astype(np.float32)
    for head in range(3):
        ids = R.synth_tokens(5, head, 2 * (head + 1), 2048).reshape(2, head + 1)
        got = hip.forward_mtp_head(head, anchors, ids)
        for b in range(2):
            want = ref.mtp_head(head, anchors[b], ids[b])
            assert rel_rows(got[b][None], want[None]).max() < TOL
    with pytest.raises(A.ConfigError):
        hip.forward_mtp_head(3, anchors, np.zeros((2, 4), np.uint32))
    hip.close()


def test_shape_errors_are_reported():
    kw = dict(vocab_size=1024, hidden_dim=256, ffn_dim=512, n_layers=1, n_heads=2, n_kv_heads=1, max_seq_len=32)
    hip = A.HipModel(A.ModelConfig(**kw), max_batch=1, max_rows=32)
    hip.init_synthetic(0)
    with pytest.raises(A.ShapeError):  # offset beyond the cached length
        hip.forward_with_cache_output(np.zeros((1, 2), np.uint32), [5])
    with pytest.raises(A.ShapeError):  # context overflow (check_token_ids, model.rs:886-907)
        hip.forward_with_cache_output(np.zeros((1, 33), np.uint32), [0])
    with pytest.raises(A.ShapeError):
        hip.forward_with_cache_output(np.full((1, 2), 5000, np.uint32), [0])
    with pytest.raises(A.ShapeError):
        hip.restore(3)  # cannot grow by rollback
    hip.close()


@pytest.mark.parametrize("kvfmt", [A.KV_INT8, A.KV_F16])
def test_forwards_above_128_rows(kvfmt):
    """max_rows up to 512: a 32-sequence x 5-row verify (k = 4, 160 rows) at ragged
    offsets, and a 384-token single-sequence prefill, at hd 128 against the oracle."""
    kw = dict(vocab_size=2048, hidden_dim=512, ffn_dim=1024, n_layers=2, n_heads=4, n_kv_heads=2, max_seq_len=512,
              weight_format=A.W_INT4_G128, kv_format=kvfmt, lm_head_format=1)
    ref, hip = make_pair(seed=12, max_batch=32, max_rows=512, **kw)
    B, P, K = 32, 20, 5
    rng = np.random.default_rng(12)
    toks = R.synth_tokens(12, 1, B * (P + K), 2048).reshape(B, P + K)
    plen = rng.integers(6, P + 1, B)
    # prefill every sequence to its own length (ragged), 32 x 20 = 640 rows in two calls
    for half in (slice(0, 16), slice(16, 32)):
        hip.forward_with_cache_output(toks[half, :P], [0] * 16, slots=np.arange(32)[half], want_logits=False,
                                      want_hidden=False)
    ids = np.stack([toks[b, plen[b]:plen[b] + K] for b in range(B)])
    gl, gh = hip.forward_with_cache_output(ids, plen)  # rewinds each slot to its offset
    worst = 0.0
    for b in range(B):
        kv = ref.kv(512)  # same call structure: prefill P, rewind to plen, verify K rows
        kv.forward(toks[b, :P], 0)
        kv.truncate(int(plen[b]))
        wl, wh = kv.forward(ids[b], int(plen[b]))
        worst = max(worst, rel_rows(gl[b], wl).max(), rel_rows(gh[b], wh).max())
    assert worst < TOL, worst
    long = R.synth_tokens(12, 2, 384, 2048)
    gl, _ = hip.forward_with_cache_output(long[None], [0])
    wl, _ = ref.kv(512).forward(long, 0, nthreads=16)
    assert rel_rows(gl[0], wl).max() < TOL
    hip.close()


def test_weight_tensors_of_2gib_are_rejected():
    # a bf16 LM head of 131072 x 8192 is 2 GiB: beyond the 32-bit offsets of the
    # projection kernels' buffer resources, so creation fails instead of wrapping
    kw = dict(vocab_size=131072, hidden_dim=8192, ffn_dim=128, n_layers=1, n_heads=64, n_kv_heads=8, max_seq_len=32,
              weight_format=A.W_INT4_G128, lm_head_format=1)
    with pytest.raises(A.UnsupportedError, match="2 GiB"):
        A.HipModel(A.ModelConfig(**kw), max_batch=1, max_rows=8)
    # 128 rows less fits
    hip = A.HipModel(A.ModelConfig(**dict(kw, vocab_size=130944)), max_batch=1, max_rows=8)
    hip.close()


@pytest.mark.parametrize("kvfmt", [A.KV_INT8, A.KV_F16])
def test_long_context_verify_over_synthetic_cache(kvfmt):
    """Verify K=4 rows over 700- and 300-token caches (many attention chunks,
    ragged offsets); the cache contents come from the shared synthetic formula."""
    kw = dict(vocab_size=2048, hidden_dim=512, ffn_dim=1024, n_layers=2, n_heads=8, n_kv_heads=2, max_seq_len=800,
              weight_format=A.W_INT4_G128, kv_format=kvfmt, lm_head_format=1)
    ref, hip = make_pair(seed=8, max_batch=2, max_rows=64, **kw)
    lens = [700, 300]
    kvs = []
    for b, L in enumerate(lens):
        hip.kv_fill_synthetic(b, L, seed=11 + b)
        kv = ref.kv(800)
        kv.fill_synthetic(11 + b, L)
        kvs.append(kv)
    ids = R.synth_tokens(8, 2, 8, 2048).reshape(2, 4)
    gl, gh = hip.forward_with_cache_output(ids, lens)
    for b in range(2):
        wl, wh = kvs[b].forward(ids[b], lens[b])
        assert rel_rows(gl[b], wl).max() < TOL, (b, rel_rows(gl[b], wl).max())
        assert rel_rows(gh[b], wh).max() < TOL
    hip.close()


@pytest.mark.parametrize("ffn", [5632, 11008])
@pytest.mark.parametrize("wfmt", [A.W_INT4_G128, A.W_INT8_ROW])
def test_wide_ffn_register_fragment_paths(ffn, wfmt):
    """Down projections with K = 5632 / 11008 fed 6, 4 and 1 rows: the GEMV
    variants holding 8 and 12 groups of activation fragments per wave in
    registers (and the L2-fragment variant at 6 rows with K = 11008)."""
    kw = dict(vocab_size=1024, hidden_dim=256, ffn_dim=ffn, n_layers=1, n_heads=2, n_kv_heads=1, max_seq_len=64,
              weight_format=wfmt, kv_format=A.KV_F16, lm_head_format=1)
    ref, hip = make_pair(seed=9, max_batch=1, max_rows=16, **kw)
    ids = R.synth_tokens(9, 0, 11, 1024)
    kv = ref.kv(64)
    pos = 0
    for n in (6, 4, 1):
        wl, wh = kv.forward(ids[pos:pos + n], pos)
        gl, gh = hip.forward_with_cache_output(ids[None, pos:pos + n], [pos])
        assert rel_rows(gl[0], wl).max() < TOL, (n, rel_rows(gl[0], wl).max())
        assert rel_rows(gh[0], wh).max() < TOL, (n, rel_rows(gh[0], wh).max())
        pos += n
    hip.close()


@pytest.mark.parametrize("nseq,S", [(1, 17), (2, 20), (4, 25), (8, 16)])
@pytest.mark.parametrize("wfmt,lmfmt", [(A.W_INT4_G128, 1), (A.W_INT8_ROW, 1), (A.W_BF16, 1)])
def test_many_row_gemm_variants(wfmt, lmfmt, nseq, S):
    """M = nseq * S rows in (16, 128]: the MFMA GEMM with 2, 4 and 8 row chunks per
    block, split-K over K = 1024 / 2816 (ragged last split), every epilogue (QKV
    RoPE, residual, SwiGLU, LM-head store + final hidden), plain fp16 / bf16
    activation fragments.  Logits and hidden within 2e-3 of the f32 oracle."""
    kw = dict(vocab_size=4096, hidden_dim=1024, ffn_dim=2816, n_layers=2, n_heads=8, n_kv_heads=2, max_seq_len=64,
              weight_format=wfmt, kv_format=A.KV_F16, lm_head_format=lmfmt)
    ref, hip = make_pair(seed=12, max_batch=nseq, max_rows=128, **kw)
    ids = R.synth_tokens(12, nseq, nseq * S, 4096).reshape(nseq, S)
    gl, gh = hip.forward_with_cache_output(ids, [0] * nseq)
    for b in range(nseq):
        wl, wh = ref.kv(64).forward(ids[b], 0)
        assert rel_rows(gl[b], wl).max() < TOL, (b, rel_rows(gl[b], wl).max())
        assert rel_rows(gh[b], wh).max() < TOL, (b, rel_rows(gh[b], wh).max())
    # a second, shorter batched call on the same caches (counters re-armed, partials reused)
    ids2 = R.synth_tokens(12, 100 + nseq, nseq * 3, 4096).reshape(nseq, 3)
    gl2, _ = hip.forward_with_cache_output(ids2, [S] * nseq)
    kv0 = ref.kv(64)
    kv0.forward(ids[0], 0)
    wl2, _ = kv0.forward(ids2[0], S)
    assert rel_rows(gl2[0], wl2).max() < TOL
    hip.close()


@pytest.mark.parametrize("wfmt,nseq,S", [(A.W_INT4_G128, 32, 1), (A.W_INT4_G128, 8, 4), (A.W_INT4_G128, 5, 4),
                                         (A.W_INT4_G128, 12, 4),
                                         (A.W_INT4_G128, 32, 4), (A.W_INT8_ROW, 32, 4), (A.W_INT8_ROW, 10, 4),
                                         (A.W_BF16, 32, 4)])
def test_c4_width_gemm_plans(wfmt, nseq, S):
    """C4 projection widths (d_model 4096, ffn 11008, 32 query / 8 kv heads) at M = 32,
    32, 20, 48, 128 (INT4 g128), 128, 40 (INT8) and 128 (BF16) rows: the tuned INT4 GEMM
    plans (2 x 4 and 1 x 8 wave grids, the K-split mode of gate/up and down at 32 rows
    and below, 20 rows leaving the second 16-row chunk partial) and the rule's plans for
    the other formats (32- and 64-row blocks, 1 to 4 weight tiles per wave, 1 to 8
    k-splits) through a one-layer forward.  Logits and hidden within 2e-3 of the f32
    oracle."""
    kw = dict(vocab_size=2048, hidden_dim=4096, ffn_dim=11008, n_layers=1, n_heads=32, n_kv_heads=8,
              max_seq_len=64, weight_format=wfmt, kv_format=A.KV_INT8, lm_head_format=1)
    print("c4-width gemm", wfmt, nseq, S, flush=True)
    ref, hip = make_pair(seed=21, max_batch=nseq, max_rows=128, **kw)
    ids = R.synth_tokens(21, nseq, nseq * S, 2048).reshape(nseq, S)
    gl, gh = hip.forward_with_cache_output(ids, [0] * nseq)
    for b in range(0, nseq, max(1, nseq // 4)):
        wl, wh = ref.kv(64).forward(ids[b], 0, nthreads=16)
        assert rel_rows(gl[b], wl).max() < TOL, (b, rel_rows(gl[b], wl).max())
        assert rel_rows(gh[b], wh).max() < TOL, (b, rel_rows(gh[b], wh).max())
    hip.close()


def test_graph_replay_is_bit_identical_to_direct_launches():
    """Repeated verify shapes replay a captured HIP graph (first sighting direct, second
    captured, later replayed); every replay, with other-shape eager forwards and
    rollbacks in between, gives the bits of the directly launched forward."""
    kw = dict(vocab_size=2048, hidden_dim=512, ffn_dim=1024, n_layers=2, n_heads=4, n_kv_heads=2, max_seq_len=600,
              weight_format=A.W_INT4_G128, lm_head_format=1, kv_format=A.KV_INT8)
    ref, hip = make_pair(seed=9, max_batch=3, max_rows=128, **kw)
    hip.set_graphs(False)
    for b in range(3):
        hip.kv_fill_synthetic(b, 300, seed=40 + b)
    ids = R.synth_tokens(9, 4, 3 * 4, 2048).reshape(3, 4)
    other = R.synth_tokens(9, 5, 3 * 2, 2048).reshape(3, 2)
    want, wh = hip.forward_with_cache_output(ids, [300, 300, 300])
    want_o, _ = hip.forward_with_cache_output(other, [300, 300, 300])
    hip.set_graphs(True)
    for it in range(5):
        got, gh = hip.forward_with_cache_output(ids, [300, 300, 300])
        assert np.array_equal(got, want) and np.array_equal(gh, wh), it
        got_o, _ = hip.forward_with_cache_output(other, [300, 300, 300])
        assert np.array_equal(got_o, want_o), it
        for b in range(3):
            hip.restore(300, slot=b)
    hip.close()


@pytest.mark.parametrize("kvfmt", [A.KV_INT8, A.KV_F16])
def test_hd128_long_context_chunk_merge(kvfmt):
    """head_dim 128 (the MFMA decode attention) over caches of 600, 3000, 5400 and
    9000 tokens with one KV head: 3, 12, 22 and 36 chunks of 256 tokens, so the chunk
    merge runs with one pass and with the running-max rescale across passes of 20
    chunks.  Logits and hidden within 2e-3 of the oracle."""
    kw = dict(vocab_size=2048, hidden_dim=512, ffn_dim=1024, n_layers=1, n_heads=4, n_kv_heads=1,
              max_seq_len=9100, weight_format=A.W_INT4_G128, kv_format=kvfmt, lm_head_format=1)
    ref, hip = make_pair(seed=15, max_batch=4, max_rows=64, **kw)
    lens = [600, 3000, 5400, 9000]
    for b, L in enumerate(lens):
        hip.kv_fill_synthetic(b, L, seed=60 + b)
    ids = R.synth_tokens(15, 2, 16, 2048).reshape(4, 4)
    gl, gh = hip.forward_with_cache_output(ids, lens)
    for b, L in enumerate(lens):
        kv = ref.kv(9100)
        kv.fill_synthetic(60 + b, L)
        wl, wh = kv.forward(ids[b], L, nthreads=16)
        assert rel_rows(gl[b], wl).max() < TOL, (L, rel_rows(gl[b], wl).max())
        assert rel_rows(gh[b], wh).max() < TOL, (L, rel_rows(gh[b], wh).max())
    # each length alone (its own chunking: up to 36 chunks for one sequence)
    for b, L in enumerate(lens):
        hip.restore(L, slot=b)
        gl1, _ = hip.forward_with_cache_output(ids[b:b + 1], [L], slots=[b])
        kv = ref.kv(9100)
        kv.fill_synthetic(60 + b, L)
        wl, _ = kv.forward(ids[b], L, nthreads=16)
        assert rel_rows(gl1[0], wl).max() < TOL, (L, "single", rel_rows(gl1[0], wl).max())
    hip.close()


def test_hd128_int8_tail_blocks_and_cache_write_back():
    """The INT8 decode attention writes the new positions into its staged copy of each
    block that holds them and stores the block back whole.  New rows ending a block,
    straddling two blocks and starting one (offsets 28, 29, 31, 1021), then a 64-row
    prompt chunk over three blocks (rows spread over the waves, sixteen query tiles
    storing the same blocks), and a second forward after each that reads the first
    one's rows back from the cache: logits and hidden within 2e-3 of the oracle."""
    kw = dict(vocab_size=2048, hidden_dim=512, ffn_dim=1024, n_layers=2, n_heads=4, n_kv_heads=1,
              max_seq_len=1200, weight_format=A.W_INT4_G128, kv_format=A.KV_INT8, lm_head_format=1)
    ref, hip = make_pair(seed=21, max_batch=4, max_rows=64, **kw)
    lens = [28, 29, 31, 1021]
    kvs = []
    for b, L in enumerate(lens):
        hip.kv_fill_synthetic(b, L, seed=80 + b)
        kv = ref.kv(1200)
        kv.fill_synthetic(80 + b, L)
        kvs.append(kv)
    for step in range(2):
        ids = R.synth_tokens(21, 3 + step, 16, 2048).reshape(4, 4)
        pos = [L + 4 * step for L in lens]
        gl, gh = hip.forward_with_cache_output(ids, pos)
        for b in range(4):
            wl, wh = kvs[b].forward(ids[b], pos[b], nthreads=16)
            assert rel_rows(gl[b], wl).max() < TOL, (step, pos[b], rel_rows(gl[b], wl).max())
            assert rel_rows(gh[b], wh).max() < TOL, (step, pos[b], rel_rows(gh[b], wh).max())
    # a 64-row prompt chunk at offset 20 (positions 20 .. 83: three blocks), then 4 rows at 84
    hip.kv_fill_synthetic(0, 20, seed=90)
    kv = ref.kv(1200)
    kv.fill_synthetic(90, 20)
    for S, L in ((64, 20), (4, 84)):
        ids = R.synth_tokens(22, S, S, 2048).reshape(1, S)
        gl, gh = hip.forward_with_cache_output(ids, [L], slots=[0])
        wl, wh = kv.forward(ids[0], L, nthreads=16)
        assert rel_rows(gl[0], wl).max() < TOL, (S, L, rel_rows(gl[0], wl).max())
        assert rel_rows(gh[0], wh).max() < TOL, (S, L, rel_rows(gh[0], wh).max())
    hip.close()


@pytest.mark.parametrize("group", [128, 256, 512])
def test_packed_int4_tensor_loads(group):
    """PackedInt4Tensor as the quant crate holds it (f32 scales / zeros, group_size):
    at group 128 the device holds exactly what the device quantiser makes of the same
    f32 weights (logits bit-identical); at every group size the logits equal the
    oracle's forward on dequantise_packed_i4_to_vec's values with fp16 scales (the
    device's stored function) within 2e-3, and on the f32-scale values within 2e-3."""
    # fp16 KV and an f32 LM head: this small model's INT8 KV / bf16 head roundings move its
    # logits by up to 1.6e-3 under a 3e-6 input perturbation, which is not what this tests
    kw = dict(vocab_size=1024, hidden_dim=256, ffn_dim=512, n_layers=2, n_heads=2, n_kv_heads=1, max_seq_len=64,
              weight_format=A.W_INT4_G128, lm_head_format=0, kv_format=A.KV_F16)
    fkw = dict(kw, weight_format=A.W_F32)
    ref_dev = R.Model(R.make_config(**fkw))   # values the device stores
    ref_f32 = R.Model(R.make_config(**fkw))   # values dequantise_packed_i4_to_vec gives
    hip = A.HipModel(A.ModelConfig(**kw), max_batch=1, max_rows=64)
    hq = A.HipModel(A.ModelConfig(**kw), max_batch=1, max_rows=64) if group == 128 else None
    for i, (name, r, c, kind) in enumerate(hip.tensors()):
        raw = R.synth_fill(17, i, r * c, 0.02) if kind != R.T_NORM else np.ones(r * c, np.float32)
        if kind == R.T_LINEAR:
            data, sc, zz = R.quantise_i4(raw, group)
            t = A.PackedInt4Tensor((r, c), group, data, sc, zz)
            hip.load_packed_i4(i, t)
            sh, zh = A.packed_i4_params(t)
            codes = np.zeros(r * c, np.float32)
            codes[0::2], codes[1::2] = data & 15, data >> 4
            gi = np.repeat(np.arange(c // 128), 128)
            s, z = sh.view(np.float16).astype(np.float32), zh.view(np.float16).astype(np.float32)
            ref_dev.set(i, (codes.reshape(r, c) - z[:, gi]) * s[:, gi])
            ref_f32.set(i, R.dequantise_i4(data, r * c, group, sc, zz))
            if hq:
                hq.load_f32(i, raw)
        else:
            for m in (hip, hq):
                if m:
                    m.load_f32(i, raw)
            ref_dev.set(i, raw)
            ref_f32.set(i, raw)
    ids = R.synth_tokens(17, 1, 9, 1024)
    got, _ = hip.forward_with_cache_output(ids[None], [0])
    if hq:
        same, _ = hq.forward_with_cache_output(ids[None], [0])
        assert np.array_equal(got, same)
        hq.close()
    for ref in (ref_dev, ref_f32):
        want, _ = ref.kv(64).forward(ids, 0)
        assert rel_rows(got[0], want).max() < 2e-3
    hip.close()
