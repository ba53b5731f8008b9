"""aarh_accept_sample_static (no allocation: statically allocated per-GPU scratch)
against aarh_accept_sample on the same inputs, through the C ABI: two calls in a
row, the second smaller, sampled and greedy; sizes beyond the static scratch are
rejected."""
import numpy as np
import pytest
import torch

import aarambh_hip as A
import refcpu as R

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _inputs(B, K, V, seed):
    rng = np.random.default_rng(seed)
    tgt = rng.normal(0, 3, (B, K + 1, V)).astype(np.float32)
    drf = (tgt[:, :K] + rng.normal(0, 1, (B, K, V))).astype(np.float32)
    s = R.sampler(temperature=0.8)
    toks = np.zeros((B, K), np.uint32)
    for b in range(B):
        r = R.Rng(40_000 + b)
        for i in range(K):
            toks[b, i] = R.sample_probabilities(s, r, R.probabilities(s, drf[b, i]))
    t = lambda a, dt: torch.from_numpy(np.ascontiguousarray(a).astype(dt)).to(DEV)
    return t(tgt, np.float32), t(drf, np.float32), t(toks, np.int32), t(np.arange(B) + seed, np.int64)


@pytest.fixture(scope="module")
def ctx():
    m = A.HipModel(A.ModelConfig(vocab_size=128, hidden_dim=128, ffn_dim=128, n_layers=1, n_heads=1,
                                 n_kv_heads=1, max_seq_len=16), max_batch=1, max_rows=16)
    yield m
    m.close()


@pytest.mark.parametrize("sampler", [A.Sampler.top_k_top_p(0.8), A.Sampler.top_k_top_p(0.7, top_k=50, top_p=0.9),
                                     A.Sampler.greedy_sampler()])
def test_static_scratch_entry_equals_allocating_entry(ctx, sampler):
    for B, K, V, bonus, seed in ((32, 4, 32000, True, 1), (5, 2, 4096, False, 2)):
        tgt, drf, toks, seeds = _inputs(B, K, V, seed)
        want = ctx.accept_sample(tgt, drf, toks, sampler, bonus, seeds=seeds)
        got = ctx.accept_sample(tgt, drf, toks, sampler, bonus, seeds=seeds, no_alloc=True)
        for k in ("accept_len", "token", "flags", "draws", "status"):
            assert torch.equal(got[k], want[k]), (B, k, got[k], want[k])


def test_static_scratch_limits_are_rejected(ctx):
    tgt, drf, toks, seeds = _inputs(1025, 1, 128, 3)  # 1025 sequences > 1024
    with pytest.raises(A.ShapeError):
        ctx.accept_sample(tgt, drf, toks, A.Sampler.top_k_top_p(1.0), True, seeds=seeds, no_alloc=True)
    tgt, drf, toks, seeds = _inputs(600, 3, 128, 4)  # 600 x 7 rows > 4096
    with pytest.raises(A.ShapeError):
        ctx.accept_sample(tgt, drf, toks, A.Sampler.top_k_top_p(1.0), True, seeds=seeds, no_alloc=True)
    # the entry still works after a rejected call
    tgt, drf, toks, seeds = _inputs(4, 2, 256, 5)
    want = ctx.accept_sample(tgt, drf, toks, A.Sampler.top_k_top_p(1.0), True, seeds=seeds)
    got = ctx.accept_sample(tgt, drf, toks, A.Sampler.top_k_top_p(1.0), True, seeds=seeds, no_alloc=True)
    assert all(torch.equal(got[k], want[k]) for k in want)
