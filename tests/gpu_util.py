"""Shared helpers for the GPU parity tests: build matching oracle / HIP models."""
import numpy as np

import aarambh_hip as A
import refcpu as R


def rel_rows(got, want):
    """Norm-wise relative error per row: max|d| / max|ref| (the logit tolerance rule)."""
    got = np.asarray(got, np.float64).reshape(-1, got.shape[-1])
    want = np.asarray(want, np.float64).reshape(-1, want.shape[-1])
    return np.max(np.abs(got - want), axis=1) / np.maximum(np.max(np.abs(want), axis=1), 1e-30)


def make_pair(seed=0, std=0.02, max_batch=1, max_rows=64, **kw):
    """Identical random-init weights in the oracle and on the device (f32 host values,
    quantised by each side's own codec)."""
    rc = R.make_config(**kw)
    ref = R.Model(rc)
    mc = A.ModelConfig(**kw)
    hip = A.HipModel(mc, max_batch=max_batch, max_rows=max_rows)
    for i, (name, r, c, kind) in enumerate(ref.tensors()):
        raw = R.synth_fill(seed, i, r * c, std) if kind != R.T_NORM else np.ones(r * c, np.float32)
        ref.set(i, raw)
        hip.load_f32(i, raw)
    return ref, hip
