"""Writes the tiny checkpoint fixtures of the weight-ingestion tests (run from anywhere):

  weights_tiny_q4km.gguf / weights_tiny_q80.gguf   GGUF v1 files in the layout of
      save_gguf (aarambh-studio weights/src/gguf.rs:47-72) covering every encoding
      rule of encode_tensor (gguf.rs:127-141): 1-D and "_conv." tensors F32,
      ".dsa.index_" tensors Q8_0, other 2-D tensors Q4_K_M or Q8_0; ragged final
      Q4_K_M blocks; constant, sub-f16-normal and f16-overflowing block ranges.
  weights_tiny_{f32,f16,bf16}.safetensors           the same tensors as safetensors.
  weights_tiny_expected.npz                          f32 values a reader must return
      for each (file, tensor), as the oracle decodes them (key "<file>|<tensor>").

The files are written by the oracle's encoder (oracle/refgguf.py), which is pinned by
tests/test_weights.py against the reference's own known-answer tests and closed forms.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "..", "..", "oracle"))
import refgguf as G  # noqa: E402


def fixture_tensors():
    rng = np.random.default_rng(20261202)
    t = {
        "embedding.weight": rng.normal(0, 0.05, (24, 16)).astype(np.float32),
        "blocks.0.norm1.weight": (1 + 0.1 * rng.normal(size=16)).astype(np.float32),
        "blocks.0.attn.wq.weight": rng.normal(0, 0.2, (17, 33)).astype(np.float32),  # 561 values, ragged block
        "blocks.0.mixer_conv.weight": rng.normal(0, 0.3, (4, 6)).astype(np.float32),  # "_conv." stays F32
        "blocks.0.attn.dsa.index_q.weight": rng.normal(0, 0.4, (5, 12)).astype(np.float32),  # DSA -> Q8_0
        "edge.constant": np.full((2, 256), -0.75, np.float32),                     # range 0 -> scale 1.0
        "edge.subnormal_scale": (1e-6 * rng.random((1, 256))).astype(np.float32),  # f16-subnormal scale
        "edge.overflow": np.linspace(-7e5, 7e5, 256, dtype=np.float32).reshape(1, 256),  # f16 inf scale
        "edge.wide": np.concatenate([rng.normal(0, 1, 300), [70000.0, -70000.0, 1e-9, -0.0]]).astype(
            np.float32).reshape(8, 38),
    }
    return t


def main():
    tensors = fixture_tensors()
    cfg = G.model_config_json(24, 16, 32, 1, 2, 1, 64)
    expected = {}
    for fmt, fname in (("Q4KM", "weights_tiny_q4km.gguf"), ("Q80", "weights_tiny_q80.gguf")):
        path = os.path.join(HERE, fname)
        G.save_gguf(path, cfg, fmt, tensors)
        _, dec = G.load_gguf_tensors(path)
        for k, v in dec.items():
            expected[f"{fname}|{k}"] = v
    for dt in ("F32", "F16", "BF16"):
        fname = f"weights_tiny_{dt.lower()}.safetensors"
        G.save_safetensors(os.path.join(HERE, fname), tensors, dt, metadata={"format": "pt"})
        for k, v in G.safetensors_values(tensors, dt).items():
            expected[f"{fname}|{k}"] = v
    np.savez_compressed(os.path.join(HERE, "weights_tiny_expected.npz"), **expected)


if __name__ == "__main__":
    with np.errstate(all="ignore"):  # the edge tensors overflow f16 on purpose
        main()
