"""The latent checkpoint config reader (aarh_lat_gguf_config, host code, no GPU): MlaConfig::resolve
(core/src/config.rs:558-612), MoeConfig fine-grained experts and validate (:133-211), the attention
schedule (:656-708), RopeScalingConfig::validate (:52-96), dsa_config (model.rs:316-337) and serde's
field defaults, on GGUF files written by the oracle's encoder.  Pinned against the reference's own
tests (config.rs:1110-1135) and, for each validation rule, the reference's message; configs a
latent context cannot hold (MLA or MoE not in every layer) are UNSUPPORTED; tie_embeddings false
gives an untied head."""
import copy

import numpy as np
import pytest

import aarambh_hip as A
import refgguf as G

SHAPE = dict(vocab_size=256, hidden_dim=128, n_layers=2, n_heads=2, max_seq_len=64, latent_dim=64, rope_dim=16,
             nope_dim=48, v_dim=48, n_experts=4, top_k=2, expert_dim=128, n_shared=1)


def write(tmp_path, cfg, name="m.gguf"):
    p = str(tmp_path / name)
    G.save_gguf(p, cfg, "Q80", {"embedding.weight": np.zeros((4, 4), np.float32)})
    return p


def read(tmp_path, cfg):
    return A.LatConfig.from_gguf(write(tmp_path, cfg))


def base(**kw):
    return G.lat_model_config_json(**dict(SHAPE, **kw))


def test_reference_mla_resolution_kat(tmp_path):  # config.rs:1110-1123
    cfg = base()
    cfg["attention_schedule"]["mla"] = {"latent_dim": 64, "rope_head_dim": 16}  # nope, v, heads derived
    got = read(tmp_path, cfg)
    assert (got.n_heads, got.nope_dim, got.v_dim, got.latent_dim, got.rope_dim) == (2, 48, 48, 64, 16)
    assert got.latent_dim + got.rope_dim == 80  # cache_width


def test_reference_odd_rope_dim_rejected(tmp_path):  # config.rs:1125-1135
    cfg = base()
    cfg["attention_schedule"]["mla"]["rope_head_dim"] = 15
    with pytest.raises(A.ConfigError, match="rope_head_dim"):
        read(tmp_path, cfg)


def test_nope_floor_and_serde_defaults(tmp_path):
    cfg = base(hidden_dim=64, n_heads=4)  # host head_dim 16 - rope 16 = 0 -> floor 8 (config.rs:567-569)
    cfg["attention_schedule"]["mla"] = {"rope_head_dim": 16}
    del cfg["moe"]["top_k"]
    got = read(tmp_path, cfg)
    assert (got.nope_dim, got.v_dim, got.latent_dim, got.n_heads, got.top_k) == (8, 8, 512, 4, 2)
    cfg["attention_schedule"]["mla"] = {}
    assert read(tmp_path, cfg).rope_dim == 16  # MlaConfig::default


def test_bench_shape_and_fine_grained_subdivision(tmp_path):
    c5 = dict(vocab_size=32000, hidden_dim=2048, n_layers=24, n_heads=16, max_seq_len=4096, latent_dim=512,
              rope_dim=64, nope_dim=128, v_dim=128, n_experts=64, top_k=6, expert_dim=1408, n_shared=2)
    got = read(tmp_path, G.lat_model_config_json(**c5))
    for k, v in c5.items():
        assert getattr(got, k) == v, k
    # 16 coarse experts of width 5632, each split 4 ways: the same 64 fine experts of 1408
    cfg = G.lat_model_config_json(**c5, fine_grained_factor=4)
    assert cfg["moe"]["num_experts"] == 16 and cfg["moe"]["expert_ffn_dim"] == 5632
    got = read(tmp_path, cfg)
    assert (got.n_experts, got.expert_dim) == (64, 1408)
    # MLA heads differ from the transformer's
    got = read(tmp_path, G.lat_model_config_json(**dict(c5, n_heads=16), mla_heads=8))
    assert got.n_heads == 8


def test_tie_embeddings_selects_the_head(tmp_path):
    # LmHead::new (model.rs:239-248): tied reads the embedding, untied its own lm_head.weight
    assert read(tmp_path, base()).tie_embeddings is True
    assert read(tmp_path, base(tie_embeddings=False)).tie_embeddings is False


def edit(path, value):
    cfg = base()
    node = cfg
    for k in path[:-1]:
        node = node[k]
    if value is KeyError:
        del node[path[-1]]
    else:
        node[path[-1]] = value
    return cfg


@pytest.mark.parametrize("path,value,msg", [
    (("moe", "num_experts"), 1, "moe.num_experts must be at least 2"),
    (("moe", "fine_grained_factor"), 0, "moe.fine_grained_factor must be non-zero"),
    (("moe", "expert_ffn_dim"), 130, None),  # not divisible by fine_grained_factor 4, set below
    (("moe", "top_k"), 0, "moe.top_k must be in 1..=4 for num_experts=4 and fine_grained_factor=1"),
    (("moe", "top_k"), 5, "moe.top_k must be in 1..=4 for num_experts=4 and fine_grained_factor=1"),
    (("moe", "aux_loss_weight"), -0.5, "moe.aux_loss_weight must be finite and non-negative"),
    (("moe", "every_n_layers"), 0, "moe.every_n_layers must be non-zero"),
    (("moe", "every_n_layers"), 3, "moe.every_n_layers does not select any model layer"),
    (("attention_schedule", "full_attention_every_n"), 0, "attention_schedule.full_attention_every_n must be non-zero"),
    (("attention_schedule", "mla_layers"), [], "attention_schedule must select at least one Gated DeltaNet or LatentMLA layer"),
    (("attention_schedule", "mla"), KeyError, "attention_schedule.mla must be set when mla_layers is non-empty"),
    (("attention_schedule", "gated_deltanet", "chunk_size"), 48, "gated_deltanet.chunk_size must be a power of two in 16..=256"),
    (("attention_schedule", "gated_deltanet", "conv_kernel_size"), 1, "gated_deltanet.conv_kernel_size must be at least 2"),
    (("attention_schedule", "mla", "latent_dim"), 0, "mla.latent_dim must be non-zero"),
    (("n_heads",), 3, "hidden_dim must be divisible by n_heads"),
    (("rope_scaling",), dict(method="linear", factor=2.0, original_max_seq_len=128),
     "max_seq_len 64 must be >= rope_scaling.original_max_seq_len 128"),
    (("dsa_config",), {"block_size": 24}, "dsa.block_size must be a power of two in 16..=256"),
    (("dsa_config",), {}, "dsa_config does not select any sparse attention layer"),
])
def test_reference_validation_messages(tmp_path, path, value, msg):
    cfg = edit(path, value)
    if msg is None:
        cfg["moe"]["fine_grained_factor"] = 4
        msg = "moe.expert_ffn_dim 130 must be non-zero and divisible by fine_grained_factor 4"
    with pytest.raises(A.ConfigError) as e:
        read(tmp_path, cfg)
    assert str(e.value) == msg


@pytest.mark.parametrize("path,value,match", [
    (("moe", "every_n_layers"), 2, "every_n_layers 2 leaves dense FFN layers"),
    (("attention_schedule", "mla_layers"), [1], "mla_layers must list all 2 layers"),
    (("moe",), KeyError, "has no moe"),
    (("attention_schedule",), KeyError, "has no attention_schedule"),
])
def test_layouts_the_latent_context_cannot_hold(tmp_path, path, value, match):
    with pytest.raises(A.UnsupportedError, match=match):
        read(tmp_path, edit(path, value))


def test_reference_checks_come_before_layout_checks(tmp_path):
    # every_n_layers 2 is a layout the context cannot hold, but the schedule error the
    # reference raises first wins
    cfg = edit(("moe", "every_n_layers"), 2)
    cfg["attention_schedule"]["full_attention_every_n"] = 0
    with pytest.raises(A.ConfigError, match="full_attention_every_n"):
        read(tmp_path, cfg)


def test_ignored_fields_and_required_ones(tmp_path):
    cfg = base()
    cfg["mtp"] = {"num_future_tokens": 2, "aux_loss_weight": 0.3}
    cfg["qat"] = {"bits": "int4"}
    cfg["rope_scaling"] = dict(method="yarn", factor=4.0, original_max_seq_len=16)
    cfg["attention_schedule"]["mla_layers"] = [1, 0, 7]  # order free, out-of-range index ignored
    assert read(tmp_path, cfg).n_layers == 2
    for key in ("tie_embeddings", "ffn_dim", "n_kv_heads"):
        bad = copy.deepcopy(base())
        del bad[key]
        with pytest.raises(A.CheckpointError, match=key):
            read(tmp_path, bad)
    bad = base()
    bad["moe"]["top_k"] = "two"
    with pytest.raises(A.CheckpointError, match="moe"):
        read(tmp_path, bad)
