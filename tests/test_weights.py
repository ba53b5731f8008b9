"""Weight ingestion (GGUF v1 and safetensors) -- CPU tests.

1. The oracle codecs (oracle/refgguf.py) pinned by the reference's own known-answer
   tests (gguf_quant.rs:115-137, gguf.rs:316-340) and by closed forms: the IEEE
   binary16 value formula for all 65536 bit patterns, round-to-nearest with ties away
   from zero for f32 -> f16, exactly representable Q4_K_M / Q8_0 grids, and the
   container bytes packed field by field.
2. The library's host readers (aarh_gguf_read_tensor, aarh_safetensors_read_tensor,
   aarh_gguf_config) bit-exact against the committed fixtures of
   tests/golden/make_weight_fixtures.py and against the oracle on files written at
   test time; the reference's error kinds for malformed files.
No device call is made (these entry points are host code)."""
import json
import os
import struct

import numpy as np
import pytest

import aarambh_hip as A
import refgguf as G

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def same_bits(a, b):
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    if a.shape != b.shape:
        return False
    na, nb = np.isnan(a), np.isnan(b)
    return bool(np.array_equal(na, nb) and np.array_equal(a[~na].view(np.uint32), b[~nb].view(np.uint32)))


# ---------------------------------------------------------------- oracle pins
def test_reference_kat_f16_roundtrip():
    # gguf_quant.rs:115-122
    for v in [-12.5, -1.0, 0.0, 0.5, 3.25, 100.0]:
        d = G.f16_to_f32(G.f32_to_f16(np.float32(v)))
        assert abs(float(d) - v) < 0.05


def test_reference_kat_q4_block_ramp():
    # gguf_quant.rs:124-136: idx * 0.01 - 1.28 round-trips within 0.09
    w = (np.arange(256, dtype=np.float32) * np.float32(0.01) - np.float32(1.28)).astype(np.float32)
    d = G.dequantise_block_q4km(G.quantise_block_q4km(w))
    assert np.abs(d - w).max() < 0.09


def test_reference_kat_f16_pair_and_q4_payload_shape():
    # gguf.rs:316-340: (0.125, -2.5) survive the f16 pair; a (20, 15) tensor -> 2 blocks, same dims
    s, m = G.f16_to_f32(G.f32_to_f16(np.array([0.125, -2.5], np.float32)))
    assert abs(s - 0.125) < 1e-3 and abs(m + 2.5) < 1e-3
    t = (np.arange(300, dtype=np.float32) * np.float32(0.01) - np.float32(1.5)).reshape(20, 15)
    pl = G.encode_tensor(G.ENC_Q4KM, t)
    assert len(pl) == 2 * G.Q4KM_BYTES
    assert G.decode_tensor(G.ENC_Q4KM, (20, 15), pl).shape == (20, 15)


def test_f16_to_f32_closed_form_all_patterns():
    h = np.arange(65536, dtype=np.uint32)
    s, e, m = (h >> 15) & 1, (h >> 10) & 31, (h & 1023).astype(np.float64)
    sign = np.where(s == 1, -1.0, 1.0)
    val = np.where(e == 0, m * 2.0 ** -24, (1 + m / 1024) * 2.0 ** (e.astype(np.float64) - 15)) * sign
    got = G.f16_to_f32(h.astype(np.uint16)).astype(np.float64)
    fin = e != 31
    assert np.array_equal(got[fin], val[fin])
    assert np.all(np.isinf(got[(e == 31) & (m == 0)])) and np.all(np.isnan(got[(e == 31) & (m != 0)]))
    assert np.array_equal(np.signbit(got[fin]), s[fin] == 1)


def _half_away(x):
    """Nearest f16 to f32 x, ties away from zero, from the binary16 value set."""
    grid = G.f16_to_f32(np.arange(0, 0x7C00, dtype=np.uint16)).astype(np.float64)  # +0 .. max finite
    ax = np.abs(x.astype(np.float64))
    i = np.clip(np.searchsorted(grid, ax, side="right") - 1, 0, grid.size - 1)
    lo = grid[i]
    hi = np.where(i + 1 < grid.size, grid[np.minimum(i + 1, grid.size - 1)], 65536.0)
    pick_hi = (ax - lo) >= (hi - ax)
    code = np.where(pick_hi, i + 1, i).astype(np.int64)  # 0x7C00 = inf when past max
    return (code | np.where(np.signbit(x), 0x8000, 0)).astype(np.uint16)


def test_f32_to_f16_nearest_ties_away():
    rng = np.random.default_rng(5)
    # every exponent a half can reach (subnormals included) plus overflow/underflow margins
    exps = rng.integers(127 - 26, 127 + 17, 400000)
    bits = (rng.integers(0, 2, exps.size) << 31) | (exps << 23) | rng.integers(0, 1 << 23, exps.size)
    # exact ties and their neighbours for every finite half
    g = G.f16_to_f32(np.arange(0, 0x7BFF, dtype=np.uint16)).astype(np.float64)
    mid = ((g[:-1] + g[1:]) / 2).astype(np.float32)
    x = np.concatenate([bits.astype(np.uint32).view(np.float32), mid, np.nextafter(mid, 0), np.nextafter(mid, 1),
                        -mid, np.float32([0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e-8, 5.96e-8, 2.98e-8])])
    x = x[np.isfinite(x)]
    assert np.array_equal(G.f32_to_f16(x), _half_away(x))
    assert G.f32_to_f16(np.float32(np.inf)) == 0x7C00 and G.f32_to_f16(np.float32(-np.inf)) == 0xFC00
    assert G.f32_to_f16(np.float32(np.nan)) & 0x7E00 == 0x7E00


def test_q4km_exact_grid_and_nibble_order():
    # min -2 and scale 0.5 are exact in f16; values min + q * scale round-trip exactly
    q = (np.arange(256) * 7 + 3) % 16
    q[0], q[1] = 0, 15  # range exactly 15 * 0.5
    w = (-2.0 + 0.5 * q).astype(np.float32)
    blk = G.quantise_block_q4km(w)
    assert struct.unpack("<HH", blk[:4]) == (0x3800, 0xC000)  # 0.5, -2.0
    assert blk[4] == (q[0] | (q[1] << 4)) and blk[5] == (q[2] | (q[3] << 4))  # even index in the low nibble
    assert np.array_equal(G.dequantise_block_q4km(blk), w)
    c = G.dequantise_block_q4km(G.quantise_block_q4km(np.full(256, 3.0, np.float32)))
    assert np.array_equal(c, np.full(256, 3.0, np.float32))  # zero range: scale 1.0, codes 0


def test_q8_exact_integers_and_epsilon_scale():
    v = np.arange(-127, 128, dtype=np.float32)
    pl = G.encode_tensor(G.ENC_Q8_0, v)
    assert struct.unpack("<f", pl[:4])[0] == 1.0 and np.array_equal(np.frombuffer(pl[4:], np.int8), v)
    assert np.array_equal(G.decode_tensor(G.ENC_Q8_0, v.shape, pl), v)
    tiny = np.full(5, 1e-9, np.float32)
    pl = G.encode_tensor(G.ENC_Q8_0, tiny)
    assert struct.unpack("<f", pl[:4])[0] == 1.0 and not any(pl[4:])


def test_container_bytes_field_by_field(tmp_path):
    a = np.arange(6, dtype=np.float32).reshape(2, 3)
    cfg = G.model_config_json(8, 4, 8, 1, 1, 1, 16)
    meta = json.dumps({"config": cfg, "format": "Q80"}, separators=(",", ":")).encode()
    want = b"GGUF" + struct.pack("<IQ", 1, len(meta)) + meta + struct.pack("<Q", 2)
    # sorted by name: "a.w" (2-D -> Q8_0), then "b" (1-D -> F32)
    want += struct.pack("<Q", 3) + b"a.w" + struct.pack("<QQQ", 2, 2, 3) + bytes([1])
    q8 = struct.pack("<f", np.float32(5.0) / np.float32(127.0)) + bytes(
        [int(round(x * 127 / 5)) & 0xFF for x in range(6)])
    want += struct.pack("<Q", len(q8)) + q8
    want += struct.pack("<Q", 1) + b"b" + struct.pack("<QQ", 1, 3) + bytes([0]) + struct.pack("<Q", 12)
    want += np.float32([1, 2, 3]).tobytes()
    p = tmp_path / "t.gguf"
    G.save_gguf(str(p), cfg, "Q80", {"b": np.float32([1, 2, 3]), "a.w": a})
    assert p.read_bytes() == want
    meta_r, t = G.load_gguf_tensors(str(p))
    assert meta_r["config"] == cfg and np.array_equal(t["b"], [1, 2, 3])


# ------------------------------------------------------- library host readers
FIXTURES = ["weights_tiny_q4km.gguf", "weights_tiny_q80.gguf", "weights_tiny_f32.safetensors",
            "weights_tiny_f16.safetensors", "weights_tiny_bf16.safetensors"]


def test_committed_fixtures_decode_bit_exact():
    exp = np.load(os.path.join(GOLD, "weights_tiny_expected.npz"))
    seen = 0
    for key in exp.files:
        fname, name = key.split("|", 1)
        path = os.path.join(GOLD, fname)
        if fname.endswith(".gguf"):
            got, enc = A.gguf_read_tensor(path, name)
            _, ref = G.load_gguf_tensors(path)
            assert same_bits(ref[name], exp[key]), key
            assert enc == G.encoding_for(name, exp[key].shape, "Q80" if "q80" in fname else "Q4KM")
        else:
            got = A.safetensors_read_tensor(path, name)
        assert same_bits(got, exp[key]), key
        seen += 1
    assert seen == 9 * len(FIXTURES)


@pytest.mark.parametrize("fmt", ["Q4KM", "Q80"])
def test_random_gguf_library_equals_oracle(tmp_path, fmt):
    rng = np.random.default_rng(11 if fmt == "Q4KM" else 12)
    tensors = {}
    for i in range(12):
        shape = tuple(int(d) for d in rng.integers(1, 70, rng.integers(1, 3)))
        tensors[f"t{i}.w" if i % 5 else f"t{i}_conv.w"] = (rng.standard_cauchy(shape) * 0.1).astype(np.float32)
    tensors["x.dsa.index_k.weight"] = rng.normal(size=(3, 300)).astype(np.float32)
    p = str(tmp_path / "r.gguf")
    with np.errstate(all="ignore"):
        G.save_gguf(p, G.model_config_json(8, 4, 8, 1, 1, 1, 16), fmt, tensors)
        _, ref = G.load_gguf_tensors(p)
    for name, v in ref.items():
        got, _ = A.gguf_read_tensor(p, name)
        assert same_bits(got, v), name


def test_gguf_config_from_file(tmp_path):
    p = str(tmp_path / "c.gguf")
    G.save_gguf(p, G.model_config_json(4096, 512, 1536, 3, 8, 2, 777, rope_theta=500000.0, norm_eps=1e-6,
                                       num_future_tokens=3), "Q4KM", {"n": np.ones(3, np.float32)})
    c = A.ModelConfig.from_gguf(p, weight_format=A.W_INT4_G128)
    assert (c.vocab_size, c.hidden_dim, c.ffn_dim, c.n_layers, c.n_heads, c.n_kv_heads, c.max_seq_len) == \
        (4096, 512, 1536, 3, 8, 2, 777)
    assert c.rope_theta == 500000.0 and c.norm_eps == np.float32(1e-6) and c.num_future_tokens == 3
    assert c.weight_format == A.W_INT4_G128


def _gguf_bytes(version=1, enc=0, payload=b"\0" * 8, shape=(2,), magic=b"GGUF", meta_edit=None):
    meta = json.dumps({"config": G.model_config_json(8, 4, 8, 1, 1, 1, 16), "format": "Q80"})
    if meta_edit:
        meta = meta_edit(meta)
    meta = meta.encode()
    b = magic + struct.pack("<IQ", version, len(meta)) + meta + struct.pack("<Q", 1)
    b += struct.pack("<Q", 1) + b"w" + struct.pack("<Q", len(shape)) + b"".join(struct.pack("<Q", d) for d in shape)
    return b + bytes([enc]) + struct.pack("<Q", len(payload)) + payload


@pytest.mark.parametrize("blob,err", [
    (_gguf_bytes(magic=b"GGUX"), A.CheckpointError),           # gguf.rs:101-106
    (_gguf_bytes(version=2), A.CheckpointError),               # gguf.rs:107-112
    (_gguf_bytes(enc=3), A.CheckpointError),                   # TensorEncoding::from_u8
    (_gguf_bytes(payload=b"\0" * 7), A.CheckpointError),       # invalid F32 payload length
    (_gguf_bytes(enc=1, payload=b"\0" * 3), A.CheckpointError),  # invalid Q8_0 payload
    (_gguf_bytes(enc=2, payload=b"\0" * 131), A.CheckpointError),  # invalid Q4_K_M payload length
    (_gguf_bytes()[:-3], A.IoError),                           # read_exact past the end
    # a NUL byte after a number is not JSON (serde_json rejects the metadata)
    (_gguf_bytes(meta_edit=lambda m: m.replace('"vocab_size": 8', '"vocab_size": 8\0')), A.CheckpointError),
])
def test_malformed_gguf_errors(tmp_path, blob, err):
    p = tmp_path / "bad.gguf"
    p.write_bytes(blob)
    with pytest.raises(err):
        A.gguf_read_tensor(str(p), "w")


def test_corrupt_sizes_fail_before_allocating(tmp_path):
    # a shape of 2^20 x 2^20 values over an 8-byte payload, and a payload length past the
    # end of the file, are refused from the header alone
    p = tmp_path / "big.gguf"
    p.write_bytes(_gguf_bytes(shape=(1 << 20, 1 << 20)))
    with pytest.raises(A.CheckpointError):
        A.gguf_read_tensor(str(p), "w")
    b = bytearray(_gguf_bytes())
    struct.pack_into("<Q", b, len(b) - 16, 1 << 60)  # the payload length field
    p.write_bytes(bytes(b))
    with pytest.raises(A.IoError):
        A.gguf_read_tensor(str(p), "w")


def test_missing_file_and_tensor(tmp_path):
    with pytest.raises(A.IoError):
        A.gguf_read_tensor(str(tmp_path / "none.gguf"), "w")
    p = tmp_path / "ok.gguf"
    p.write_bytes(_gguf_bytes())
    assert np.array_equal(A.gguf_read_tensor(str(p), "w")[0], [0.0, 0.0])
    with pytest.raises(A.ShapeError):
        A.gguf_read_tensor(str(p), "v")


def test_safetensors_bad_ranges(tmp_path):
    p = str(tmp_path / "s.safetensors")
    G.save_safetensors(p, {"a": np.ones((2, 3), np.float32)})
    raw = bytearray(open(p, "rb").read())
    (hl,) = struct.unpack_from("<Q", raw, 0)
    hdr = json.loads(raw[8:8 + hl])
    hdr["a"]["shape"] = [2, 4]  # byte range no longer matches the shape
    h = json.dumps(hdr).encode()
    open(p, "wb").write(struct.pack("<Q", len(h)) + h + raw[8 + hl:])
    with pytest.raises(A.CheckpointError):
        A.safetensors_read_tensor(p, "a")
    hdr["a"]["shape"], hdr["a"]["dtype"] = [2, 3], "I64"
    h = json.dumps(hdr).encode()
    open(p, "wb").write(struct.pack("<Q", len(h)) + h + raw[8 + hl:])
    with pytest.raises(A.UnsupportedError):
        A.safetensors_read_tensor(p, "a")
