"""Pins the oracle's codecs (quant/src/int4.rs, absmax.rs, qat.rs:140-169) and
numeric-format conversions."""
import numpy as np
import torch

import refcpu as R


def test_int4_pack_order_low_nibble_is_even_index():  # int4.rs:45-53, 93-98
    w = np.arange(16, dtype=np.float32) * 0.1  # codes 0..15 exactly
    packed, sc, zz = R.quantise_i4(w, 16)
    assert list(packed) == [0x10, 0x32, 0x54, 0x76, 0x98, 0xBA, 0xDC, 0xFE]
    # odd count: last byte holds one low nibble (pack_unpack_i4_roundtrip_odd_count)
    packed, _, _ = R.quantise_i4(np.array([0, 1, 15, 7, 9], np.float32) / 15.0 * 15.0, 5)
    deq_codes = [(packed[i // 2] >> (4 * (i & 1))) & 15 for i in range(5)]
    assert deq_codes == [0, 1, 15, 7, 9]
    assert packed[2] >> 4 == 0


def test_int4_roundtrip_shape_and_error():  # int4.rs:100-121
    values = (np.arange(31, dtype=np.float32) * np.float32(0.03) - np.float32(0.5)).astype(np.float32)
    packed, sc, zz = R.quantise_i4(values, 8)
    dq = R.dequantise_i4(packed, 31, 8, sc, zz)
    assert np.max(np.abs(values - dq)) < 0.04


def test_int4_rounds_half_away_from_zero():
    # scale = 1, zero = 0: 2.5 -> 3 under Rust f32::round (banker's rounding would give 2).
    packed, sc, zz = R.quantise_i4(np.array([0.0, 2.5, 15.0, 6.5], np.float32), 4)
    assert sc[0] == 1.0 and zz[0] == 0.0
    assert packed[0] == (0 | (3 << 4)) and packed[1] == (15 | (7 << 4))


def test_int4_degenerate_group_uses_unit_scale():
    packed, sc, zz = R.quantise_i4(np.full(8, 0.3, np.float32), 8)
    assert sc[0] == 1.0
    dq = R.dequantise_i4(packed, 8, 8, sc, zz)
    assert np.allclose(dq, 0.0)


def test_int4_error_bound_and_code_range_exhaustive():
    rng = np.random.default_rng(0)
    w = rng.normal(0, 0.02, 128 * 64).astype(np.float32)
    packed, sc, zz = R.quantise_i4(w, 128)
    dq = R.dequantise_i4(packed, w.size, 128, sc, zz)
    for g in range(64):
        seg = slice(g * 128, (g + 1) * 128)
        assert sc[g] == np.float32((w[seg].max() - w[seg].min()) / np.float32(15.0))
        assert np.max(np.abs(dq[seg] - w[seg])) <= sc[g] * 0.5 * (1 + 1e-5)


def test_int4_f16_storage_codes_from_f32_scale():
    rng = np.random.default_rng(1)
    w = rng.normal(0, 0.02, 128 * 16).astype(np.float32)
    p32, sc, zz = R.quantise_i4(w, 128)
    p16, sh, zh = R.quantise_i4_f16(w, 128)
    assert np.array_equal(p32, p16)  # codes derived with the f32 scale
    assert np.array_equal(sh, sc.astype(np.float16).view(np.uint16))
    assert np.array_equal(zh, zz.astype(np.float16).view(np.uint16))
    dq = R.dequantise_i4_f16(p16, w.size, 128, sh, zh)
    codes = np.stack([p16 & 15, p16 >> 4], 1).ravel().astype(np.float32)
    s16 = np.repeat(sh.view(np.float16).astype(np.float32), 128)
    z16 = np.repeat(zh.view(np.float16).astype(np.float32), 128)
    assert np.array_equal(dq, ((codes - z16) * s16).astype(np.float32))


def test_int8_per_row_symmetric():  # qat.rs:155-169
    w = np.array([[0.5, -1.0, 0.25, 0.0], [0.0, 0.0, 0.0, 0.0], [3.0, 1.5, -0.75, 0.01]], np.float32)
    codes, sc = R.quantise_i8_rows(w)
    assert sc[0] == np.float32(1.0) / np.float32(127.0) and sc[1] == 1.0
    assert codes[0, 1] == -127 and codes[2, 0] == 127 and codes[0, 0] == 64  # 63.5 -> 64 away from zero
    assert np.all(codes[1] == 0)
    assert np.max(np.abs(codes * sc[:, None] - w)) <= np.max(sc) * 0.5 * (1 + 1e-5)


def test_kv_row_int8_rule():
    x = np.array([0.0, 1.27, -2.54, 0.005], np.float32)
    codes, sh = R.quantise_kv_row(x)
    s = np.float32(np.float32(2.54) / np.float32(127.0))
    assert sh == np.array([s], np.float32).astype(np.float16).view(np.uint16)[0]
    assert list(codes) == [0, int(np.round(np.float32(1.27) / s)), -127, 0]


def test_f16_conversion_matches_numpy_rne():
    rng = np.random.default_rng(2)
    xs = np.concatenate([
        rng.normal(0, 1, 20000), rng.normal(0, 1e-5, 5000), rng.normal(0, 3e4, 5000),
        [0.0, -0.0, 65504.0, 65519.0, 65520.0, 1e9, -1e9, 2.0**-24, 2.0**-25, 3 * 2.0**-26,
         2.0**-14, 1.0 + 2.0**-11, 1.0 + 3 * 2.0**-11, np.inf, -np.inf]]).astype(np.float32)
    got = R.f32_to_f16_bits(xs)
    assert np.array_equal(got, xs.astype(np.float16).view(np.uint16))
    back = np.array([R.lib().ref_f16_to_f32(int(h)) for h in got], np.float32)
    assert np.array_equal(back, got.view(np.float16).astype(np.float32))


def test_bf16_conversion_matches_torch_rne():
    rng = np.random.default_rng(3)
    xs = np.concatenate([rng.normal(0, 1, 20000), rng.normal(0, 1e30, 100),
                         [1.0 + 2.0**-8, 1.0 + 3 * 2.0**-8, 0.0, -0.0]]).astype(np.float32)
    got = np.array([R.lib().ref_f32_to_bf16(float(v)) for v in xs], np.uint16)
    want = torch.from_numpy(xs).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, want)


def test_synthetic_generator_is_normal_and_deterministic():
    a = R.synth_fill(0, 5, 200000, 0.02)
    assert np.array_equal(a, R.synth_fill(0, 5, 200000, 0.02))
    assert abs(a.mean()) < 2e-4 and abs(a.std() - 0.02) < 2e-4
    assert not np.array_equal(a[:100], R.synth_fill(0, 6, 100, 0.02))
    t = R.synth_tokens(0, 1, 10000, 4096)
    assert t.max() < 4096 and len(np.unique(t)) > 3000
