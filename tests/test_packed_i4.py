"""The PackedInt4Tensor boundary (quant/src/types.rs:79-90) on the host: the
conversion aarh_load_tensor_packed_i4 applies to the reference type's f32 group
scales and zeros (any multiple-of-128 group size) before the device repack.
Pinned against dequantise_packed_i4_to_vec (int4.rs:70-91, restated by the
oracle's ref_dequantise_i4), numpy's IEEE binary16 conversion (round to nearest,
ties to even), and the reference's error cases.  No GPU."""
import numpy as np
import pytest

import aarambh_hip as A
import refcpu as R


def packed(w, shape, group):
    data, sc, zz = R.quantise_i4(np.ascontiguousarray(w, np.float32).reshape(-1), group)
    return A.PackedInt4Tensor(tuple(shape), group, data, sc, zz)


def device_values(t):
    """(q - zero) * scale per element from the device parameters: the function the
    device's INT4 GEMV multiplies by (fp16 scale and zero of each 128-column group)."""
    sh, zh = A.packed_i4_params(t)
    rows, cols = int(np.prod(t.shape[:-1])), t.shape[-1]
    n = rows * cols
    codes = np.zeros(n, np.float32)
    codes[0::2] = t.data[: (n + 1) // 2] & 15
    codes[1::2] = (t.data[: n // 2] >> 4) & 15
    s = sh.view(np.float16).astype(np.float32)
    z = zh.view(np.float16).astype(np.float32)
    g = np.repeat(np.arange(cols // 128), 128)
    q = codes.reshape(rows, cols)
    return ((q - z[:, g]) * s[:, g]).astype(np.float32)


def reference_values(t):
    n = int(np.prod(t.shape))
    return R.dequantise_i4(t.data, n, t.group_size, t.scales, t.zeros).reshape(-1, t.shape[-1])


@pytest.mark.parametrize("shape,group", [((8, 256), 128), ((6, 512), 256), ((4, 256), 384), ((3, 384), 1152),
                                         ((2, 4, 128), 256)])
def test_device_values_follow_dequantise_packed_i4(shape, group):
    rng = np.random.default_rng(group)
    w = rng.normal(0, 0.02, int(np.prod(shape))).astype(np.float32)
    t = packed(w, shape, group)
    got, want = device_values(t), reference_values(t)
    # fp16 scale: within one half-ulp of binary16 (2^-11 relative) of the f32 scale's value
    assert np.all(np.abs(got - want) <= np.abs(want) * 2.0 ** -11 + 1e-12)
    # with scales that are fp16 values the device value is the reference value exactly
    t.scales = t.scales.astype(np.float16).astype(np.float32)
    assert np.array_equal(device_values(t), reference_values(t))


def test_group_mapping_across_rows():
    # group 256 over rows of 128: row r takes group r // 2; group 256 over rows of 512: two groups a row
    t = A.PackedInt4Tensor((4, 128), 256, np.zeros(256, np.uint8), np.array([1, 2], np.float32),
                           np.array([3, -4], np.float32))
    sh, zh = A.packed_i4_params(t)
    assert sh.view(np.float16).ravel().tolist() == [1, 1, 2, 2]
    assert zh.view(np.float16).ravel().tolist() == [3, 3, -4, -4]
    t = A.PackedInt4Tensor((2, 512), 256, np.zeros(512, np.uint8), np.arange(1, 5, dtype=np.float32),
                           np.zeros(4, np.float32))
    sh, _ = A.packed_i4_params(t)
    assert sh.view(np.float16).tolist() == [[1, 1, 2, 2], [3, 3, 4, 4]]


def test_scale_rounding_is_binary16_nearest_even():
    rng = np.random.default_rng(5)
    # every binade of the normal and subnormal fp16 range, plus exact tie points
    mags = np.exp2(rng.uniform(-26, 15.9, 60000)).astype(np.float32)
    ties = (np.arange(1, 2049, dtype=np.float32) + np.float32(0.5)) * np.float32(2.0 ** -10)  # halfway, [1, 3)
    sub_ties = (np.arange(0, 1024, dtype=np.float32) + np.float32(0.5)) * np.float32(2.0 ** -24)
    vals = np.concatenate([mags, -mags[:1000], ties, sub_ties, [0.0, 65504.0, 65519.99, 6.1e-5, 2.0 ** -25]])
    vals = vals.astype(np.float32)
    n = vals.size
    t = A.PackedInt4Tensor((n, 128), 128, np.zeros(n * 64, np.uint8), vals, np.zeros(n, np.float32))
    sh, _ = A.packed_i4_params(t)
    assert np.array_equal(sh.ravel(), vals.astype(np.float16).view(np.uint16))


@pytest.mark.parametrize("edit,err,text", [
    (dict(group_size=0), A.ConfigError, "group_size must be non-zero"),
    (dict(scales=np.ones(3, np.float32), zeros=np.zeros(3, np.float32)), A.ShapeError, "expected 4 int4 groups"),
    (dict(data=np.zeros(255, np.uint8)), A.ShapeError, "512 elements"),
    (dict(group_size=64, scales=np.ones(8, np.float32), zeros=np.zeros(8, np.float32)), A.UnsupportedError,
     "multiple of 128"),
    (dict(shape=(5, 100), group_size=125), A.UnsupportedError, "last dimension"),
    (dict(zeros=np.array([0, 1.5, 0, 0], np.float32)), A.UnsupportedError, "zero point"),
    (dict(zeros=np.array([0, 0, 1024, 0], np.float32)), A.UnsupportedError, "zero point"),
    (dict(scales=np.array([1, 1, 1, 7e4], np.float32)), A.UnsupportedError, "fp16"),
    (dict(scales=np.array([1, np.nan, 1, 1], np.float32)), A.UnsupportedError, "fp16"),
])
def test_errors(edit, err, text):
    kw = dict(shape=(4, 128), group_size=128, data=np.zeros(256, np.uint8), scales=np.ones(4, np.float32),
              zeros=np.zeros(4, np.float32))
    kw.update(edit)
    with pytest.raises(err, match=text):
        A.packed_i4_params(A.PackedInt4Tensor(**kw))


def test_zero_points_kept_exactly():
    z = np.array([-1023, -8, 0, 7, 15, 1023], np.float32)
    t = A.PackedInt4Tensor((6, 128), 128, np.zeros(384, np.uint8), np.ones(6, np.float32), z)
    _, zh = A.packed_i4_params(t)
    assert np.array_equal(zh.view(np.float16).astype(np.float32).ravel(), z)
