"""Pins the oracle's RNG (rand 0.8 StdRng = ChaCha12, seed_from_u64) against
published vectors.  The 12-round StdRng word values themselves are not pinned by
any reference test (sampler.rs only checks distributions): parity unpinned for
the exact stream; the block function and seeding primitives are pinned here."""
import numpy as np

import refcpu as R


def test_chacha20_rfc7539_block_vector():
    # RFC 7539 section 2.3.2: key 00..1f, counter 1, nonce 00000009 0000004a 00000000.
    st = [0x61707865, 0x3320646E, 0x79622D32, 0x6B206574,
          0x03020100, 0x07060504, 0x0B0A0908, 0x0F0E0D0C,
          0x13121110, 0x17161514, 0x1B1A1918, 0x1F1E1D1C,
          0x00000001, 0x09000000, 0x4A000000, 0x00000000]
    want = [0xE4E7F110, 0x15593BD1, 0x1FDD0F50, 0xC47120A3,
            0xC7F4D1C7, 0x0368C033, 0x9AAA2204, 0x4E6CD4C3,
            0x466482D2, 0x09AA9F07, 0x05D7C214, 0xA2028BD9,
            0xD19C12B5, 0xB94E16DE, 0xE883D0CB, 0x4E3C50A2]
    assert list(R.chacha_core(st, 20)) == want


def test_chacha20_zero_key_keystream():
    # Zero key / zero nonce block 0 keystream (the vector rand_chacha's own tests use).
    st = [0x61707865, 0x3320646E, 0x79622D32, 0x6B206574] + [0] * 12
    want = [0xADE0B876, 0x903DF1A0, 0xE56A5D40, 0x28BD8653, 0xB819D2BD, 0x1AED8DA0,
            0xCCEF36A8, 0xC70D778B, 0x7C5941DA, 0x8D485751, 0x3FE02477, 0x374AD8B8,
            0xF4B8436A, 0x1CA11815, 0x69B687C3, 0x8665EEB2]
    assert list(R.chacha_core(st, 20)) == want


def test_pcg32_output_function_demo_vector():
    # pcg-c-basic demo (initstate 42, initseq 54) first outputs.
    MUL, M64 = 6364136223846793005, (1 << 64) - 1
    inc = ((54 << 1) | 1) & M64
    state = 0
    state = (state * MUL + inc) & M64
    state = (state + 42) & M64
    state = (state * MUL + inc) & M64
    got = []
    for _ in range(6):
        old = state
        state = (old * MUL + inc) & M64
        got.append(R.lib().ref_pcg32_xsh_rr(old))
    assert got == [0xA15C02B7, 0x7B47F409, 0xBA1D3330, 0x83D2F293, 0xBFA4784B, 0xCBED606E]


def test_stream_is_block_concatenation_and_seekable():
    r = R.Rng(1234)
    words = [r.next_u32() for _ in range(40)]
    for pos in (0, 15, 16, 17, 33):
        r2 = R.Rng(1234, pos)
        assert r2.next_u32() == words[pos]
    # Changing the round count or the seed changes the stream.
    assert words != [R.Rng(1235).next_u32() for _ in range(40)]


def test_f32_draws_are_24_bit_uniforms():
    r = R.Rng(7)
    xs = np.array([r.next_f32() for _ in range(20000)], np.float64)
    assert xs.min() >= 0.0 and xs.max() < 1.0
    assert np.all(np.floor(xs * 2**24) == xs * 2**24)
    assert abs(xs.mean() - 0.5) < 0.01
    assert abs(xs.var() - 1.0 / 12.0) < 0.003
