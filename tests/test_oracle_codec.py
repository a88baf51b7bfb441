"""Pins the CPU decode oracle against the reference's known answers.

Every expected value here is a golden vector held by the reference's own tests
or docs (cited per test) or follows from the format's mathematics by a route
independent of ``oracle.codec`` (Python integers, ``struct '<e'`` rounding,
bit-serial shift registers).
"""
import hashlib
import struct

import numpy as np
import pytest

from oracle import codec

RATES = (1, 1.5, 2, 2.5, 3, 3.5, 4, 5, 6, 7, 8)


def _byte_shift_register(tile_u16, k):
    """Physical little-endian bytes -> ring bits -> shift register.

    Restates the byte oracle of tests/test_reference.py:16-32: each uint32 is
    read from its four little-endian bytes, most significant byte first.
    """
    raw = np.asarray(tile_u16, dtype="<u2").tobytes()
    bits = []
    for offset in range(0, len(raw), 4):
        for byte in reversed(raw[offset:offset + 4]):
            bits.extend((byte >> (7 - b)) & 1 for b in range(8))
    state = 0
    for bit in bits[-16:]:
        state = ((state << 1) | bit) & 0xFFFF
    out, cursor = [], 0
    for i in range(256):
        width = int(k) + ((i % 2) if k % 1 else 0)
        for bit in bits[cursor:cursor + width]:
            state = ((state << 1) | bit) & 0xFFFF
        cursor += width
        out.append(state)
    return np.array(out, dtype=np.uint16)


@pytest.mark.parametrize("k", RATES)
def test_windows_match_byte_shift_register(k):
    # tests/test_reference.py:42-51 -- every rate, signed and big-endian storage.
    rng = np.random.default_rng(9823)
    words = rng.integers(0, 65536, (3, int(16 * k)), dtype=np.uint16)
    got = codec.unpack_states(words, k)
    for i in range(3):
        np.testing.assert_array_equal(got[i], _byte_shift_register(words[i], k))
        np.testing.assert_array_equal(got[i], codec.unpack_states_serial(words[i], k))
    np.testing.assert_array_equal(got, codec.unpack_states(words.view(np.int16), k))
    np.testing.assert_array_equal(got, codec.unpack_states(words.astype(">u2"), k))


@pytest.mark.parametrize("k", RATES)
def test_windows_multi_tile_chunking(k):
    rng = np.random.default_rng(7)
    words = rng.integers(-32768, 32768, size=(5, 3, int(16 * k)), dtype=np.int16)
    ref = np.stack([codec.unpack_states_serial(t, k) for t in words.reshape(-1, words.shape[-1])])
    for chunk in (1, 4, 8192):
        np.testing.assert_array_equal(codec.unpack_states(words, k, chunk).reshape(-1, 256), ref)


def test_ring_wrap_and_word_order():
    # tests/test_reference.py:59-67: word[1] = 0x8000 is ring bit 0 (MSB of the
    # first uint32), so at K=1 state i = 1 << i for i < 16 and state 16 = 0;
    # word[-2] = 1 is the last ring bit, i.e. bit 1 of the first window.
    words = np.zeros(16, dtype=np.uint16)
    words[1] = 0x8000
    states = codec.unpack_states(words, 1)
    np.testing.assert_array_equal(states[:16], 1 << np.arange(16))
    assert int(states[16]) == 0
    words[:] = 0
    words[-2] = 1
    assert int(codec.unpack_states(words, 1)[0]) == 2


def test_fragment_coordinates_all_positions():
    # tests/test_reference.py:69-81 lane/fragment formula over all 256 positions.
    words = np.random.default_rng(12).integers(0, 65536, 128, dtype=np.uint16)
    values = codec.decode_states(_byte_shift_register(words, 8))
    tile = codec.decode_tile(words, 8)
    seen = set()
    for lane in range(32):
        for frag in range(8):
            row = 2 * (lane % 4) + frag % 2 + 8 * ((frag // 2) % 2)
            col = lane // 4 + 8 * (frag // 4)
            assert tile[row, col].view(np.uint16) == values[8 * lane + frag].view(np.uint16)
            seen.add((row, col))
    assert len(seen) == 256


def test_first_and_last_eight_coordinates():
    # reference docs/DESIGN.md:106-109: explicit coordinates of positions 0..7 and 248..255.
    first = [(0, 0), (1, 0), (8, 0), (9, 0), (0, 8), (1, 8), (8, 8), (9, 8)]
    last = [(6, 7), (7, 7), (14, 7), (15, 7), (6, 15), (7, 15), (14, 15), (15, 15)]
    for pos, (r, c) in enumerate(first):
        assert codec.TILE_POSITION[r, c] == pos
    for pos, (r, c) in enumerate(last, start=248):
        assert codec.TILE_POSITION[r, c] == pos


def test_codebook_bit_vectors():
    # tests/test_reference.py:83-95.
    states = np.array([0, 1, 2, 255, 256, 32767, 32768, 65535])
    expected = {
        "mul1": [0xc2e8, 0x3921, 0xb72d, 0x3ab3, 0xb3db, 0x3fca, 0xbaf2, 0xb936],
        "mcg": [0x3f60, 0x304e, 0xba13, 0xbd26, 0xbaf0, 0x4172, 0xb915, 0x3acd],
        "3inst": [0x3a25, 0xbb5b, 0x3b74, 0x3cd1, 0x3c3f, 0xba96, 0xb7f8, 0xb110],
    }
    for name, bits in expected.items():
        got = codec.decode_states(states, name)
        np.testing.assert_array_equal(got.view(np.uint16), bits)
        np.testing.assert_array_equal(got.view(np.uint16), codec.decode_states(states + 65536, name).view(np.uint16))
        assert codec.decode_states(np.array([-1]), name).view(np.uint16)[0] == bits[-1]


def _half_units(bits):
    """Exact signed binary16 value in units of 2**-24 (subnormals included)."""
    exponent, fraction = (bits >> 10) & 31, bits & 1023
    magnitude = fraction if exponent == 0 else (1024 + fraction) << (exponent - 1)
    return -magnitude if bits & 0x8000 else magnitude


def _mathematical_codebook_bytes(name):
    """All 65,536 states by Python integers + stdlib binary16 rounding."""
    out = bytearray()
    for s in range(65536):
        if name == "mul1":
            p = (s * 0x83DCD12D) & 0xFFFFFFFF
            total = (p & 255) + ((p >> 8) & 255) + ((p >> 16) & 255) + (p >> 24)
            value = ((1024 + total) * 1774 - 1329 * 2048) / 262144
        else:
            mult, off = (89226354, 64248484) if name == "3inst" else (0xCBAC1FED, 0)
            q = (((s * mult + off) & 0xFFFFFFFF) & 0x8FFF8FFF) ^ 0x3B603B60
            value = (_half_units(q & 0xFFFF) + _half_units(q >> 16)) / 16777216
        out.extend(struct.pack("<e", value))
    return bytes(out)


@pytest.mark.parametrize("name,digest", [
    # docs/NUMERICS.md:128-140 and tests/test_numerics.py:74-87.
    ("3inst", "ad88de2dcff5bb05fff2faec37cceceb43aa1c2e8203f9d81a6fbd6dd3393eea"),
    ("mcg", "95383563929baa9d1ae5de0be22490284382673620bdd85929feea7bdbef04a9"),
    ("mul1", "bc48d02cb1c14939dc47b90f870dd689d63e3b1ab69a157e65538db68677a6c8"),
])
def test_codebook_sha256_all_states(name, digest):
    independent = _mathematical_codebook_bytes(name)
    assert hashlib.sha256(independent).hexdigest() == digest
    table = codec.codebook_table(name).astype("<f2").tobytes()
    assert table == independent


def test_mul1_is_single_rounding_not_two():
    # Rounding the product to half before the add must NOT reproduce the table
    # (docs/FORMAT.md:82-86): at least one state differs.
    table = codec.codebook_table("mul1").view(np.uint16)
    s = np.arange(65536, dtype=np.uint64)
    p = (s * np.uint64(0x83DCD12D)) & np.uint64(0xFFFFFFFF)
    b = sum(((p >> np.uint64(sh)) & np.uint64(255)).astype(np.int64) for sh in (0, 8, 16, 24))
    c1 = np.array([0x1EEE], dtype=np.uint16).view(np.float16)[0]
    c2 = np.array([0xC931], dtype=np.uint16).view(np.float16)[0]
    two = ((1024 + b).astype(np.float16) * c1).astype(np.float16) + c2
    assert np.any(two.astype(np.float16).view(np.uint16) != table)


def test_dequantize_multi_tile_layout():
    # Tile (a, b) -> Q[16a + r, 16b + c], input-major storage (FORMAT.md:66-69).
    rng = np.random.default_rng(11)
    for k in RATES:
        words = rng.integers(0, 65536, size=(2, 4, int(16 * k)), dtype=np.uint16)
        for cb in (("mul1",) if k % 1 else codec.CODEBOOKS):
            q = codec.dequantize_rotated(words, k, cb)
            assert q.shape == (32, 64)
            for a in range(2):
                for b in range(4):
                    states = codec.unpack_states_serial(words[a, b], k)
                    vals = codec.codebook_table(cb)[states]
                    for pos in (0, 1, 37, 128, 255):
                        t, j = divmod(pos, 8)
                        r = 2 * (t % 4) + j % 2 + 8 * ((j // 2) % 2)
                        c = t // 4 + 8 * (j // 4)
                        assert q[16 * a + r, 16 * b + c].view(np.uint16) == vals[pos].view(np.uint16)


def test_rejects_unsupported():
    for rate in [0, 9, 4.5, 1.25, float("nan"), float("inf"), True, "3"]:
        with pytest.raises(ValueError):
            codec.step_widths(rate)
    with pytest.raises(ValueError):
        codec.unpack_states(np.zeros(47, dtype=np.int16), 3)
    with pytest.raises(ValueError):
        codec.unpack_states(np.zeros(48, dtype=np.int32), 3)
    with pytest.raises(ValueError):
        codec.decode_tile(np.zeros(24, dtype=np.int16), 1.5, "mcg")
    with pytest.raises(ValueError):
        codec.decode_states([1], "unknown")
    with pytest.raises(ValueError):
        codec.decode_states([1.0])
