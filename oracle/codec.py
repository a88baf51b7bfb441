"""EXL3 trellis decode oracle (NumPy).  TEST INFRASTRUCTURE ONLY.

Restates the reference's CPU codec (python/strix_trellis/codec.py) from the
format specification (docs/FORMAT.md:42-101).  The window extraction used here
is a word-pair shift (two consecutive 32-bit ring words, shifted so the 16-bit
window lands in the low half) rather than the reference's bit unpacking, so the
two are independent derivations of the same rule.  A third, bit-serial form
(``unpack_states_serial``) advances a 16-bit shift register one stream bit at a
time and is what the tests pin the fast form against.

Parity pinning (tests/test_oracle_codec.py):
  * windows       -- bit-serial shift register, ring-wrap vectors of
                     tests/test_reference.py:59-67, and brute force at all rates;
  * codebooks     -- SHA-256 of all 65,536 states per codebook
                     (docs/NUMERICS.md:128-140) recomputed from Python integers
                     and ``struct '<e'`` rounding, plus the 8-state bit vectors
                     of tests/test_reference.py:83-95;
  * permutation   -- the explicit first/last eight coordinates of
                     reference docs/DESIGN.md:106-109 and the lane/fragment formula of
                     tests/test_reference.py:69-81 over all 256 positions.
"""
from functools import lru_cache
import math

import numpy as np

CODEBOOKS = ("3inst", "mcg", "mul1")
MUL1_MULTIPLIER = 0x83DCD12D
MCG_MULTIPLIER = 0xCBAC1FED
INST3_MULTIPLIER, INST3_OFFSET = 89226354, 64248484
# binary16 constants of the mul1 FMA: 0x1EEE = 1774 / 2**18, 0xC931 = -1329 / 128.
MUL1_SCALE_NUM, MUL1_SCALE_SHIFT = 1774, 18
MUL1_OFFSET_NUM = -1329 * 2048  # -1329/128 expressed in units of 2**-18


def step_widths(k):
    """Widths of the 256 ring transitions for rate ``k`` (codec.py:12-20).

    Integer rates 1..8 advance ``k`` bits per state; half rates 1.5, 2.5, 3.5
    alternate ``floor(k)`` (even positions) and ``floor(k)+1`` (odd positions),
    the 0xAAAA mask of docs/FORMAT.md:52-54.
    """
    if isinstance(k, (bool, np.bool_)) or not isinstance(k, (int, float, np.integer, np.floating)):
        raise ValueError("k must be an integer 1..8 or one of 1.5, 2.5, 3.5")
    rate = float(k)
    if not math.isfinite(rate) or rate not in (1, 2, 3, 4, 5, 6, 7, 8, 1.5, 2.5, 3.5):
        raise ValueError("Unsupported EXL3 bitrate")
    base = int(rate)
    odd = 1 if rate != base else 0
    return tuple(base + (odd if i & 1 else 0) for i in range(256))


def words_per_tile(k):
    """Number of 16-bit words in one tile: 256*k bits / 16."""
    return sum(step_widths(k)) // 16


@lru_cache(maxsize=16)
def _window_table(k):
    """Per state: (first ring word, next ring word, right shift) of its window.

    State ``i`` is the 16 ring bits ``[S(i)-16, S(i))`` modulo the ring length,
    MSB first, with ``S(i)`` the inclusive cumulative width (FORMAT.md:55-59).
    """
    widths = np.array(step_widths(k), dtype=np.int64)
    ring_bits = int(widths.sum())
    n32 = ring_bits // 32
    start = (np.cumsum(widths) - 16) % ring_bits
    first = start // 32
    second = (first + 1) % n32
    shift = 48 - (start % 32)
    return first, second, shift.astype(np.uint64), n32


def _as_u16_words(packed, k):
    words = np.asarray(packed)
    need = words_per_tile(k)
    if words.ndim < 1 or words.shape[-1] != need:
        raise ValueError(f"Expected {need} words per tile")
    if words.dtype.kind not in "iu" or words.dtype.itemsize != 2:
        raise ValueError("Packed storage must contain int16 or uint16 words")
    # Numerical reinterpretation: int16 wraps two's-complement, '>u2' keeps value.
    return words.astype(np.uint16, copy=False), need


def ring_words(packed, k):
    """[..., 16k] 16-bit words -> [..., 8k] uint32 ring words (lo | hi << 16)."""
    words, need = _as_u16_words(packed, k)
    pairs = words.reshape(words.shape[:-1] + (need // 2, 2)).astype(np.uint32)
    return pairs[..., 0] | (pairs[..., 1] << np.uint32(16))


def unpack_states(packed, k, chunk_tiles=16384):
    """[..., 16k] words -> [..., 256] uint16 states (codec.py:58-85, 123-147)."""
    words, need = _as_u16_words(packed, k)
    first, second, shift, n32 = _window_table(k)
    flat = words.reshape(-1, need)
    out = np.empty((flat.shape[0], 256), dtype=np.uint16)
    for begin in range(0, flat.shape[0], chunk_tiles):
        ring = ring_words(flat[begin:begin + chunk_tiles], k).astype(np.uint64)
        pair = (ring[:, first] << np.uint64(32)) | ring[:, second]
        out[begin:begin + ring.shape[0]] = ((pair >> shift) & np.uint64(0xFFFF)).astype(np.uint16)
    return out.reshape(words.shape[:-1] + (256,))


def unpack_states_serial(tile_words, k):
    """One tile, bit-serial: a 16-bit shift register fed MSB-first ring bits.

    Independent of ``unpack_states``: it starts from the last 16 ring bits
    (the wrap of reference docs/DESIGN.md:78-83) and shifts in ``width`` bits per state.
    """
    words, need = _as_u16_words(tile_words, k)
    if words.ndim != 1:
        raise ValueError("one tile expected")
    bits = []
    for pair in range(0, need, 2):
        value = int(words[pair]) | (int(words[pair + 1]) << 16)
        bits.extend((value >> (31 - b)) & 1 for b in range(32))
    register = 0
    for bit in bits[-16:]:
        register = ((register << 1) | bit) & 0xFFFF
    cursor, states = 0, []
    for width in step_widths(k):
        for bit in bits[cursor:cursor + width]:
            register = ((register << 1) | bit) & 0xFFFF
        cursor += width
        states.append(register)
    return np.array(states, dtype=np.uint16)


@lru_cache(maxsize=3)
def codebook_table(name):
    """binary16 value of every state 0..65535 (FORMAT.md:71-86, codec.py:27-46).

    mul1: ``p = s*0x83DCD12D mod 2**32``; ``b`` = sum of the four unsigned
    bytes of ``p``; value = RN16((1024+b)*h(0x1EEE) + h(0xC931)) with one
    rounding, evaluated exactly as the integer numerator
    ``(1024+b)*1774 - 1329*2048`` over ``2**18`` (exact in binary64).
    3inst/mcg: ``q = (p & 0x8FFF8FFF) ^ 0x3B603B60``; value = RN16 of the exact
    sum of q's two binary16 halves.
    """
    if name not in CODEBOOKS:
        raise ValueError(f"Unsupported codebook: {name}")
    s = np.arange(65536, dtype=np.uint64)
    mask32 = np.uint64(0xFFFFFFFF)
    if name == "mul1":
        p = (s * np.uint64(MUL1_MULTIPLIER)) & mask32
        b = sum(((p >> np.uint64(sh)) & np.uint64(255)).astype(np.int64) for sh in (0, 8, 16, 24))
        numerator = (1024 + b) * MUL1_SCALE_NUM + MUL1_OFFSET_NUM
        values = (numerator.astype(np.float64) / float(1 << MUL1_SCALE_SHIFT)).astype(np.float16)
    else:
        mult, off = ((INST3_MULTIPLIER, INST3_OFFSET) if name == "3inst" else (MCG_MULTIPLIER, 0))
        p = (s * np.uint64(mult) + np.uint64(off)) & mask32
        q = ((p & np.uint64(0x8FFF8FFF)) ^ np.uint64(0x3B603B60)).astype(np.uint32)
        lo = (q & np.uint32(0xFFFF)).astype(np.uint16).view(np.float16).astype(np.float64)
        hi = (q >> np.uint32(16)).astype(np.uint16).view(np.float16).astype(np.float64)
        values = (lo + hi).astype(np.float16)
    values.flags.writeable = False
    return values


def decode_states(states, codebook="mul1"):
    """Integer states (any integer dtype, reduced mod 2**16) -> binary16."""
    idx = np.asarray(states)
    if idx.dtype.kind not in "iu":
        raise ValueError("States must be integers")
    return codebook_table(codebook)[idx.astype(np.uint16)]


def _build_tile_position():
    """[16,16] ring position of every logical (row, col) of a tile.

    Inverts the fragment map of FORMAT.md:61-66: position ``8t+j`` goes to
    row ``2(t%4) + j%2 + 8((j//2)%2)``, col ``t//4 + 8(j//4)``.
    """
    table = np.full((16, 16), -1, dtype=np.int64)
    for t in range(32):
        for j in range(8):
            row = 2 * (t % 4) + (j % 2) + 8 * ((j // 2) % 2)
            col = t // 4 + 8 * (j // 4)
            table[row, col] = 8 * t + j
    assert (table >= 0).all()
    table.flags.writeable = False
    return table


TILE_POSITION = _build_tile_position()


def _check_codebook_rate(k, codebook):
    step_widths(k)
    if float(k) % 1 and codebook != "mul1":
        raise ValueError("Half-integer bitrates require mul1")


def decode_tile(packed, k, codebook="mul1"):
    """[..., 16k] words -> [..., 16, 16] logical tiles (codec.py:88-101)."""
    _check_codebook_rate(k, codebook)
    values = decode_states(unpack_states(packed, k), codebook)
    return values[..., TILE_POSITION]


def dequantize_rotated(trellis, k=None, codebook="mul1"):
    """[I/16, N/16, 16k] trellis -> float16 Q[I, N] (codec.py:150-173).

    Tile (a, b) covers Q[16a:16a+16, 16b:16b+16]; tiles are stored input-major.
    """
    data = np.asarray(trellis)
    if data.ndim != 3 or not data.shape[0] or not data.shape[1]:
        raise ValueError("Trellis must have three nonempty dimensions")
    if k is None:
        k = data.shape[-1] / 16
    tiles = decode_tile(data, k, codebook)
    return tiles.transpose(0, 2, 1, 3).reshape(data.shape[0] * 16, data.shape[1] * 16)
