"""The NumPy oracle against the reference's own scalar host oracle.

``oracle/_ref/libstrix_ref.so`` is compiled from the reference tree's
src/host_reference.hpp (recipe: ``make -C oracle ref``).  These tests pin the
restated ring-window extraction (reference host_reference.hpp:5-13) and all
three codebooks (host_reference.hpp:22-36) state by state.  They skip where the
library was not built (hosts without the reference tree).
"""
import ctypes as C
from pathlib import Path

import numpy as np
import pytest

from oracle import codec

LIB = Path(__file__).resolve().parents[1] / "oracle" / "_ref" / "libstrix_ref.so"
REF_CODEBOOK_ID = {"3inst": 0, "mcg": 1, "mul1": 2}


@pytest.fixture(scope="module")
def ref():
    if not LIB.exists():
        pytest.skip("reference host oracle not built (make -C oracle ref needs the reference tree)")
    lib = C.CDLL(str(LIB))
    lib.stx_ref_codebook_table.argtypes = [C.c_int, C.c_void_p]
    lib.stx_ref_tile_states.argtypes = [C.c_void_p, C.c_int, C.c_void_p]
    lib.stx_ref_state.argtypes = [C.c_void_p, C.c_int, C.c_int]
    lib.stx_ref_state.restype = C.c_uint16
    return lib


@pytest.mark.parametrize("name", codec.CODEBOOKS)
def test_codebook_tables_match_reference_host_oracle(ref, name):
    got = np.empty(65536, np.uint16)
    ref.stx_ref_codebook_table(REF_CODEBOOK_ID[name], got.ctypes.data)
    mine = codec.codebook_table(name).view(np.uint16)
    bad = np.flatnonzero(got != mine)
    assert bad.size == 0, f"{name}: {bad.size} states differ, first {bad[:4]}"


@pytest.mark.parametrize("k", range(1, 9))
def test_tile_states_match_reference_host_oracle(ref, k):
    rng = np.random.Generator(np.random.PCG64(700 + k))
    tiles = rng.integers(0, 65536, (64, 16 * k), dtype=np.uint16)
    # ring-wrap vectors of the reference tests: a lone MSB in word 1 and a lone
    # LSB in the second-to-last word
    tiles[0] = 0
    tiles[0, 1] = 0x8000
    tiles[1] = 0
    tiles[1, -2] = 1
    mine = codec.unpack_states(tiles, k)
    ring = codec.ring_words(tiles, k).astype(np.uint32)
    for t in range(tiles.shape[0]):
        words = np.ascontiguousarray(ring[t])
        got = np.empty(256, np.uint16)
        ref.stx_ref_tile_states(words.ctypes.data, k, got.ctypes.data)
        np.testing.assert_array_equal(mine[t], got, err_msg=f"K={k} tile {t}")


def test_dequantized_tile_matches_reference_chain(ref):
    """Full chain on one K5 tile: states -> mul1 -> 16x16 position map."""
    k = 5
    rng = np.random.Generator(np.random.PCG64(811))
    tile = rng.integers(0, 65536, (16 * k,), dtype=np.uint16)
    ring = np.ascontiguousarray(codec.ring_words(tile, k).astype(np.uint32))
    states = np.empty(256, np.uint16)
    ref.stx_ref_tile_states(ring.ctypes.data, k, states.ctypes.data)
    table = np.empty(65536, np.uint16)
    ref.stx_ref_codebook_table(2, table.ctypes.data)
    values = table[states]
    q = codec.dequantize_rotated(tile.reshape(1, 1, 16 * k), k).view(np.uint16)
    for pos in range(256):
        t, j = divmod(pos, 8)
        row = 2 * (t % 4) + (j % 2) + 8 * ((j // 2) % 2)
        col = t // 4 + 8 * (j // 4)
        assert q[row, col] == values[pos], (pos, row, col)
