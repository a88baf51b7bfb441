"""CPU tests of the STGPU001 fixture container (strix_trellis.fixture) and of
the committed fixtures in tests/golden (written by tests/golden/make_stgpu.py).

The stage arrays of every fixture are recomputed here from its trellis, scales
and x by the oracle, so a fixture that no longer matches the oracle (or a
reader that misplaces a section) fails on the CPU before any GPU run."""
import struct
from pathlib import Path

import numpy as np
import pytest

from oracle import codec, linear
from strix_trellis.fixture import CODEBOOKS, read_stgpu, write_stgpu

GOLDEN = sorted((Path(__file__).parent / "golden").glob("*.stgpu"))


def test_golden_fixtures_exist():
    assert len(GOLDEN) >= 4


@pytest.mark.parametrize("path", GOLDEN, ids=lambda p: p.stem)
def test_golden_fixture_stages_follow_the_oracle(path):
    meta, f = read_stgpu(path)
    cb = CODEBOOKS[meta["codebook"]]
    bias = f["bias"] if meta["bias"] else None
    assert f["x"].shape == (meta["rows"], meta["I"]) and (bias is None) == (f["bias"].size == 0)
    q = codec.dequantize_rotated(f["trellis"], meta["bits"], cb)
    np.testing.assert_array_equal(q.view(np.uint16), f["q"].view(np.uint16))
    ins = linear.input_stages_fp32(f["x"], f["suh"])
    for key, name in (("scaled", "scaled_fp16"), ("inh", "input_hadamard_fp32"), ("a", "core_input_fp16")):
        np.testing.assert_array_equal(np.asarray(ins[name]).view(np.uint8), f[key].view(np.uint8))
    out = linear.output_stages_fp32(f["core"], f["svh"], bias)["output_fp32"]
    np.testing.assert_array_equal(out.view(np.uint32), f["ref"].view(np.uint32))
    # the core of the first rows, recomputed
    core = linear.core_dot_fp32(f["a"][:2], f["q"])
    np.testing.assert_array_equal(core.view(np.uint32), f["core"][:2].view(np.uint32))


def _small(tmp_path, bias=True):
    g = np.random.Generator(np.random.PCG64(3))
    meta = {"I": 128, "N": 128, "bits": 2, "codebook": 2, "marker": 0x83DCD12D, "rows": 2, "bias": int(bias), "seed": 3}
    arrays = {"trellis": g.integers(0, 65536, (8, 8, 32), dtype=np.uint16),
              "suh": np.ones(128, np.float16), "svh": np.ones(128, np.float16),
              "bias": np.arange(128, dtype=np.float32) if bias else np.zeros(0, np.float32)}
    for k, (dt, shape) in {"x": ("f4", (2, 128)), "old": ("f4", (2, 128)), "scaled": ("f2", (2, 128)),
                          "inh": ("f4", (2, 128)), "a": ("f2", (2, 128)), "q": ("f2", (128, 128)),
                          "core": ("f4", (2, 128)), "ref": ("f4", (2, 128))}.items():
        arrays[k] = g.standard_normal(shape).astype(dt)
    path = tmp_path / "t.stgpu"
    write_stgpu(path, meta, arrays)
    return path, meta, arrays


def test_round_trip(tmp_path):
    for bias in (True, False):
        path, meta, arrays = _small(tmp_path, bias)
        m, a = read_stgpu(path)
        assert m == meta
        for k, v in arrays.items():
            np.testing.assert_array_equal(a[k], v)


def _sections(blob):
    count = struct.unpack_from("<I", blob, 12)[0]
    pos, out = 16, []
    for _ in range(count):
        tag = blob[pos:pos + 8]
        n = struct.unpack_from("<Q", blob, pos + 8)[0]
        out.append((tag, blob[pos + 16:pos + 16 + n]))
        pos += 16 + n
    return out


def _pack(sections, version=1, magic=b"STGPU001"):
    out = bytearray(magic + struct.pack("<II", version, len(sections)))
    for tag, payload in sections:
        out += tag + struct.pack("<Q", len(payload)) + payload
    return bytes(out)


def test_corrupt_files_are_rejected(tmp_path):
    path, meta, arrays = _small(tmp_path)
    good = path.read_bytes()
    secs = _sections(good)
    bad_meta = bytearray(secs[0][1])
    struct.pack_into("<I", bad_meta, 16, 0)          # marker that does not fit mul1
    corrupt = {
        "magic": _pack(secs, magic=b"STGPU002"),
        "version": _pack(secs, version=2),
        "duplicate": _pack(secs + [secs[-1]]),
        "missing": _pack([s for s in secs if s[0].rstrip(b"\0") != b"q"]),
        "length": _pack([(t, p[:-4] if t.rstrip(b"\0") == b"ref" else p) for t, p in secs]),
        "marker": _pack([(secs[0][0], bytes(bad_meta))] + secs[1:]),
        "unknown": _pack(secs + [(b"extra\0\0\0", b"")]),
        "trailing": good + b"\0",
        "truncated": good[:-1],
    }
    for name, blob in corrupt.items():
        path.write_bytes(blob)
        with pytest.raises(ValueError):
            read_stgpu(path)
        assert name
