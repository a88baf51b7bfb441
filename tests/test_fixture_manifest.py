"""Manifest fixtures (strix_trellis.load_fixture), on synthetic groups.

The reference loads EXL3 groups cut out of published checkpoints through a
JSON manifest of files with sizes and SHA-256 digests (reference
python/strix_trellis/fixture.py:11-29; its test tests/test_fixture_io.py:63-88
rejects a changed file and a foreign mul1 marker).  The checkpoints need the
network, so these tests write their own manifests of the same structure.
"""
import hashlib
import json

import numpy as np
import pytest

import synth
from strix_trellis import load_fixture

MUL1 = 0x83DCD12D


def _write(directory, parts, prefix="layers.0.attn.wkv", fixture_directory=None):
    meta = {"fixture_directory": str(fixture_directory or directory), "tensors": {}}
    for part, (array, dtype) in parts.items():
        data = np.ascontiguousarray(array).tobytes()
        (directory / f"{part}.bin").write_bytes(data)
        meta["tensors"][f"{prefix}.{part}"] = {"file": f"{part}.bin", "bytes": len(data),
                                               "sha256": hashlib.sha256(data).hexdigest(),
                                               "shape": list(np.shape(array)), "dtype": dtype}
    manifest = directory / "manifest.json"
    manifest.write_text(json.dumps(meta), encoding="utf-8")
    return manifest


def _group(K=4, marker=MUL1):
    tr, suh, svh, _ = synth.layer(256, 128, K, 71)
    return {"trellis": (tr.view("<i2"), "I16"), "suh": (suh.astype("<f2"), "F16"),
            "svh": (svh.astype("<f2"), "F16"), "mul1": (np.array(np.uint32(marker).view(np.int32)), "I32")}


def test_round_trip(tmp_path):
    parts = _group(K=5)
    manifest = _write(tmp_path, parts)
    trellis, suh, svh, k = load_fixture(manifest)
    assert trellis.dtype == np.dtype("<i2") and trellis.shape == parts["trellis"][0].shape
    assert np.array_equal(trellis, parts["trellis"][0])
    assert np.array_equal(suh.view(np.uint16), parts["suh"][0].view(np.uint16))
    assert np.array_equal(svh.view(np.uint16), parts["svh"][0].view(np.uint16))
    assert k == 5 and isinstance(k, float)   # the reference returns shape[-1] / 16


def test_directory_argument_overrides_the_manifest(tmp_path):
    data_dir = tmp_path / "data"
    data_dir.mkdir()
    manifest = _write(data_dir, _group(), fixture_directory=tmp_path / "elsewhere")
    with pytest.raises(FileNotFoundError):
        load_fixture(manifest)
    assert load_fixture(manifest, data_dir)[3] == 4


def test_changed_bytes_and_foreign_marker_rejected(tmp_path):
    manifest = _write(tmp_path, _group(marker=0xCBAC1FED))
    with pytest.raises(ValueError, match="Unsupported mul1 multiplier"):
        load_fixture(manifest)
    manifest = _write(tmp_path, _group())
    load_fixture(manifest)
    raw = bytearray((tmp_path / "svh.bin").read_bytes())
    raw[3] ^= 1   # same size, different digest
    (tmp_path / "svh.bin").write_bytes(bytes(raw))
    with pytest.raises(ValueError, match="integrity check failed: layers.0.attn.wkv.svh"):
        load_fixture(manifest)
    (tmp_path / "svh.bin").write_bytes(bytes(raw[:-2]))   # short file
    with pytest.raises(ValueError, match="integrity"):
        load_fixture(manifest)
