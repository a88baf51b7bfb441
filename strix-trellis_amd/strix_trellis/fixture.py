"""STGPU001: the binary container of GPU parity fixtures.

Format (reference docs/GPU_TESTS.md:44-70; reader tests/gpu_runtime.hip:70-140):
little endian throughout; 8-byte ASCII magic ``STGPU001``, uint32 version (1),
uint32 section count; then each section is an 8-byte NUL-padded ASCII tag, a
uint64 byte length and exactly that many payload bytes, with no padding.

==========  ===========================================================
tag         payload
==========  ===========================================================
meta        8 uint32: I, N, bits, codebook enum, marker, rows, bias, seed
trellis     uint16 [I/16, N/16, 16 bits]
suh, svh    float16 [I] and [N]
bias        float32 [N], or empty when absent
x           float32 [rows, I], the original input
old         float32 [rows, N], the previous output (nonzero beta)
scaled      float16 [rows, I], RN16(x * suh)
inh         float32 [rows, I], H128 of scaled
a           float16 [rows, I], the core input
q           float16 [I, N], decoded Q in logical order
core        float32 [rows, N], the product of a and q
ref         float32 [rows, N], the layer output (with bias)
==========  ===========================================================

``read_stgpu`` validates size (<= 256 MiB), magic, version, duplicate and
missing sections, every length against the meta dimensions, the codebook
marker, and that no bytes trail the last section.  ``write_stgpu`` produces
the same layout from arrays.

``load_fixture`` reads the reference's other fixture form: an EXL3 group cut
out of a published checkpoint, described by a JSON manifest (reference
python/strix_trellis/fixture.py:11-29, tests/fixtures/eaq_v1.json).
"""
import hashlib
import json
import struct
from pathlib import Path

import numpy as np

MAGIC = b"STGPU001"
VERSION = 1
MAX_BYTES = 256 << 20
CODEBOOKS = ("3inst", "mcg", "mul1")
MARKERS = (0, 0xCBAC1FED, 0x83DCD12D)
META_FIELDS = ("I", "N", "bits", "codebook", "marker", "rows", "bias", "seed")


def _sections(meta):
    """Tag -> (dtype, shape) for the meta dimensions; bias may also be empty."""
    I, N, K, R = meta["I"], meta["N"], meta["bits"], meta["rows"]
    return {
        "trellis": ("<u2", (I // 16, N // 16, 16 * K)),
        "suh": ("<f2", (I,)), "svh": ("<f2", (N,)),
        "bias": ("<f4", (N,) if meta["bias"] else (0,)),
        "x": ("<f4", (R, I)), "old": ("<f4", (R, N)),
        "scaled": ("<f2", (R, I)), "inh": ("<f4", (R, I)), "a": ("<f2", (R, I)),
        "q": ("<f2", (I, N)), "core": ("<f4", (R, N)), "ref": ("<f4", (R, N)),
    }


def read_stgpu(path):
    """(meta dict, arrays dict) of a fixture file, validated as described above."""
    with open(path, "rb") as f:
        data = f.read(MAX_BYTES + 1)
    if len(data) > MAX_BYTES:
        raise ValueError("STGPU001 file exceeds 256 MiB")
    if len(data) < 16 or data[:8] != MAGIC:
        raise ValueError("Not an STGPU001 file")
    version, count = struct.unpack_from("<II", data, 8)
    if version != VERSION:
        raise ValueError(f"Unsupported STGPU001 version {version}")
    pos, raw = 16, {}
    for _ in range(count):
        if pos + 16 > len(data):
            raise ValueError("Truncated STGPU001 section header")
        tag_bytes = data[pos:pos + 8]
        tag = tag_bytes.rstrip(b"\0")
        if not tag or b"\0" in tag or not tag.isascii():
            raise ValueError("Invalid STGPU001 section tag")
        (length,) = struct.unpack_from("<Q", data, pos + 8)
        pos += 16
        if length > len(data) - pos:
            raise ValueError(f"Truncated STGPU001 section {tag!r}")
        name = tag.decode()
        if name in raw:
            raise ValueError(f"Duplicate STGPU001 section {name}")
        raw[name] = data[pos:pos + length]
        pos += length
    if pos != len(data):
        raise ValueError("Trailing bytes after the last STGPU001 section")
    if "meta" not in raw or len(raw["meta"]) != 32:
        raise ValueError("Missing or malformed STGPU001 meta section")
    meta = dict(zip(META_FIELDS, struct.unpack("<8I", raw["meta"])))
    I, N, K = meta["I"], meta["N"], meta["bits"]
    if not (I and N and I % 128 == 0 and N % 128 == 0 and 1 <= K <= 8 and meta["codebook"] < 3
            and meta["bias"] in (0, 1)):
        raise ValueError("Invalid STGPU001 dimensions, bits, codebook or bias flag")
    if meta["marker"] != MARKERS[meta["codebook"]]:
        raise ValueError("STGPU001 codebook marker does not match the codebook")
    arrays = {}
    for name, (dtype, shape) in _sections(meta).items():
        if name not in raw:
            raise ValueError(f"Missing STGPU001 section {name}")
        dt = np.dtype(dtype)
        want = int(np.prod(shape)) * dt.itemsize
        if len(raw[name]) != want:
            raise ValueError(f"STGPU001 section {name} holds {len(raw[name])} bytes, expected {want}")
        arrays[name] = np.frombuffer(raw[name], dtype=dt).reshape(shape)
    unknown = set(raw) - set(arrays) - {"meta"}
    if unknown:
        raise ValueError(f"Unknown STGPU001 sections: {sorted(unknown)}")
    return meta, arrays


def write_stgpu(path, meta, arrays):
    """Write `meta` (the eight fields) and the twelve arrays as an STGPU001 file."""
    meta = {k: int(meta[k]) for k in META_FIELDS}
    sections = [("meta", struct.pack("<8I", *(meta[k] for k in META_FIELDS)))]
    for name, (dtype, shape) in _sections(meta).items():
        arr = np.ascontiguousarray(arrays[name], dtype=np.dtype(dtype))
        if arr.shape != shape and not (arr.size == 0 and int(np.prod(shape)) == 0):
            raise ValueError(f"Section {name} has shape {arr.shape}, expected {shape}")
        sections.append((name, arr.tobytes()))
    out = bytearray(MAGIC + struct.pack("<II", VERSION, len(sections)))
    for name, payload in sections:
        out += name.encode().ljust(8, b"\0") + struct.pack("<Q", len(payload)) + payload
    if len(out) > MAX_BYTES:
        raise ValueError("STGPU001 file would exceed 256 MiB")
    with open(path, "wb") as f:
        f.write(out)


# ---------------------------------------------------------------------------
# Manifest fixtures (reference python/strix_trellis/fixture.py:11-29)
# ---------------------------------------------------------------------------
_MANIFEST_DTYPES = {"I16": "<i2", "I32": "<i4", "F16": "<f2"}
_MUL1_MULTIPLIER = MARKERS[CODEBOOKS.index("mul1")]


def load_fixture(manifest, directory=None):
    """(trellis, suh, svh, k) of the EXL3 group a fixture manifest describes.

    The manifest names each tensor ``<prefix>.<part>`` with its file, byte
    count, SHA-256, shape and dtype (I16 / I32 / F16); the files are read from
    `directory`, else from the manifest's ``fixture_directory``.  A file whose
    size or digest differs raises ValueError("Fixture integrity check failed:
    <name>"), and a ``mul1`` marker other than the mul1 multiplier raises
    ValueError("Unsupported mul1 multiplier").  k is the trellis's last
    dimension over 16, as the reference returns it (a float).
    """
    meta = json.loads(Path(manifest).read_text(encoding="utf-8"))
    base = Path(directory if directory is not None else meta["fixture_directory"])
    parts = {}
    for name, entry in meta["tensors"].items():
        data = (base / entry["file"]).read_bytes()
        if len(data) != entry["bytes"] or hashlib.sha256(data).hexdigest() != entry["sha256"]:
            raise ValueError(f"Fixture integrity check failed: {name}")
        part = name.rsplit(".", 1)[1]
        parts[part] = np.frombuffer(data, dtype=_MANIFEST_DTYPES[entry["dtype"]]).reshape(entry["shape"])
    if int(parts["mul1"].item()) & 0xFFFFFFFF != _MUL1_MULTIPLIER:
        raise ValueError("Unsupported mul1 multiplier")
    trellis = parts["trellis"]
    return trellis, parts["suh"], parts["svh"], trellis.shape[-1] / 16
