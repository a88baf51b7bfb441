"""CPU tests of the EXL3 safetensors loader and its transport exports
(strix_trellis.loader), modelled on the reference's tests/test_container.py.

Files are written two ways: with the ``safetensors`` package (an independent
writer, for the happy paths) and by a small writer here that can corrupt the
header.  The transport blob is checked against a packing written out
independently below, not against the loader's own layout code.
"""
import json
import struct

import numpy as np
import pytest

from strix_trellis.loader import Exl3Tensor, SafetensorsFile, load_exl3

safetensors_numpy = pytest.importorskip("safetensors.numpy")

MUL1, MCG = 0x83DCD12D, 0xCBAC1FED


def group_tensors(bits=3, marker="mul1", empty_marker=False, bias_dtype=np.float16, I=128, N=256):
    g = np.random.Generator(np.random.PCG64(73))
    out = {
        "proj.trellis": g.integers(-32768, 32768, (I // 16, N // 16, int(16 * bits)), dtype=np.int16),
        "proj.suh": np.linspace(-1, 1, I, dtype=np.float16),
        "proj.svh": np.linspace(0.25, -0.5, N, dtype=np.float16),
    }
    if bias_dtype is not None:
        out["proj.bias"] = (np.arange(N) / N).astype(bias_dtype)
    if marker:
        out["proj." + marker] = (np.empty(0, np.float16) if empty_marker
                                 else np.array([{"mul1": MUL1, "mcg": MCG}[marker]], np.uint32).view(np.int32).reshape(()))
    return out


def write_raw(path, tensors, mutate=None, pad=True):
    tags = {"int16": "I16", "int32": "I32", "float16": "F16", "float32": "F32", "uint16": "BF16"}
    data, header = bytearray(), {}
    for name, arr in tensors.items():
        payload = np.ascontiguousarray(arr).tobytes()
        header[name] = {"dtype": tags[arr.dtype.name], "shape": list(arr.shape),
                        "data_offsets": [len(data), len(data) + len(payload)]}
        data += payload
    if mutate:
        mutate(header)
    raw = json.dumps(header).encode()
    if pad:
        raw += b" " * (-len(raw) % 8)
    path.write_bytes(struct.pack("<Q", len(raw)) + raw + data)


def independent_blob(group):
    """Transport v1 by hand: trellis i16, suh f16, svh f16, bias f32 at 4-byte aligned offsets."""
    blob, fields = bytearray(), {}
    for name, dt in (("trellis", "<i2"), ("suh", "<f2"), ("svh", "<f2"), ("bias", "<f4")):
        v = getattr(group, name)
        if v is None:
            fields[name + "_offset"] = fields[name + "_bytes"] = 0
            continue
        blob += bytes(-len(blob) % 4)
        raw = np.asarray(v).astype(dt).tobytes()
        fields[name + "_offset"], fields[name + "_bytes"] = len(blob), len(raw)
        blob += raw
    fields.update(rows=group.output_size, columns=group.input_size, bits_x2=int(group.bits) * 2,
                  codebook={"3inst": 0, "mcg": 1, "mul1": 2}[group.codebook],
                  marker={"3inst": 0, "mcg": MCG, "mul1": MUL1}[group.codebook], transport_version=1)
    return bytes(blob), fields


@pytest.mark.parametrize("marker", [None, "mcg", "mul1"])
def test_groups_map_read_only_and_export(tmp_path, marker):
    path = tmp_path / "w.safetensors"
    src = group_tensors(marker=marker)
    safetensors_numpy.save_file(src, str(path))
    group = SafetensorsFile(path).exl3("proj")
    assert isinstance(group.trellis, np.memmap) and not group.trellis.flags.writeable
    assert (group.input_size, group.output_size, group.bits, group.codebook) == (128, 256, 3, marker or "3inst")
    np.testing.assert_array_equal(group.trellis, src["proj.trellis"])
    np.testing.assert_array_equal(group.svh, src["proj.svh"])
    assert group.bias.dtype == np.float32 and not group.bias.flags.writeable
    np.testing.assert_array_equal(group.bias, src["proj.bias"].astype(np.float32))
    blob, meta = group.transport_blob()
    want_blob, want_meta = independent_blob(group)
    assert meta == want_meta and blob == want_blob
    for name in ("trellis", "suh", "svh", "bias"):
        assert meta[name + "_offset"] % 4 == 0
    # regions: same bytes, views of the mapped file where no conversion is needed
    regions, rmeta = group.transport_regions()
    assert rmeta == meta
    assert np.shares_memory(np.frombuffer(regions["trellis"], np.uint8), group.trellis)
    for name in ("trellis", "suh", "svh", "bias"):
        off, n = meta[name + "_offset"], meta[name + "_bytes"]
        assert bytes(regions[name]) == blob[off:off + n]
        assert regions[name].readonly


def test_output_and_input_partitions(tmp_path):
    path = tmp_path / "w.safetensors"
    safetensors_numpy.save_file(group_tensors(bits=4, I=256, N=384), str(path))
    group = load_exl3(path, "proj")
    part = group.slice_outputs(128, 384)
    assert (part.input_size, part.output_size) == (256, 256)
    np.testing.assert_array_equal(part.trellis, group.trellis[:, 8:24])
    np.testing.assert_array_equal(part.svh, group.svh[128:384])
    np.testing.assert_array_equal(part.bias, group.bias[128:384])
    blob, meta = part.transport_blob()
    assert (blob, meta) == independent_blob(part)
    regions, _ = part.transport_regions()   # strided trellis: packed, scales borrowed
    assert not np.shares_memory(np.frombuffer(regions["trellis"], np.uint8), group.trellis)
    k = group.slice_inputs(128, 256, include_bias=False)
    assert (k.input_size, k.output_size, k.bias) == (128, 384, None)
    np.testing.assert_array_equal(k.suh, group.suh[128:256])
    assert k.slice_inputs(0, 128, include_bias=True).bias is None
    assert group.slice_inputs(0, 128, include_bias=True).bias is group.bias
    for bad in ((1, 129), (0, 0), (128, 512), (0.0, 128)):
        with pytest.raises(ValueError):
            group.slice_outputs(*bad)
    with pytest.raises(ValueError):
        group.slice_inputs(0, 128, include_bias=1)


def test_transport_buffer_destinations(tmp_path):
    path = tmp_path / "w.safetensors"
    src = group_tensors(bits=4, bias_dtype=None)
    safetensors_numpy.save_file(src, str(path))
    group = load_exl3(path, "proj")
    blob, meta = group.transport_blob()
    assert meta["bias_offset"] == meta["bias_bytes"] == 0
    buf, meta2 = group.transport_buffer()
    assert isinstance(buf, bytearray) and bytes(buf) == blob and meta2 == meta
    store = bytearray(b"\xab" * (len(blob) + 64))
    used, _ = group.transport_buffer(store)
    assert bytes(used) == blob and store[len(blob):] == b"\xab" * 64   # tail preserved
    arr = np.full(len(blob), 7, np.uint8)
    used, _ = group.transport_buffer(arr)
    assert arr.tobytes() == blob
    with pytest.raises(ValueError, match="too small"):
        group.transport_buffer(bytearray(len(blob) - 1))
    with pytest.raises(ValueError, match="writable"):
        group.transport_buffer(bytes(len(blob)))
    with pytest.raises(ValueError, match="contiguous"):
        group.transport_buffer(np.zeros(2 * len(blob), np.uint8)[::2])
    # a destination sharing memory with a source is refused before any write
    big = np.zeros(2 * len(blob), np.uint8)
    tr = big[-group.trellis.nbytes:].view(np.int16).reshape(group.trellis.shape)
    tr[...] = group.trellis
    aliased = Exl3Tensor(tr, group.suh, group.svh, group.bits, group.codebook, None, "x", "p")
    before = big.copy()
    with pytest.raises(ValueError, match="overlap"):
        aliased.transport_buffer(big)
    np.testing.assert_array_equal(big, before)


def test_padding_is_zeroed_and_big_endian_sources_are_converted():
    g = np.random.Generator(np.random.PCG64(5))
    tr = g.integers(-32768, 32768, (8, 8, 48), dtype=np.int16)
    suh = np.linspace(-1, 1, 128).astype(">f2")            # big endian source
    svh = np.linspace(1, 2, 128).astype(np.float16)
    bias = np.arange(128, dtype=">f4")
    group = Exl3Tensor(tr.astype(">i2"), suh, svh, 3.0, "mul1", bias, "mem", "p")
    buf = bytearray(b"\xff" * 40000)
    used, meta = group.transport_buffer(buf)
    blob, want = independent_blob(group)
    assert bytes(used) == blob and meta == want
    np.testing.assert_array_equal(np.frombuffer(blob, "<i2", tr.size, meta["trellis_offset"]).reshape(tr.shape), tr)


def test_half_rates_map_but_do_not_export(tmp_path):
    path = tmp_path / "w.safetensors"
    write_raw(path, group_tensors(bits=2.5, empty_marker=True))
    group = load_exl3(path, "proj")
    assert group.bits == 2.5 and group.codebook == "mul1"
    for export in (group.transport_blob, group.transport_buffer, group.transport_regions):
        with pytest.raises(ValueError, match="integer bitrates"):
            export()
    write_raw(path, group_tensors(bits=2.5, marker="mcg"))
    with pytest.raises(ValueError, match="Half-integer"):
        load_exl3(path, "proj")


def test_corrupt_containers_and_ambiguous_groups_are_rejected(tmp_path):
    path = tmp_path / "w.safetensors"
    corrupt = [
        lambda h: h["proj.trellis"].update(data_offsets=[0, 99999999]),
        lambda h: h["proj.trellis"].update(shape=[True, 16, 48]),
        lambda h: h["proj.trellis"].update(shape=[7, 16, 48]),
        lambda h: h["proj.trellis"].update(dtype="F16"),
        lambda h: h["proj.svh"].update(data_offsets=h["proj.suh"]["data_offsets"]),
        lambda h: h.pop("proj.svh"),
    ]
    for mutate in corrupt:
        write_raw(path, group_tensors(), mutate)
        with pytest.raises(ValueError):
            load_exl3(path, "proj")
    cases = [
        ({"proj.mcg": np.array(0, np.int32)}, "Simultaneous"),
        ({"proj.mul1": np.array(1, np.int32)}, "marker"),
        ({"proj.out_scales": np.ones(256, np.float16)}, "scale contract"),
    ]
    for extra, msg in cases:
        write_raw(path, {**group_tensors(), **extra})
        with pytest.raises(ValueError, match=msg):
            load_exl3(path, "proj")
    src = group_tensors()
    src["proj.suh"] = src["proj.suh"].copy()
    src["proj.suh"][4] = np.nan
    write_raw(path, src)
    with pytest.raises(ValueError, match="scale"):
        load_exl3(path, "proj")
    src = group_tensors()
    src["proj.bias"] = np.full(256, np.inf, np.float32)
    write_raw(path, src)
    with pytest.raises(ValueError, match="bias"):
        load_exl3(path, "proj")
    with pytest.raises(ValueError):
        load_exl3(path, "")
    path.write_bytes(b"bad")
    with pytest.raises(ValueError):
        SafetensorsFile(path)
    dup = b'{"x":{},"x":{}}'
    path.write_bytes(struct.pack("<Q", len(dup)) + dup)
    with pytest.raises(ValueError, match="Duplicate"):
        SafetensorsFile(path)
    path.write_bytes(struct.pack("<Q", 1 << 40) + b"{}")
    with pytest.raises(ValueError, match="oversized"):
        SafetensorsFile(path)


def test_unquantized_tensors(tmp_path):
    path = tmp_path / "w.safetensors"
    bf16 = (np.array([1.5, -2.25, 3.0e38], np.float32).view(np.uint32) >> 16).astype(np.uint16)
    write_raw(path, {"norm": bf16, "emb": np.array([0.5, -1.0], np.float16)})
    f = SafetensorsFile(path)
    with pytest.raises(ValueError):
        f.tensor("norm")
    np.testing.assert_array_equal(f.tensor("norm", raw_bf16=True), bf16)
    np.testing.assert_array_equal(f.tensor_float32("norm"), (bf16.astype(np.uint32) << 16).view(np.float32))
    np.testing.assert_array_equal(f.tensor_float32("emb"), np.array([0.5, -1.0], np.float32))
    with pytest.raises(ValueError):
        f.tensor("missing")


def test_legacy_signs_unpack_bit_b_of_word_j():
    # Sign 16 j + b is -1 where bit b of word j is set (reference
    # python/strix_trellis/linear.py:183-193), checked against a scalar
    # unpacking and on words whose bits are known.
    from strix_trellis import decode_legacy_signs
    rng = np.random.default_rng(5)
    words = rng.integers(0, 1 << 16, 37).astype(np.uint16)
    signs = decode_legacy_signs(words)
    assert signs.dtype == np.float16 and signs.shape == (37 * 16,)
    for j, word in enumerate(words):
        for b in range(16):
            assert signs[16 * j + b] == (-1.0 if (int(word) >> b) & 1 else 1.0)
    assert np.array_equal(decode_legacy_signs(words.view(np.int16)), signs)
    known = decode_legacy_signs(np.array([0x0001, 0x8000, 0xFFFF, 0], dtype=np.uint16))
    assert known[0] == -1 and (known[1:16] == 1).all()
    assert (known[16:31] == 1).all() and known[31] == -1
    assert (known[32:48] == -1).all() and (known[48:] == 1).all()
    for bad in (np.zeros((2, 2), np.uint16), np.zeros(4, np.uint32), np.zeros(4, np.float16)):
        with pytest.raises(ValueError, match="one-dimensional int16/uint16"):
            decode_legacy_signs(bad)
