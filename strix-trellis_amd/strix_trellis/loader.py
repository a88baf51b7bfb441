"""EXL3 tensor groups from local safetensors files, and their transport to the
native preparation functions.

Same interface as the reference loader (python/strix_trellis/container.py:
``SafetensorsFile`` :30-95, ``Exl3Tensor`` :98-240, ``load_exl3`` :243-288;
docs/LOADER.md), so a caller of the reference can switch to this package:

* a ``SafetensorsFile`` parses and validates the header once and maps only the
  tensors asked for (read-only ``np.memmap``), never a whole shard;
* ``load_exl3(file, prefix)`` selects one modern EXL3 group -- trellis I16
  ``[I/16, N/16, 16 K]``, folded F16 ``suh[I]`` / ``svh[N]``, an optional mul1 or
  mcg marker, an optional F16/F32 bias -- and rejects what the transport
  contract cannot carry (external out_scales, simultaneous or unknown
  markers, non-finite scales, overlapping payloads), raising ``ValueError``;
* an ``Exl3Tensor`` exports the canonical transport -- four little-endian
  payloads at 4-byte aligned offsets plus the ``strix_exl3_metadata_v1``
  fields -- as borrowed regions, as one caller-owned buffer, or as an immutable
  blob, and slices H128-aligned output or input partitions without expanding Q.

One difference: the reference's ``Exl3Tensor.matmul`` is its CPU reference.
Here the product path is the HIP library, so a group is instead ``prepare``d
into device weights (``runtime.Weights``) and multiplied there.
"""
from dataclasses import dataclass
import json
import math
from pathlib import Path
import struct

import numpy as np

# safetensors dtype tags this loader maps; BF16 has no NumPy type and is only
# mapped as its raw little-endian 16-bit patterns on request.
_DTYPES = {"I16": np.dtype("<i2"), "I32": np.dtype("<i4"), "F16": np.dtype("<f2"), "F32": np.dtype("<f4")}
_RAW_BF16 = np.dtype("<u2")
_MAX_HEADER = 8_000_000

# Codebooks: enum order of strix_exl3_codebook and the multiplier each numeric
# marker must carry (3inst has no marker).
CODEBOOKS = ("3inst", "mcg", "mul1")
MARKERS = {"3inst": 0, "mcg": 0xCBAC1FED, "mul1": 0x83DCD12D}
TRANSPORT_VERSION = 1
# Transport payloads in blob order with their wire dtypes.
_PAYLOADS = (("trellis", np.dtype("<i2")), ("suh", np.dtype("<f2")), ("svh", np.dtype("<f2")),
             ("bias", np.dtype("<f4")))
# Rates the EXL3 format defines: whole bits 1..8, and 1.5 / 2.5 / 3.5 for mul1
# (CPU only; GPU transport v1 carries whole rates).
_RATES = {float(k) for k in range(1, 9)} | {1.5, 2.5, 3.5}


def _object_without_duplicates(pairs):
    out = {}
    for key, value in pairs:
        if key in out:
            raise ValueError(f"Duplicate JSON key: {key}")
        out[key] = value
    return out


def _int_list(value, length=None):
    return (isinstance(value, list) and (length is None or len(value) == length) and
            all(type(v) is int for v in value))


class SafetensorsFile:
    """Header of a local safetensors file; tensors are mapped on request.

    Only the tensors asked for are validated (range, dtype, element count);
    unrelated tensors of a multi-format shard need not be understood.  Keep
    the file unchanged while mapped arrays are alive.
    """

    def __init__(self, path):
        self.path = Path(path)
        self.file_bytes = self.path.stat().st_size
        with self.path.open("rb") as f:
            head = f.read(8)
            if len(head) != 8:
                raise ValueError("Truncated safetensors header length")
            (n,) = struct.unpack("<Q", head)
            if n < 2 or n > min(_MAX_HEADER, self.file_bytes - 8):
                raise ValueError("Invalid or oversized safetensors header")
            text = f.read(n)
        try:
            header = json.loads(text, object_pairs_hook=_object_without_duplicates)
        except json.JSONDecodeError as e:
            raise ValueError(f"Invalid safetensors header JSON: {e}") from None
        if not isinstance(header, dict):
            raise ValueError("Safetensors header must be an object")
        self.header = header
        self.data_offset = 8 + n

    def tensor(self, name, *, raw_bf16=False):
        """Read-only map of one tensor (BF16 only with raw_bf16: uint16 bit patterns)."""
        info = self.header.get(name)
        tag = info.get("dtype") if isinstance(info, dict) else None
        if tag in _DTYPES:
            dtype = _DTYPES[tag]
        elif tag == "BF16" and raw_bf16:
            dtype = _RAW_BF16
        else:
            raise ValueError(f"Missing tensor or unsupported dtype: {name}")
        shape, offsets = info.get("shape"), info.get("data_offsets")
        if not _int_list(shape) or len(shape) > 8 or any(v < 0 for v in shape) or not _int_list(offsets, 2):
            raise ValueError(f"Invalid tensor shape or offsets: {name}")
        begin, end = offsets
        if not 0 <= begin <= end <= self.file_bytes - self.data_offset:
            raise ValueError(f"Tensor range exceeds file: {name}")
        if math.prod(shape) * dtype.itemsize != end - begin:
            raise ValueError(f"Tensor size does not match shape/dtype: {name}")
        if begin == end:
            empty = np.empty(shape, dtype=dtype)
            empty.flags.writeable = False
            return empty
        return np.memmap(self.path, mode="r", dtype=dtype, offset=self.data_offset + begin, shape=tuple(shape))

    def tensor_float32(self, name):
        """An unquantized BF16 / F16 / F32 tensor widened (exactly) to a float32 copy."""
        info = self.header.get(name)
        tag = info.get("dtype") if isinstance(info, dict) else None
        if tag not in ("BF16", "F16", "F32"):
            raise ValueError(f"Not a floating tensor: {name}")
        raw = self.tensor(name, raw_bf16=True)
        if tag == "BF16":
            return (raw.astype(np.uint32) << 16).view(np.float32)
        return np.asarray(raw, dtype=np.float32).copy()

    def exl3(self, prefix):
        return load_exl3(self, prefix)


@dataclass(frozen=True)
class Exl3Tensor:
    """One folded-scale EXL3 linear: logical Q is [input, output]."""
    trellis: np.ndarray      # int16 [I/16, N/16, 16 * bits]
    suh: np.ndarray          # float16 [I]
    svh: np.ndarray          # float16 [N]
    bits: float
    codebook: str
    bias: np.ndarray | None  # float32 [N] or None
    source: str
    prefix: str

    @property
    def input_size(self):
        return self.trellis.shape[0] * 16

    @property
    def output_size(self):
        return self.trellis.shape[1] * 16

    # ---------------------------------------------------------------- partitions
    def slice_outputs(self, begin, end):
        """H128-aligned output partition [begin, end): a view of its tile columns.

        The output transform is block-diagonal over 128 columns, so each part
        keeps complete H128 blocks; its trellis is repacked at export only.
        """
        if type(begin) is not int or type(end) is not int or not 0 <= begin < end <= self.output_size \
                or begin % 128 or end % 128:
            raise ValueError("Output partitions must be nonempty, in range and H128 aligned")
        return Exl3Tensor(self.trellis[:, begin // 16:end // 16, :], self.suh, self.svh[begin:end], self.bits,
                          self.codebook, None if self.bias is None else self.bias[begin:end], self.source,
                          f"{self.prefix}[{begin}:{end}]")

    def slice_inputs(self, begin, end, *, include_bias):
        """H128-aligned input partition [begin, end) for a K-split sum over parts.

        Exactly one part of a sum may carry the bias, so the choice is an
        explicit bool.  svh stays whole (every part produces all outputs).
        """
        if type(begin) is not int or type(end) is not int or not 0 <= begin < end <= self.input_size \
                or begin % 128 or end % 128:
            raise ValueError("Input partitions must be nonempty, in range and H128 aligned")
        if type(include_bias) is not bool:
            raise ValueError("include_bias must be an explicit bool")
        return Exl3Tensor(self.trellis[begin // 16:end // 16], self.suh[begin:end], self.svh, self.bits,
                          self.codebook, self.bias if include_bias else None, self.source,
                          f"{self.prefix}[K{begin}:{end}]")

    # ----------------------------------------------------------------- transport
    def _layout(self):
        """Payloads, strix_exl3_metadata_v1 fields and blob size; copies nothing."""
        if not float(self.bits).is_integer():
            raise ValueError("GPU transport v1 supports integer bitrates only")
        meta = {"rows": self.output_size, "columns": self.input_size, "bits_x2": int(self.bits) * 2,
                "codebook": CODEBOOKS.index(self.codebook), "marker": MARKERS[self.codebook],
                "transport_version": TRANSPORT_VERSION}
        payloads, pos = [], 0
        for name, dtype in _PAYLOADS:
            values = getattr(self, name)
            if values is None:
                meta[name + "_offset"] = meta[name + "_bytes"] = 0
                continue
            values = np.asarray(values)
            pos = (pos + 3) & ~3
            meta[name + "_offset"], meta[name + "_bytes"] = pos, values.size * dtype.itemsize
            pos += values.size * dtype.itemsize
            payloads.append((name, values, dtype))
        return payloads, meta, pos

    def transport_regions(self):
        """(name -> read-only byte view or None, metadata fields).

        A payload that is already contiguous little-endian is borrowed (a
        mapped file stays mapped); only others (e.g. the strided trellis of an
        output slice) are packed.  Offsets in the fields describe the
        equivalent blob; each view starts at its own payload.  The sources
        must stay unchanged until native preparation returns.
        """
        payloads, meta, _ = self._layout()
        regions = {name: None for name, _ in _PAYLOADS}
        for name, values, dtype in payloads:
            regions[name] = memoryview(np.ascontiguousarray(values, dtype=dtype)).cast("B").toreadonly()
        return regions, meta

    def transport_buffer(self, destination=None):
        """(buffer, metadata fields): the blob written into one buffer.

        With no destination a bytearray of the exact size is returned; a
        given writable C-contiguous buffer (at least that large, not sharing
        memory with any source) receives the blob in its prefix and a
        memoryview of that prefix is returned, the rest left untouched.
        Alignment gaps are zeroed; each payload is copied once, straight into
        its typed place.
        """
        payloads, meta, size = self._layout()
        owned = destination is None
        buf = bytearray(size) if owned else destination
        try:
            view = memoryview(buf)
        except TypeError:
            raise ValueError("Destination must expose a writable contiguous buffer") from None
        if view.readonly or not view.c_contiguous:
            raise ValueError("Destination must be writable and C-contiguous")
        view = view.cast("B")
        if view.nbytes < size:
            raise ValueError("Destination is too small for the transport")
        if not owned:
            target = np.frombuffer(view, dtype=np.uint8)
            if any(np.may_share_memory(target, values) for _, values, _ in payloads):
                raise ValueError("Destination must not overlap transport source arrays")
        pos = 0
        for name, values, dtype in payloads:
            offset = meta[name + "_offset"]
            view[pos:offset] = bytes(offset - pos)
            np.copyto(np.ndarray(values.shape, dtype=dtype, buffer=view, offset=offset), values, casting="unsafe")
            pos = offset + meta[name + "_bytes"]
        return (buf if owned else view[:size]), meta

    def transport_blob(self):
        """(immutable bytes, metadata fields) for strix_weights_prepare."""
        buf, meta = self.transport_buffer()
        return bytes(buf), meta

    # ------------------------------------------------------------------ device
    def prepare(self, ctx, stream=None, *, blob=False):
        """Device weights (``runtime.Weights``) from the transport regions
        (strix_weights_prepare_parts) or, with blob=True, from the blob
        (strix_weights_prepare).  The library copies the payloads; the views
        and mapped file may be released once this returns."""
        from . import runtime
        return runtime.Weights.from_transport(ctx, self, stream=stream, blob=blob)


def load_exl3(file, prefix):
    """Map and validate the EXL3 group `prefix` of a path or SafetensorsFile."""
    f = file if isinstance(file, SafetensorsFile) else SafetensorsFile(file)
    if not isinstance(prefix, str) or not prefix:
        raise ValueError("A nonempty tensor prefix is required")
    if prefix + ".out_scales" in f.header:
        raise ValueError("External out_scales requires an explicit scale contract")
    selected = {}

    def take(suffix):
        name = prefix + suffix
        selected[name] = f.tensor(name)
        return selected[name]

    trellis, suh, svh = take(".trellis"), take(".suh"), take(".svh")
    if trellis.dtype != np.dtype("<i2") or trellis.ndim != 3 or 0 in trellis.shape:
        raise ValueError("EXL3 trellis must be nonempty I16 [I/16,O/16,words]")
    bits = trellis.shape[2] / 16
    if bits not in _RATES:
        raise ValueError(f"Unsupported EXL3 bitrate: {bits}")
    inputs, outputs = trellis.shape[0] * 16, trellis.shape[1] * 16
    if inputs % 128 or outputs % 128:
        raise ValueError("Complete EXL3 linear requires I/O multiples of 128")
    for name, values, size in (("suh", suh, inputs), ("svh", svh, outputs)):
        if values.dtype != np.dtype("<f2") or values.shape != (size,) or not np.isfinite(values).all():
            raise ValueError(f"Invalid folded F16 scale vector: {name}")
    present = [cb for cb in ("mul1", "mcg") if f"{prefix}.{cb}" in f.header]
    if len(present) > 1:
        raise ValueError("Simultaneous mul1/mcg markers")
    codebook = present[0] if present else "3inst"
    if present:
        marker = take("." + codebook)
        # An empty marker is the historical form; a numeric one must carry the multiplier.
        if marker.size and (marker.dtype != np.dtype("<i4") or marker.size != 1 or
                            int(marker.reshape(-1)[0]) & 0xFFFFFFFF != MARKERS[codebook]):
            raise ValueError("Unsupported EXL3 codebook marker")
    if not bits.is_integer() and codebook != "mul1":
        raise ValueError("Half-integer EXL3 rates require mul1")
    bias = None
    if prefix + ".bias" in f.header:
        raw = take(".bias")
        if raw.dtype.kind != "f" or raw.shape != (outputs,) or not np.isfinite(raw).all():
            raise ValueError("Invalid bias vector")
        bias = raw.astype(np.float32, copy=False)   # F32 stays mapped, F16 widens once
        bias.flags.writeable = False
    spans = sorted(tuple(f.header[name]["data_offsets"]) for name, arr in selected.items() if arr.nbytes)
    if any(a[1] > b[0] for a, b in zip(spans, spans[1:])):
        raise ValueError("Overlapping selected EXL3 tensor ranges")
    return Exl3Tensor(trellis, suh, svh, bits, codebook, bias, str(f.path), prefix)
