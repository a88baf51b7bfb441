"""EXL3 tensor groups from local safetensors files, and their transport to the
native preparation functions.

The interface is the reference loader's (docs/LOADER.md; names
``SafetensorsFile``, ``Exl3Tensor``, ``load_exl3``, ``transport_regions`` /
``transport_buffer`` / ``transport_blob``, ``slice_outputs`` / ``slice_inputs``),
so loading code moves over unchanged; the product path is the HIP library, so a
group is ``prepare``d into device weights, and ``matmul(x, production=True)``
runs on the GPU (NumPy in and out, no torch) instead of on the CPU.

How it is organised here:

* ``_Catalog`` reads a file's header once (length prefix, JSON object with no
  duplicate keys) and resolves single tensors to read-only memory maps after
  checking their dtype, shape, byte range and size -- only the tensors asked
  for, never a whole shard;
* ``load_exl3`` picks one modern EXL3 group by the checks in ``_GROUP_CHECKS``
  order: member tensors, trellis geometry and rate, folded F16 scales, the
  codebook marker, the optional bias, disjoint payloads.  Anything the
  transport contract cannot carry is a ``ValueError``;
* ``_Transport`` lays a group out as the canonical transport (trellis I16,
  suh/svh F16, bias F32 at 4-byte aligned offsets, plus the
  ``strix_exl3_metadata_v1`` fields) without copying; the three exports read it;
* partitions cut H128-aligned column or channel ranges as views of the tiles.
"""
from dataclasses import dataclass
import json
import math
from pathlib import Path
import struct

import numpy as np

CODEBOOKS = ("3inst", "mcg", "mul1")                          # strix_exl3_codebook order
MARKERS = {"3inst": 0, "mcg": 0xCBAC1FED, "mul1": 0x83DCD12D}  # multiplier a numeric marker carries
TRANSPORT_VERSION = 1

_MAP_DTYPES = {"I16": "<i2", "I32": "<i4", "F16": "<f2", "F32": "<f4"}
_HEADER_LIMIT = 8_000_000
# Whole rates 1..8 bits, and the half rates the format defines for mul1 (the
# CPU reference reads them; GPU transport v1 carries whole rates only).
_WHOLE_RATES = frozenset(float(b) for b in range(1, 9))
_HALF_RATES = frozenset((1.5, 2.5, 3.5))


def _no_duplicate_keys(pairs):
    seen = {}
    for key, value in pairs:
        if key in seen:
            raise ValueError(f"Duplicate JSON key in safetensors header: {key}")
        seen[key] = value
    return seen


def _ints(value, count=None):
    return isinstance(value, list) and all(type(v) is int for v in value) and (count is None or len(value) == count)


@dataclass(frozen=True)
class _Entry:
    name: str
    dtype: np.dtype
    shape: tuple
    begin: int
    end: int


class _Catalog:
    """The parsed header of one safetensors file."""

    def __init__(self, path):
        self.path = Path(path)
        self.file_bytes = self.path.stat().st_size
        with self.path.open("rb") as f:
            prefix = f.read(8)
            if len(prefix) < 8:
                raise ValueError("Truncated safetensors file: no header length")
            (length,) = struct.unpack("<Q", prefix)
            if not 2 <= length <= min(_HEADER_LIMIT, self.file_bytes - 8):
                raise ValueError("Safetensors header length is invalid or oversized")
            text = f.read(length)
        try:
            header = json.loads(text, object_pairs_hook=_no_duplicate_keys)
        except json.JSONDecodeError as error:
            raise ValueError(f"Safetensors header is not valid JSON: {error}") from None
        if not isinstance(header, dict):
            raise ValueError("Safetensors header is not a JSON object")
        self.header = header
        self.data_offset = 8 + length

    def entry(self, name, raw_bf16=False):
        info = self.header.get(name)
        tag = info.get("dtype") if isinstance(info, dict) else None
        if tag in _MAP_DTYPES:
            dtype = np.dtype(_MAP_DTYPES[tag])
        elif tag == "BF16" and raw_bf16:
            dtype = np.dtype("<u2")   # raw bit patterns: BF16 has no NumPy type
        else:
            raise ValueError(f"Tensor {name} is missing or has an unsupported dtype")
        shape, offsets = info.get("shape"), info.get("data_offsets")
        if not (_ints(shape) and len(shape) <= 8 and min(shape, default=0) >= 0 and _ints(offsets, 2)):
            raise ValueError(f"Tensor {name} has an invalid shape or data_offsets")
        begin, end = offsets
        if not 0 <= begin <= end <= self.file_bytes - self.data_offset:
            raise ValueError(f"Tensor {name} lies outside the file")
        if math.prod(shape) * dtype.itemsize != end - begin:
            raise ValueError(f"Tensor {name} byte size does not match its shape and dtype")
        return _Entry(name, dtype, tuple(shape), begin, end)

    def map(self, e):
        if e.begin == e.end:
            out = np.empty(e.shape, dtype=e.dtype)
            out.flags.writeable = False
            return out
        return np.memmap(self.path, mode="r", dtype=e.dtype, offset=self.data_offset + e.begin, shape=e.shape)


class SafetensorsFile:
    """A local safetensors file: its header parsed and validated once; tensors
    mapped read-only on request.  Only tensors asked for are checked, so a
    shard may hold others this loader does not understand.  Keep the file
    unchanged while mapped arrays are alive."""

    def __init__(self, path):
        self._catalog = _Catalog(path)
        self.path = self._catalog.path
        self.header = self._catalog.header
        self.data_offset = self._catalog.data_offset
        self.file_bytes = self._catalog.file_bytes

    def tensor(self, name, *, raw_bf16=False):
        """Read-only map of one tensor (BF16 only with raw_bf16, as uint16 bit patterns)."""
        return self._catalog.map(self._catalog.entry(name, raw_bf16))

    def tensor_float32(self, name):
        """A BF16 / F16 / F32 tensor widened (exactly) into a float32 copy."""
        e = self._catalog.entry(name, raw_bf16=True)
        tag = self.header[name]["dtype"]
        if tag not in ("BF16", "F16", "F32"):
            raise ValueError(f"Tensor {name} is not a floating tensor")
        raw = self._catalog.map(e)
        if tag == "BF16":
            return (raw.astype(np.uint32) << 16).view(np.float32)
        return np.array(raw, dtype=np.float32)

    def exl3(self, prefix):
        return load_exl3(self, prefix)


# ----------------------------------------------------------------------------
# Transport layout
# ----------------------------------------------------------------------------
@dataclass(frozen=True)
class _Part:
    name: str
    values: np.ndarray
    dtype: np.dtype
    offset: int
    nbytes: int


class _Transport:
    """The canonical transport of a group: payloads in blob order at 4-byte
    aligned offsets and the strix_exl3_metadata_v1 fields; nothing is copied."""

    WIRE = (("trellis", np.dtype("<i2")), ("suh", np.dtype("<f2")), ("svh", np.dtype("<f2")),
            ("bias", np.dtype("<f4")))

    def __init__(self, t):
        if not float(t.bits).is_integer():
            raise ValueError("GPU transport v1 supports integer bitrates only")
        self.fields = {"transport_version": TRANSPORT_VERSION, "rows": t.output_size, "columns": t.input_size,
                       "bits_x2": 2 * int(t.bits), "codebook": CODEBOOKS.index(t.codebook),
                       "marker": MARKERS[t.codebook]}
        self.parts, end = [], 0
        for name, dtype in self.WIRE:
            values = getattr(t, name)
            if values is None:
                self.fields[f"{name}_offset"] = self.fields[f"{name}_bytes"] = 0
                continue
            values = np.asarray(values)
            offset = -(-end // 4) * 4
            part = _Part(name, values, dtype, offset, values.size * dtype.itemsize)
            self.fields[f"{name}_offset"], self.fields[f"{name}_bytes"] = part.offset, part.nbytes
            self.parts.append(part)
            end = part.offset + part.nbytes
        self.size = end

    def regions(self):
        views = {name: None for name, _ in self.WIRE}
        for p in self.parts:
            views[p.name] = memoryview(np.ascontiguousarray(p.values, dtype=p.dtype)).cast("B").toreadonly()
        return views

    def write(self, destination):
        """Pack into `destination` (a byte view of at least self.size)."""
        cursor = 0
        for p in self.parts:
            destination[cursor:p.offset] = bytes(p.offset - cursor)   # zero the alignment gap
            typed = np.ndarray(p.values.shape, dtype=p.dtype, buffer=destination, offset=p.offset)
            np.copyto(typed, p.values, casting="unsafe")
            cursor = p.offset + p.nbytes


def _writable_bytes(buffer):
    try:
        view = memoryview(buffer)
    except TypeError:
        raise ValueError("Destination must expose a writable, contiguous buffer") from None
    if view.readonly or not view.c_contiguous:
        raise ValueError("Destination must be writable and C-contiguous")
    return view.cast("B")


def _checked_cut(begin, end, limit, what):
    if type(begin) is not int or type(end) is not int or not 0 <= begin < end <= limit or begin % 128 or end % 128:
        raise ValueError(f"{what} partitions must be nonempty, in range and H128 aligned")


@dataclass(frozen=True)
class Exl3Tensor:
    """One folded-scale EXL3 linear; the logical Q is [input, output]."""
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
        """Output columns [begin, end), H128 aligned: the output transform is
        block diagonal over 128 columns, so each part keeps whole blocks.  The
        tile columns are a view; the trellis is packed only at export."""
        _checked_cut(begin, end, self.output_size, "Output")
        cols = slice(begin // 16, end // 16)
        bias = None if self.bias is None else self.bias[begin:end]
        return Exl3Tensor(self.trellis[:, cols, :], self.suh, self.svh[begin:end], self.bits, self.codebook, bias,
                          self.source, f"{self.prefix}[{begin}:{end}]")

    def slice_inputs(self, begin, end, *, include_bias):
        """Input channels [begin, end), H128 aligned, for a sum over parts:
        exactly one part of the sum carries the bias (an explicit bool); svh
        stays whole, every part producing all outputs."""
        _checked_cut(begin, end, self.input_size, "Input")
        if type(include_bias) is not bool:
            raise ValueError("include_bias must be an explicit bool")
        rows = slice(begin // 16, end // 16)
        return Exl3Tensor(self.trellis[rows], self.suh[begin:end], self.svh, self.bits, self.codebook,
                          self.bias if include_bias else None, self.source, f"{self.prefix}[K{begin}:{end}]")

    # ----------------------------------------------------------------- transport
    def transport_regions(self):
        """(name -> read-only byte view, or None for an absent bias; metadata fields).

        Contiguous little-endian payloads are borrowed (a mapped file stays
        mapped); only the others are packed.  The offsets in the fields are
        those of the equivalent blob; each view starts at its own payload.
        Keep the sources unchanged until native preparation returns."""
        layout = _Transport(self)
        return layout.regions(), layout.fields

    def transport_buffer(self, destination=None):
        """(buffer, metadata fields): the blob packed into one buffer.

        Without a destination, an exact-size bytearray.  A given writable,
        C-contiguous destination at least that large and sharing no memory with
        the sources receives the blob in its prefix (alignment gaps zeroed, the
        rest untouched); a memoryview of that prefix is returned."""
        layout = _Transport(self)
        if destination is None:
            out = bytearray(layout.size)
            layout.write(memoryview(out))
            return out, layout.fields
        view = _writable_bytes(destination)
        if view.nbytes < layout.size:
            raise ValueError("Destination is too small for the transport")
        target = np.frombuffer(view, dtype=np.uint8)
        if any(np.may_share_memory(target, p.values) for p in layout.parts):
            raise ValueError("Destination must not overlap the transport's source arrays")
        layout.write(view)
        return view[:layout.size], layout.fields

    def transport_blob(self):
        """(immutable bytes, metadata fields) for strix_weights_prepare."""
        packed, fields = self.transport_buffer()
        return bytes(packed), fields

    # ------------------------------------------------------------------ device
    def prepare(self, ctx, stream=None, *, blob=False):
        """Device weights (``runtime.Weights``) from the transport regions
        (strix_weights_prepare_parts) or, with blob=True, the blob
        (strix_weights_prepare).  The library copies the payloads, so the views
        and the mapped file may be released once this returns."""
        from . import runtime
        return runtime.Weights.from_transport(ctx, self, stream=stream, blob=blob)

    def matmul(self, x, *, production=False, context=None, stream=None):
        """y = this linear applied to x: [I] -> [N] or [rows, I] -> [rows, N]
        (reference python/strix_trellis/container.py:112-115).

        production=True runs the library: strix_gemv for 1-8 rows, strix_gemm
        above, on device weights prepared once per context and kept with this
        tensor (``context`` defaults to ``runtime.default_context()``).  x
        and the result are NumPy arrays (x is converted to float32); device
        memory and the stream (``stream``, else the context's own HIP stream)
        come from the HIP runtime through ``strix_trellis.device``, so no
        torch is needed.  The call returns when the result has been copied
        back.  The arithmetic is the staged FP32
        contract of the reference's production path (matmul_fp32): input and
        output stages bit-exact, the core within its FP64 tolerance.

        production=False, the reference's FP64 algebraic matmul, is a CPU
        mathematical reference; this library keeps it with its tests
        (oracle/linear.py) rather than in the package, and raises
        NotImplementedError."""
        if not production:
            raise NotImplementedError("the FP64 algebraic reference matmul is not part of this library; "
                                      "matmul(x, production=True) runs the GPU path")
        from . import device, runtime
        xa = np.asarray(x, dtype=np.float32)
        if xa.ndim not in (1, 2) or xa.shape[-1] != self.input_size:
            raise ValueError(f"x must be [{self.input_size}] or [rows, {self.input_size}]")
        rows = 1 if xa.ndim == 1 else xa.shape[0]
        if rows == 0:
            return np.zeros((0, self.output_size), np.float32)
        ctx = context if context is not None else runtime.default_context()
        s = stream if stream is not None else runtime.host_stream(ctx)
        cache = self.__dict__.setdefault("_prepared", {})
        if id(ctx) not in cache:
            cache[id(ctx)] = (ctx, self.prepare(ctx, s))
        weights = cache[id(ctx)][1]
        dx = device.DeviceArray.from_numpy(xa, device=ctx.device)
        dy = device.DeviceArray.empty(xa.shape[:-1] + (self.output_size,), np.float32, ctx.device)
        ws = device.DeviceArray.empty(runtime.workspace_bytes(weights, dx, dy), np.uint8, ctx.device)
        try:
            (runtime.gemv if rows <= 8 else runtime.gemm)(weights, dx, dy, workspace=ws, stream=s)
            s.synchronize()
            return dy.numpy()
        finally:
            for a in (dx, dy, ws):
                a.free()


# ----------------------------------------------------------------------------
# Group selection
# ----------------------------------------------------------------------------
class _Group:
    """The tensors of one group as they are picked, with their byte ranges."""

    def __init__(self, catalog, prefix):
        self.catalog, self.prefix, self.picked = catalog, prefix, []

    def has(self, suffix):
        return self.prefix + suffix in self.catalog.header

    def take(self, suffix):
        e = self.catalog.entry(self.prefix + suffix)
        self.picked.append(e)
        return self.catalog.map(e)


def _geometry(trellis):
    if trellis.dtype != np.dtype("<i2") or trellis.ndim != 3 or 0 in trellis.shape:
        raise ValueError("EXL3 trellis must be a nonempty I16 array [I/16, O/16, words]")
    bits = trellis.shape[2] / 16
    if bits not in _WHOLE_RATES | _HALF_RATES:
        raise ValueError(f"Unsupported EXL3 bitrate: {bits}")
    inputs, outputs = 16 * trellis.shape[0], 16 * trellis.shape[1]
    if inputs % 128 or outputs % 128:
        raise ValueError("A complete EXL3 linear needs input and output sizes that are multiples of 128")
    return inputs, outputs, bits


def _folded_scale(values, size, name):
    if values.dtype != np.dtype("<f2") or values.shape != (size,) or not np.isfinite(values).all():
        raise ValueError(f"Invalid folded F16 scale vector {name}")


def _codebook(group):
    named = [cb for cb in ("mul1", "mcg") if group.has("." + cb)]
    if len(named) > 1:
        raise ValueError("Simultaneous mul1 and mcg markers")
    if not named:
        return "3inst"
    marker = group.take("." + named[0])
    # Empty: the historical marker; numeric: one I32 that carries the multiplier.
    numeric_ok = marker.dtype == np.dtype("<i4") and marker.size == 1 and \
        int(marker.reshape(-1)[0]) & 0xFFFFFFFF == MARKERS[named[0]]
    if marker.size and not numeric_ok:
        raise ValueError("Unsupported EXL3 codebook marker")
    return named[0]


def _bias(group, outputs):
    if not group.has(".bias"):
        return None
    raw = group.take(".bias")
    if raw.dtype.kind != "f" or raw.shape != (outputs,) or not np.isfinite(raw).all():
        raise ValueError("Invalid bias vector")
    bias = raw.astype(np.float32, copy=False)   # F32 stays mapped, F16 widens once
    bias.flags.writeable = False
    return bias


def _disjoint(group):
    ranges = sorted((e.begin, e.end) for e in group.picked if e.end > e.begin)
    if any(prev[1] > cur[0] for prev, cur in zip(ranges, ranges[1:])):
        raise ValueError("Selected EXL3 tensors overlap in the file")


def load_exl3(file, prefix):
    """Map and validate the EXL3 group ``prefix`` of a path or SafetensorsFile."""
    sf = file if isinstance(file, SafetensorsFile) else SafetensorsFile(file)
    if not isinstance(prefix, str) or not prefix:
        raise ValueError("A nonempty tensor prefix is required")
    group = _Group(sf._catalog, prefix)
    if group.has(".out_scales"):
        raise ValueError("External out_scales need an explicit scale contract; not supported")
    trellis, suh, svh = group.take(".trellis"), group.take(".suh"), group.take(".svh")
    inputs, outputs, bits = _geometry(trellis)
    _folded_scale(suh, inputs, "suh")
    _folded_scale(svh, outputs, "svh")
    codebook = _codebook(group)
    if bits in _HALF_RATES and codebook != "mul1":
        raise ValueError("Half-integer EXL3 rates require the mul1 codebook")
    bias = _bias(group, outputs)
    _disjoint(group)
    return Exl3Tensor(trellis, suh, svh, bits, codebook, bias, str(sf.path), prefix)


def decode_legacy_signs(packed):
    """FP16 +-1 signs of a legacy packed su/sv vector (one-dimensional 16-bit
    words): sign 16 j + b is -1 where bit b of word j is set, else +1
    (reference python/strix_trellis/linear.py:183-193).  Such groups carry no
    scale contract, so ``load_exl3`` rejects them; this only unpacks the bits."""
    words = np.asarray(packed)
    if words.ndim != 1 or words.dtype.kind not in "iu" or words.dtype.itemsize != 2:
        raise ValueError("Legacy signs require a one-dimensional int16/uint16 array")
    bits = np.unpackbits(words.astype("<u2").view(np.uint8), bitorder="little")
    return (1 - 2 * bits.astype(np.int8)).astype(np.float16)
