"""Python host layer over the C ABI (ctypes): contexts, prepared weights, calls, plans.

Device buffers are PyTorch-ROCm tensors or :class:`device.DeviceArray`
(memory from the HIP runtime itself, for hosts without PyTorch); streams are
torch streams or :class:`device.Stream`.  Either only supplies device memory
and streams: every computation runs in libstrix_trellis.so.  torch is
imported only when a torch tensor or stream is handed in (or, for the default
stream, when the caller has imported it).  Errors surface as
:class:`abi.StrixError` carrying the C status.
"""
import ctypes as C
import sys

import numpy as np

from . import abi
from . import device as _hipdev

_torch = None


def _t():
    global _torch
    if _torch is None:
        import torch
        _torch = torch
    return _torch


def _is_torch(obj):
    return type(obj).__module__.split(".")[0] == "torch"


def stream_desc(stream=None):
    """strix_stream for a torch or HIP stream.  None: torch's current stream
    when the caller has imported torch, else the device's default (NULL)
    stream."""
    if stream is None:
        torch = sys.modules.get("torch")
        if torch is None:
            return abi.header(abi.Stream, hip_stream=C.c_void_p(None))
        stream = torch.cuda.current_stream()
    return abi.header(abi.Stream, hip_stream=C.c_void_p(stream.cuda_stream or None))


def _is_f32(t):
    return t.dtype == (_t().float32 if _is_torch(t) else np.float32)


def tensor_desc(t, rank=None, width=None):
    """F32 tensor descriptor of a contiguous torch tensor or DeviceArray (rank 1 or 2)."""
    d = abi.header(abi.TensorDesc)
    d.dtype = abi.DTYPE_F32
    if t is None:
        d.rank = rank or 2
        d.shape[0] = 0
        d.shape[1] = width or 0
        d.strides[0] = width or 0
        d.strides[1] = 1
        return d
    if not _is_f32(t) or not t.is_contiguous():
        raise ValueError("tensors must be contiguous float32")
    d.data = C.c_void_p(t.data_ptr() or None)
    d.buffer_bytes = t.numel() * 4
    d.rank = t.dim() if rank is None else rank
    if d.rank == 1:
        d.shape[0] = t.shape[0]
        d.strides[0] = 1
    else:
        d.shape[0], d.shape[1] = t.shape[0], t.shape[1]
        d.strides[0], d.strides[1] = t.shape[1], 1
    return d


class Context:
    def __init__(self, device=0):
        self.lib = abi.load()
        desc = abi.header(abi.ContextDesc, device_ordinal=device)
        h = C.c_void_p()
        abi.check(self.lib.strix_context_create(C.byref(desc), C.byref(h)), "strix_context_create")
        self.handle = h
        self.device = device

    def set_gemv_poll_limit(self, limit=abi.GEMV_POLL_DEFAULT):
        """Poll rounds of single-launch GEMV finishers on later submissions (0: give up at once)."""
        abi.check(self.lib.strix_amd_set_gemv_poll_limit(self.handle, int(limit)), "strix_amd_set_gemv_poll_limit")

    def set_plan_state_reuse(self, enable=True):
        """Let plans created later take a destroyed plan's single-launch state (off by default)."""
        abi.check(self.lib.strix_amd_set_plan_state_reuse(self.handle, int(bool(enable))),
                  "strix_amd_set_plan_state_reuse")

    def set_grouped_fold(self, fold=abi.FOLD_AUTO):
        """Fold of grouped plans created later: FOLD_AUTO, FOLD_SPLIT or FOLD_OWNER."""
        abi.check(self.lib.strix_amd_set_grouped_fold(self.handle, int(fold)), "strix_amd_set_grouped_fold")

    def close(self):
        if self.handle:
            abi.check(self.lib.strix_context_destroy(self.handle), "strix_context_destroy")
            self.handle = None


_DEFAULT_CONTEXTS = {}


def default_context(device=0):
    """A library context on `device`, created on first use and kept for the
    process (used by ``loader.Exl3Tensor.matmul``)."""
    if device not in _DEFAULT_CONTEXTS:
        _DEFAULT_CONTEXTS[device] = Context(device)
    return _DEFAULT_CONTEXTS[device]


_HOST_STREAMS = {}


def host_stream(ctx):
    """A HIP stream of the context's device for NumPy-level calls
    (``loader.Exl3Tensor.matmul``), created on first use."""
    if id(ctx) not in _HOST_STREAMS:
        _HOST_STREAMS[id(ctx)] = (ctx, _hipdev.Stream(ctx.device))
    return _HOST_STREAMS[id(ctx)][1]


class Weights:
    """Prepared EXL3 weights (one private device allocation)."""

    def __init__(self, ctx, trellis, suh, svh, bias=None, codebook="mul1", stream=None, blob=False):
        self.ctx, self.lib = ctx, ctx.lib
        tr = np.ascontiguousarray(trellis)
        if tr.ndim != 3 or tr.dtype.itemsize != 2:
            raise ValueError("trellis must be [I/16, N/16, 16K] 16-bit words")
        self.input, self.output = tr.shape[0] * 16, tr.shape[1] * 16
        self.bits = tr.shape[2] // 16
        self.codebook = codebook
        self._keep = [tr.view(np.uint16), np.ascontiguousarray(suh, dtype=np.float16),
                      np.ascontiguousarray(svh, dtype=np.float16),
                      None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)]
        h = C.c_void_p()
        sd = stream_desc(stream)
        if blob:
            status = self._prepare_blob(sd, h)
        else:
            parts = abi.header(abi.PartsDesc, transport_version=abi.TRANSPORT_VERSION, bits_x2=2 * self.bits,
                               rows=self.output, columns=self.input, codebook=abi.CODEBOOK[codebook],
                               marker=abi.MARKER[codebook])
            for name, arr in zip(("trellis", "suh", "svh", "bias"), self._keep):
                if arr is not None:
                    setattr(parts, name, abi.HostRegion(arr.ctypes.data, arr.nbytes))
            status = self.lib.strix_weights_prepare_parts(ctx.handle, C.byref(parts), C.byref(sd), C.byref(h))
        abi.check(status, "strix_weights_prepare")
        self.handle = h

    def _prepare_blob(self, sd, h):
        tr, suh, svh, bias = self._keep
        chunks, offsets, pos = [], [], 0
        for arr in (tr, suh, svh, bias):
            if arr is None:
                offsets.append((0, 0))
                continue
            pos = (pos + 3) & ~3
            offsets.append((pos, arr.nbytes))
            chunks.append((pos, arr))
            pos += arr.nbytes
        blob = np.zeros(pos, dtype=np.uint8)
        for off, arr in chunks:
            blob[off:off + arr.nbytes] = arr.view(np.uint8).reshape(-1)
        m = abi.Metadata(struct_size=C.sizeof(abi.Metadata), transport_version=abi.TRANSPORT_VERSION,
                         rows=self.output, columns=self.input, bits_x2=2 * self.bits,
                         codebook=abi.CODEBOOK[self.codebook], marker=abi.MARKER[self.codebook])
        (m.trellis_offset, m.trellis_bytes), (m.suh_offset, m.suh_bytes), (m.svh_offset, m.svh_bytes), \
            (m.bias_offset, m.bias_bytes) = offsets
        t = abi.header(abi.TransportDesc, format=abi.TRANSPORT_EXL3_CANONICAL,
                       transport_version=abi.TRANSPORT_VERSION, data=blob.ctypes.data, data_bytes=blob.nbytes,
                       metadata=C.addressof(m), metadata_bytes=C.sizeof(m), rows=self.output, columns=self.input)
        self._blob, self._meta = blob, m
        return self.lib.strix_weights_prepare(self.ctx.handle, C.byref(t), C.byref(sd), C.byref(h))

    @classmethod
    def from_transport(cls, ctx, group, stream=None, blob=False):
        """Weights prepared from an EXL3 group's canonical transport (a
        ``loader.Exl3Tensor``): its borrowed regions through
        strix_weights_prepare_parts, or with blob=True its blob through
        strix_weights_prepare.  Preparation copies and synchronises, so the
        host views may go once this returns."""
        self = cls.__new__(cls)
        self.ctx, self.lib = ctx, ctx.lib
        h = C.c_void_p()
        sd = stream_desc(stream)
        if blob:
            data, meta = group.transport_blob()
            raw = np.frombuffer(data, dtype=np.uint8)
            m = abi.Metadata(struct_size=C.sizeof(abi.Metadata), **meta)
            t = abi.header(abi.TransportDesc, format=abi.TRANSPORT_EXL3_CANONICAL,
                           transport_version=meta["transport_version"], data=raw.ctypes.data, data_bytes=raw.nbytes,
                           metadata=C.addressof(m), metadata_bytes=C.sizeof(m), rows=meta["rows"],
                           columns=meta["columns"])
            status = self.lib.strix_weights_prepare(ctx.handle, C.byref(t), C.byref(sd), C.byref(h))
        else:
            regions, meta = group.transport_regions()
            parts = abi.header(abi.PartsDesc, transport_version=meta["transport_version"], bits_x2=meta["bits_x2"],
                               rows=meta["rows"], columns=meta["columns"], codebook=meta["codebook"],
                               marker=meta["marker"])
            views = []
            for name, view in regions.items():
                if view is not None:
                    arr = np.frombuffer(view, dtype=np.uint8)
                    views.append(arr)
                    setattr(parts, name, abi.HostRegion(arr.ctypes.data, arr.nbytes))
            status = self.lib.strix_weights_prepare_parts(ctx.handle, C.byref(parts), C.byref(sd), C.byref(h))
        abi.check(status, "strix_weights_prepare")
        self.handle = h
        self.input, self.output = meta["columns"], meta["rows"]
        self.bits = meta["bits_x2"] // 2
        self.codebook = group.codebook
        self._keep = []
        return self

    @property
    def packed_bytes(self):
        return self.input * self.output * self.bits // 8

    def destroy(self):
        if self.handle:
            abi.check(self.lib.strix_weights_destroy(self.handle), "strix_weights_destroy")
            self.handle = None

    def gemv_shape(self):
        bps, splits = C.c_uint32(), C.c_uint32()
        abi.check(self.lib.strix_amd_gemv_shape(self.handle, C.byref(bps), C.byref(splits)))
        return bps.value, splits.value

    def gemm_splits(self, rows):
        """K splits of a GEMM call of `rows` rows (calls with equal counts share row bits)."""
        splits = C.c_uint32()
        abi.check(self.lib.strix_amd_gemm_splits(self.handle, C.c_uint64(rows), C.byref(splits)))
        return splits.value

    # -- diagnostics -----------------------------------------------------------
    def decode(self, stream=None):
        torch = _t()
        q = torch.empty((self.input, self.output), dtype=torch.float16, device=f"cuda:{self.ctx.device}")
        abi.check(self.lib.strix_amd_decode(self.handle, C.c_void_p(q.data_ptr()), q.numel() * 2,
                                            C.byref(stream_desc(stream))), "strix_amd_decode")
        return q

    def input_stage(self, x, stream=None):
        torch = _t()
        x = x.reshape(-1, self.input)
        a = torch.empty(x.shape, dtype=torch.float16, device=x.device)
        abi.check(self.lib.strix_amd_input_stage(self.handle, C.c_void_p(x.data_ptr() or None), x.shape[0],
                                                 C.c_void_p(a.data_ptr() or None), a.numel() * 2,
                                                 C.byref(stream_desc(stream))), "strix_amd_input_stage")
        return a

    def output_stage(self, core, y=None, alpha=1.0, beta=0.0, stream=None):
        torch = _t()
        core = core.reshape(-1, self.output)
        if y is None:
            y = torch.empty(core.shape, dtype=torch.float32, device=core.device)
        abi.check(self.lib.strix_amd_output_stage(self.handle, C.c_void_p(core.data_ptr() or None), core.shape[0],
                                                  C.c_void_p(y.data_ptr() or None), y.numel() * 4, alpha, beta,
                                                  C.byref(stream_desc(stream))), "strix_amd_output_stage")
        return y


def matmul_desc(weights, x, y, alpha=1.0, beta=0.0, workspace=None, rank=None):
    d = abi.MatmulDesc()
    weights.lib.strix_matmul_desc_init(C.byref(d))
    d.weights = weights.handle
    d.input = tensor_desc(x, rank, weights.input)
    d.output = tensor_desc(y, rank, weights.output)
    d.alpha, d.beta = alpha, beta
    if workspace is not None:
        d.workspace = C.c_void_p(workspace.data_ptr() or None)
        d.workspace_bytes = workspace.numel() * workspace.element_size()
    return d


def workspace_bytes(weights, x, y, rank=None):
    d = matmul_desc(weights, x, y, rank=rank)
    out = C.c_uint64()
    abi.check(weights.lib.strix_matmul_workspace_bytes(weights.ctx.handle, C.byref(d), C.byref(out)),
              "strix_matmul_workspace_bytes")
    return out.value


def alloc_workspace(nbytes, device, like=None):
    """A workspace of at least `nbytes` bytes: a torch tensor on `device`, or a
    DeviceArray when `like` is one (both at least 256-byte aligned)."""
    if like is not None and not _is_torch(like):
        return _hipdev.DeviceArray.empty(max(int(nbytes), 256), np.uint8, like.device)
    torch = _t()
    # torch's caching allocator returns 512-byte aligned blocks.
    return torch.empty(max(int(nbytes), 256), dtype=torch.uint8, device=device)



def _on_stream(t, stream):
    """Tell torch's caching allocator that `t` is used on `stream` (when that is
    not the current stream), so its memory is not reused before the work
    enqueued there has finished.  DeviceArrays are freed by their owner."""
    if _is_torch(t) and stream is not None and _is_torch(stream) and stream != _t().cuda.current_stream(t.device):
        t.record_stream(stream)
    return t


def _call(fn, weights, x, y, alpha, beta, workspace, stream, rank):
    if workspace is None:
        workspace = _on_stream(alloc_workspace(workspace_bytes(weights, x, y, rank), x.device, x), stream)
    d = matmul_desc(weights, x, y, alpha, beta, workspace, rank)
    abi.check(fn(weights.ctx.handle, C.byref(d), C.byref(stream_desc(stream))), fn.__name__)
    return y


def gemv(weights, x, y, alpha=1.0, beta=0.0, workspace=None, stream=None):
    return _call(weights.lib.strix_gemv, weights, x, y, alpha, beta, workspace, stream, None)


def gemm(weights, x, y, alpha=1.0, beta=0.0, workspace=None, stream=None):
    return _call(weights.lib.strix_gemm, weights, x, y, alpha, beta, workspace, stream, None)


def gemv_noalloc(weights, x, y, alpha=1.0, beta=0.0, stream=None):
    """strix_amd_gemv_noalloc: strix_gemv for 1-8 rows with no workspace and no
    allocation (the split planes use the library's static device scratch)."""
    d = matmul_desc(weights, x, y, alpha, beta, None)
    abi.check(weights.lib.strix_amd_gemv_noalloc(weights.ctx.handle, C.byref(d), C.byref(stream_desc(stream))),
              "strix_amd_gemv_noalloc")
    return y


class LinearPlan:
    def __init__(self, weights, x, y, alpha=1.0, beta=0.0, workspace=None, stream=None, operation="gemv"):
        self.lib = weights.lib
        if workspace is None:
            workspace = _on_stream(alloc_workspace(workspace_bytes(weights, x, y), x.device, x), stream)
        self._keep = (weights, x, y, workspace)
        d = matmul_desc(weights, x, y, alpha, beta, workspace)
        op = abi.OPERATION_GEMV if operation == "gemv" else abi.OPERATION_GEMM
        h = C.c_void_p()
        abi.check(self.lib.strix_linear_plan_create(weights.ctx.handle, C.byref(d), C.byref(stream_desc(stream)), op,
                                                    C.byref(h)), "strix_linear_plan_create")
        self.handle = h

    def submit(self):
        abi.check(self.lib.strix_linear_plan_submit(self.handle), "strix_linear_plan_submit")

    def launches(self):
        n = C.c_uint32()
        abi.check(self.lib.strix_amd_plan_launches(self.handle, C.byref(n)))
        return n.value

    def status(self, clear=False):
        """Sticky status flags of a single-launch plan (abi.GEMV_GAVE_UP); synchronises its stream.

        clear=True re-initialises the plan's whole single-launch state (status,
        epochs, planes), which lifts the poison a give-up leaves."""
        f = C.c_uint32()
        abi.check(self.lib.strix_amd_plan_status(self.handle, int(bool(clear)), C.byref(f)), "strix_amd_plan_status")
        return f.value

    def destroy(self):
        if self.handle:
            abi.check(self.lib.strix_linear_plan_destroy(self.handle), "strix_linear_plan_destroy")
            self.handle = None


class GroupedGemvPlan:
    """Grouped strided GEMV: y[r][g*ogs + n] = Linear_g(x[r][g*igs + i])."""

    def __init__(self, weights_list, x, y, rows, igs, ogs, irs, ors, stream=None, workspace=None):
        self.lib = weights_list[0].lib
        ctx = weights_list[0].ctx
        handles = (C.c_void_p * len(weights_list))(*[w.handle.value for w in weights_list])
        d = abi.header(abi.GroupedGemvDesc, weights=C.cast(handles, C.POINTER(C.c_void_p)),
                       group_count=len(weights_list), rows=rows, flags=abi.GEMV_ROW_INVARIANT_R1,
                       input=C.c_void_p(x.data_ptr()), input_row_stride=irs, input_group_stride=igs,
                       input_buffer_bytes=x.numel() * 4, output=C.c_void_p(y.data_ptr()),
                       output_row_stride=ors, output_group_stride=ogs, output_buffer_bytes=y.numel() * 4)
        need = C.c_uint64()
        abi.check(self.lib.strix_grouped_gemv_workspace_bytes(ctx.handle, C.byref(d), C.byref(need)),
                  "strix_grouped_gemv_workspace_bytes")
        if workspace is None:
            workspace = _on_stream(alloc_workspace(need.value, x.device), stream)
        d.workspace = C.c_void_p(workspace.data_ptr())
        d.workspace_bytes = workspace.numel()
        self._keep = (weights_list, x, y, workspace, handles)
        h = C.c_void_p()
        abi.check(self.lib.strix_grouped_gemv_plan_create(ctx.handle, C.byref(d), C.byref(stream_desc(stream)),
                                                          C.byref(h)), "strix_grouped_gemv_plan_create")
        self.handle = h

    def submit(self):
        abi.check(self.lib.strix_grouped_gemv_plan_submit(self.handle), "strix_grouped_gemv_plan_submit")

    def fold(self):
        """abi.FOLD_SPLIT or abi.FOLD_OWNER."""
        f = C.c_uint32()
        abi.check(self.lib.strix_amd_grouped_plan_fold(self.handle, C.byref(f)), "strix_amd_grouped_plan_fold")
        return f.value

    def status(self, clear=False):
        """Sticky status flags (abi.GEMV_GAVE_UP); synchronises the plan's stream."""
        f = C.c_uint32()
        abi.check(self.lib.strix_amd_grouped_plan_status(self.handle, int(bool(clear)), C.byref(f)),
                  "strix_amd_grouped_plan_status")
        return f.value

    def destroy(self):
        if self.handle:
            abi.check(self.lib.strix_grouped_gemv_plan_destroy(self.handle), "strix_grouped_gemv_plan_destroy")
            self.handle = None


def row_view_desc(t):
    """F32 descriptor of a rank-2 row view (unit channel stride, any row stride)."""
    if t.dtype != _t().float32 or t.dim() != 2 or t.stride(1) != 1:
        raise ValueError("row views must be float32 [rows, width] with unit channel stride")
    d = abi.header(abi.TensorDesc)
    d.dtype = abi.DTYPE_F32
    d.data = C.c_void_p(t.data_ptr() or None)
    d.rank = 2
    d.shape[0], d.shape[1] = t.shape[0], t.shape[1]
    d.strides[0], d.strides[1] = t.stride(0), 1
    d.buffer_bytes = ((t.shape[0] - 1) * t.stride(0) + t.shape[1]) * 4
    return d


class MoePlan:
    """Routed-expert block y = alpha * sum_s score * down(SwiGLU(gate(x), up(x))) + beta * y.

    ``experts`` is a list of (gate, up, down) Weights.  Host routes
    (``ids``/``scores`` NumPy [rows, k]) name experts by ``expert_ids`` (default
    0..E-1) and must use exactly the given experts; device routes
    (``device_ids``/``device_scores`` torch int32/float32 [rows, k]) index the
    bank, may be rewritten between submissions and are read by every launch.
    """

    def __init__(self, ctx, experts, x, y, ids=None, scores=None, expert_ids=None, device_ids=None,
                 device_scores=None, alpha=1.0, beta=0.0, workspace=None, stream=None, split=False):
        """``split`` builds a split plan: its workspace holds hidden, then the
        down core's per-split partials P [rows, k, S, I] (``self.partials``),
        which the staged ``down_core`` / ``down_finish`` /
        ``down_reference_core`` write and read."""
        self.lib = ctx.lib
        torch = _t()
        n = len(experts)
        arr = (abi.TpExpertDesc * n)()
        for i, (g, u, dn) in enumerate(experts):
            arr[i] = abi.header(abi.TpExpertDesc, expert_id=i if expert_ids is None else int(expert_ids[i]),
                                gate=g.handle.value, up=u.handle.value, down=dn.handle.value)
        self.stream = stream
        sd = stream_desc(stream)
        keep = [arr, experts, x, y]
        rows = x.shape[0]
        if device_ids is None:
            ids_np = np.ascontiguousarray(ids, dtype=np.uint32)
            sc_np = np.ascontiguousarray(scores, dtype=np.float32)
            keep += [ids_np, sc_np]
            d = abi.header(abi.TpMoeDesc, input=row_view_desc(x), output=row_view_desc(y),
                           experts=C.cast(arr, C.POINTER(abi.TpExpertDesc)), expert_count=n,
                           route_ids=ids_np.ctypes.data_as(C.POINTER(C.c_uint32)), route_ids_count=ids_np.size,
                           route_scores=sc_np.ctypes.data_as(C.POINTER(C.c_float)),
                           route_scores_count=sc_np.size, alpha=alpha, beta=beta)
            k = ids_np.size // rows
        else:
            keep += [device_ids, device_scores]
            d = abi.header(abi.TpMoeDeviceDesc, input=row_view_desc(x), output=row_view_desc(y),
                           experts=C.cast(arr, C.POINTER(abi.TpExpertDesc)), expert_count=n,
                           route_ids=C.c_void_p(device_ids.data_ptr()), route_ids_bytes=device_ids.numel() * 4,
                           route_scores=C.c_void_p(device_scores.data_ptr()),
                           route_scores_bytes=device_scores.numel() * 4, alpha=alpha, beta=beta)
            k = device_ids.numel() // rows
        H, I = experts[0][0].output, experts[0][0].input
        need = C.c_uint64(rows * k * H * 4)
        if split:
            if device_ids is None:
                abi.check(self.lib.strix_tp_moe_split_workspace_bytes(ctx.handle, C.byref(d), C.byref(need)),
                          "strix_tp_moe_split_workspace_bytes")
            else:
                abi.check(self.lib.strix_amd_tp_moe_device_workspace_bytes(ctx.handle, C.byref(d), 1,
                                                                           C.byref(need)),
                          "strix_amd_tp_moe_device_workspace_bytes")
        if workspace is None:
            workspace = _on_stream(torch.empty(need.value // 4, dtype=torch.float32, device=x.device), stream)
        d.workspace = C.c_void_p(workspace.data_ptr())
        d.workspace_bytes = workspace.numel() * workspace.element_size()
        keep.append(workspace)
        self.workspace = workspace
        self.hidden = workspace[:rows * k * H].view(rows, k, H)
        self.partials = None
        if split:
            off = (rows * k * H * 4 + 255) // 256 * 256 // 4
            splits = (need.value // 4 - off) // (rows * k * I)
            self.partials = workspace[off:off + rows * k * splits * I].view(rows, k, splits, I)
        self._keep = keep
        h = C.c_void_p()
        if device_ids is None:
            fn = self.lib.strix_tp_moe_plan_create_split if split else self.lib.strix_tp_moe_plan_create
        else:
            fn = self.lib.strix_tp_moe_plan_create_device_split if split else self.lib.strix_tp_moe_plan_create_device
        abi.check(fn(ctx.handle, C.byref(d), C.byref(sd), C.byref(h)), fn.__name__)
        self.handle = h

    def submit(self):
        abi.check(self.lib.strix_tp_moe_plan_submit(self.handle), "strix_tp_moe_plan_submit")

    def gate_up(self):
        abi.check(self.lib.strix_tp_moe_plan_gate_up(self.handle), "strix_tp_moe_plan_gate_up")

    def down(self):
        abi.check(self.lib.strix_tp_moe_plan_down(self.handle), "strix_tp_moe_plan_down")

    def down_core(self):
        abi.check(self.lib.strix_tp_moe_plan_down_core(self.handle), "strix_tp_moe_plan_down_core")

    def down_finish(self):
        abi.check(self.lib.strix_tp_moe_plan_down_finish(self.handle), "strix_tp_moe_plan_down_finish")

    def down_reference_core(self):
        abi.check(self.lib.strix_tp_moe_plan_down_reference_core(self.handle),
                  "strix_tp_moe_plan_down_reference_core")

    def destroy(self):
        if self.handle:
            abi.check(self.lib.strix_tp_moe_plan_destroy(self.handle), "strix_tp_moe_plan_destroy")
            self.handle = None


def stream_read(ctx, src, nbytes, workgroups, sink, stream=None, threads=256, depth=4):
    """Launch the streaming-read kernel: `workgroups` x `threads` threads read
    nbytes of device tensor `src` once, `depth` 16-byte loads in flight per
    lane; one word per workgroup (the XOR of its slice) goes to int32 tensor
    `sink`."""
    abi.check(ctx.lib.strix_amd_stream_read_shaped(ctx.handle, C.c_void_p(src.data_ptr()), int(nbytes),
                                                   int(workgroups), int(threads), int(depth),
                                                   C.c_void_p(sink.data_ptr()), C.byref(stream_desc(stream))),
              "strix_amd_stream_read_shaped")


def swiglu(ctx, gate, up, stream=None):
    """Device SwiGLU of the routed-expert block on float32 tensors (diagnostic)."""
    torch = _t()
    h = torch.empty_like(gate)
    abi.check(ctx.lib.strix_amd_swiglu(ctx.handle, C.c_void_p(gate.data_ptr()), C.c_void_p(up.data_ptr()),
                                       C.c_void_p(h.data_ptr()), gate.numel(), C.byref(stream_desc(stream))),
              "strix_amd_swiglu")
    return h


def view_desc(t, rank=2):
    """F32 descriptor of a row view: rank 2 [rows, width] with any row stride, or rank 1 [width]."""
    if rank == 1:
        return tensor_desc(t.reshape(-1), 1)
    return row_view_desc(t)


class TpDensePlan:
    """Tensor-parallel dense projection on row views (strix_tp_dense_plan_*).

    ``variant``: "plain", "tiled", "splitk" or "r1" (``param`` is rows_per_block;
    ``strategy`` the split-K strategy or R1 identity)."""

    def __init__(self, weights, x, y, alpha=1.0, beta=0.0, variant="plain", param=0, strategy=0, stream=None,
                 rank=2):
        self.lib = weights.lib
        d = abi.MatmulDesc()
        self.lib.strix_matmul_desc_init(C.byref(d))
        d.weights = weights.handle
        d.input = view_desc(x, rank)
        d.output = view_desc(y, rank)
        d.alpha, d.beta = alpha, beta
        self._keep = (weights, x, y)
        h = C.c_void_p()
        sd = C.byref(stream_desc(stream))
        if variant == "plain":
            st = self.lib.strix_tp_dense_plan_create(weights.ctx.handle, C.byref(d), sd, C.byref(h))
        elif variant == "tiled":
            st = self.lib.strix_tp_dense_plan_create_tiled(weights.ctx.handle, C.byref(d), sd, param, C.byref(h))
        elif variant == "splitk":
            st = self.lib.strix_tp_dense_plan_create_splitk(weights.ctx.handle, C.byref(d), sd, param, strategy,
                                                            C.byref(h))
        else:
            st = self.lib.strix_tp_dense_plan_create_r1(weights.ctx.handle, C.byref(d), sd, param, strategy,
                                                        C.byref(h))
        abi.check(st, "strix_tp_dense_plan_create")
        self.handle = h

    def submit(self):
        abi.check(self.lib.strix_tp_dense_plan_submit(self.handle), "strix_tp_dense_plan_submit")

    def destroy(self):
        if self.handle:
            abi.check(self.lib.strix_tp_dense_plan_destroy(self.handle), "strix_tp_dense_plan_destroy")
            self.handle = None


class TpPairPlan:
    """Two projections of one input (q_a || kv): strix_tp_dense_pair_plan_*."""

    def __init__(self, w0, w1, x, y0, y1, alphas=(1.0, 1.0), betas=(0.0, 0.0), stream=None):
        self.lib = w0.lib
        d = abi.TpDensePairDesc()
        self.lib.strix_tp_dense_pair_desc_init(C.byref(d))
        d.input = view_desc(x)
        for i, (w, y) in enumerate(((w0, y0), (w1, y1))):
            d.member[i].weights = w.handle
            d.member[i].output = view_desc(y)
            d.member[i].alpha = alphas[i]
            d.member[i].beta = betas[i]
        self._keep = (w0, w1, x, y0, y1)
        h = C.c_void_p()
        abi.check(self.lib.strix_tp_dense_pair_plan_create(w0.ctx.handle, C.byref(d), C.byref(stream_desc(stream)),
                                                           C.byref(h)), "strix_tp_dense_pair_plan_create")
        self.handle = h

    def submit(self):
        abi.check(self.lib.strix_tp_dense_pair_plan_submit(self.handle), "strix_tp_dense_pair_plan_submit")

    def destroy(self):
        if self.handle:
            abi.check(self.lib.strix_tp_dense_pair_plan_destroy(self.handle), "strix_tp_dense_pair_plan_destroy")
            self.handle = None


class TpSwigluPlan:
    """hidden = SwiGLU(gate(x), up(x)) (strix_tp_swiglu_plan_*); optional diagnostic gate/up outputs."""

    def __init__(self, gate, up, x, hidden, diag_gate=None, diag_up=None, stream=None):
        self.lib = gate.lib
        d = abi.TpSwigluDesc()
        self.lib.strix_tp_swiglu_desc_init(C.byref(d))
        d.input = view_desc(x)
        d.gate, d.up = gate.handle, up.handle
        d.hidden_output = view_desc(hidden)
        if diag_gate is not None:
            d.diagnostic_gate = C.c_void_p(diag_gate.data_ptr())
            d.diagnostic_up = C.c_void_p(diag_up.data_ptr())
            d.diagnostic_bytes = diag_gate.numel() * 4
        self._keep = (gate, up, x, hidden, diag_gate, diag_up)
        h = C.c_void_p()
        abi.check(self.lib.strix_tp_swiglu_plan_create(gate.ctx.handle, C.byref(d), C.byref(stream_desc(stream)),
                                                       C.byref(h)), "strix_tp_swiglu_plan_create")
        self.handle = h

    def submit(self):
        abi.check(self.lib.strix_tp_swiglu_plan_submit(self.handle), "strix_tp_swiglu_plan_submit")

    def destroy(self):
        if self.handle:
            abi.check(self.lib.strix_tp_swiglu_plan_destroy(self.handle), "strix_tp_swiglu_plan_destroy")
            self.handle = None
