"""ctypes mirror of include/strix_trellis.h and include/strix_trellis_amd.h.

Struct layouts follow the C header field by field (reference
include/strix_trellis.h:57-262); enums are 32-bit.  ``load()`` opens the
in-tree libstrix_trellis.so built by ``strix-trellis_amd/build.py`` and raises
if it is missing: there is no fallback implementation.
"""
import ctypes as C
import os
from pathlib import Path

ABI_VERSION = 1
TRANSPORT_VERSION = 1
WORKSPACE_ALIGNMENT = 256
MARKER = {"3inst": 0, "mcg": 0xCBAC1FED, "mul1": 0x83DCD12D}
CODEBOOK = {"3inst": 0, "mcg": 1, "mul1": 2}
DTYPE_F32 = 3
TRANSPORT_EXL3_CANONICAL = 1
OPERATION_GEMV = 0
OPERATION_GEMM = 1
GEMV_ROW_INVARIANT_R1 = 1

STATUS = {
    0: "SUCCESS", 1: "INVALID_ARGUMENT", 2: "ABI_MISMATCH", 3: "UNSUPPORTED_FORMAT",
    4: "UNSUPPORTED_DEVICE", 5: "INSUFFICIENT_BUFFER", 6: "OUT_OF_MEMORY", 7: "BACKEND",
    8: "NOT_IMPLEMENTED",
}
STATUS_CODE = {v: k for k, v in STATUS.items()}

u32, u64, i32, f32, vp = C.c_uint32, C.c_uint64, C.c_int32, C.c_float, C.c_void_p


class Metadata(C.Structure):
    _fields_ = [("struct_size", u32), ("transport_version", u32), ("rows", u64), ("columns", u64),
                ("bits_x2", u32), ("codebook", u32), ("marker", u32), ("flags", u32),
                ("trellis_offset", u64), ("trellis_bytes", u64), ("suh_offset", u64), ("suh_bytes", u64),
                ("svh_offset", u64), ("svh_bytes", u64), ("bias_offset", u64), ("bias_bytes", u64),
                ("reserved", u64 * 4)]


class TransportDesc(C.Structure):
    _fields_ = [("struct_size", u32), ("abi_version", u32), ("format", u32), ("transport_version", u32),
                ("data", vp), ("data_bytes", u64), ("metadata", vp), ("metadata_bytes", u64),
                ("rows", u64), ("columns", u64), ("reserved", u64 * 4)]


class HostRegion(C.Structure):
    _fields_ = [("data", vp), ("bytes", u64)]


class PartsDesc(C.Structure):
    _fields_ = [("struct_size", u32), ("abi_version", u32), ("transport_version", u32), ("bits_x2", u32),
                ("rows", u64), ("columns", u64), ("codebook", u32), ("marker", u32),
                ("trellis", HostRegion), ("suh", HostRegion), ("svh", HostRegion), ("bias", HostRegion),
                ("reserved", u64 * 4)]


class Stream(C.Structure):
    _fields_ = [("struct_size", u32), ("abi_version", u32), ("hip_stream", vp), ("reserved", u64 * 2)]


class ContextDesc(C.Structure):
    _fields_ = [("struct_size", u32), ("abi_version", u32), ("device_ordinal", i32), ("flags", u32),
                ("reserved", u64 * 4)]


class TensorDesc(C.Structure):
    _fields_ = [("struct_size", u32), ("abi_version", u32), ("data", vp), ("buffer_bytes", u64),
                ("dtype", u32), ("rank", u32), ("shape", u64 * 2), ("strides", u64 * 2), ("reserved", u64 * 4)]


class MatmulDesc(C.Structure):
    _fields_ = [("struct_size", u32), ("abi_version", u32), ("weights", vp), ("input", TensorDesc),
                ("output", TensorDesc), ("alpha", f32), ("beta", f32), ("workspace", vp),
                ("workspace_bytes", u64), ("reserved", u64 * 4)]


class GroupedMoeDesc(C.Structure):
    _fields_ = [("struct_size", u32), ("abi_version", u32), ("groups", C.POINTER(MatmulDesc)),
                ("group_count", u64), ("workspace", vp), ("workspace_bytes", u64), ("reserved", u64 * 4)]


class GroupedGemvDesc(C.Structure):
    _fields_ = [("struct_size", u32), ("abi_version", u32), ("weights", C.POINTER(vp)), ("group_count", u64),
                ("rows", u32), ("flags", u32), ("input", vp), ("input_row_stride", u64),
                ("input_group_stride", u64), ("input_buffer_bytes", u64), ("output", vp),
                ("output_row_stride", u64), ("output_group_stride", u64), ("output_buffer_bytes", u64),
                ("workspace", vp), ("workspace_bytes", u64), ("reserved", u64 * 4)]


class TpExpertDesc(C.Structure):
    _fields_ = [("struct_size", u32), ("abi_version", u32), ("expert_id", u32), ("flags", u32),
                ("gate", vp), ("up", vp), ("down", vp), ("reserved", u64 * 2)]


class TpMoeDesc(C.Structure):
    _fields_ = [("struct_size", u32), ("abi_version", u32), ("input", TensorDesc), ("output", TensorDesc),
                ("experts", C.POINTER(TpExpertDesc)), ("expert_count", u64),
                ("route_ids", C.POINTER(u32)), ("route_ids_count", u64),
                ("route_scores", C.POINTER(f32)), ("route_scores_count", u64),
                ("workspace", vp), ("workspace_bytes", u64), ("alpha", f32), ("beta", f32),
                ("reserved", u64 * 4)]


class TpMoeDeviceDesc(C.Structure):
    _fields_ = [("struct_size", u32), ("abi_version", u32), ("input", TensorDesc), ("output", TensorDesc),
                ("experts", C.POINTER(TpExpertDesc)), ("expert_count", u64),
                ("route_ids", vp), ("route_ids_bytes", u64), ("route_scores", vp), ("route_scores_bytes", u64),
                ("workspace", vp), ("workspace_bytes", u64), ("alpha", f32), ("beta", f32),
                ("reserved", u64 * 4)]


class TpDensePairMember(C.Structure):
    _fields_ = [("weights", vp), ("output", TensorDesc), ("alpha", f32), ("beta", f32)]


class TpDensePairDesc(C.Structure):
    _fields_ = [("struct_size", u32), ("abi_version", u32), ("input", TensorDesc),
                ("member", TpDensePairMember * 2), ("workspace", vp), ("workspace_bytes", u64),
                ("rows_per_block", u32), ("strategy", u32), ("reserved", u64 * 4)]


class TpSwigluDesc(C.Structure):
    _fields_ = [("struct_size", u32), ("abi_version", u32), ("input", TensorDesc), ("gate", vp), ("up", vp),
                ("hidden_output", TensorDesc), ("workspace", vp), ("workspace_bytes", u64),
                ("rows_per_block", u32), ("strategy", u32), ("diagnostic_gate", vp), ("diagnostic_up", vp),
                ("diagnostic_bytes", u64), ("reserved", u64 * 4)]


def header(struct_type, **fields):
    """Zero-initialised descriptor with struct_size / abi_version set."""
    d = struct_type()
    d.struct_size = C.sizeof(struct_type)
    if hasattr(d, "abi_version"):
        d.abi_version = ABI_VERSION
    for k, v in fields.items():
        setattr(d, k, v)
    return d


LIB_PATH = Path(__file__).resolve().parent / "_native" / "libstrix_trellis.so"

_S = C.c_int  # strix_status
_PROTOTYPES = {
    "strix_get_abi_version": (u32, []),
    "strix_status_string": (C.c_char_p, [_S]),
    "strix_matmul_desc_init": (None, [C.POINTER(MatmulDesc)]),
    "strix_context_create": (_S, [C.POINTER(ContextDesc), C.POINTER(vp)]),
    "strix_context_destroy": (_S, [vp]),
    "strix_weights_prepare": (_S, [vp, C.POINTER(TransportDesc), C.POINTER(Stream), C.POINTER(vp)]),
    "strix_weights_prepare_parts": (_S, [vp, C.POINTER(PartsDesc), C.POINTER(Stream), C.POINTER(vp)]),
    "strix_weights_destroy": (_S, [vp]),
    "strix_weights_device_span": (_S, [vp, C.POINTER(vp), C.POINTER(u64)]),
    "strix_matmul_workspace_bytes": (_S, [vp, C.POINTER(MatmulDesc), C.POINTER(u64)]),
    "strix_gemv": (_S, [vp, C.POINTER(MatmulDesc), C.POINTER(Stream)]),
    "strix_gemm": (_S, [vp, C.POINTER(MatmulDesc), C.POINTER(Stream)]),
    "strix_linear_plan_create": (_S, [vp, C.POINTER(MatmulDesc), C.POINTER(Stream), u32, C.POINTER(vp)]),
    "strix_linear_plan_submit": (_S, [vp]),
    "strix_linear_plan_destroy": (_S, [vp]),
    "strix_grouped_moe_workspace_bytes": (_S, [vp, C.POINTER(GroupedMoeDesc), C.POINTER(u64)]),
    "strix_grouped_moe": (_S, [vp, C.POINTER(GroupedMoeDesc), C.POINTER(Stream)]),
    "strix_grouped_gemv_workspace_bytes": (_S, [vp, C.POINTER(GroupedGemvDesc), C.POINTER(u64)]),
    "strix_grouped_gemv_plan_create": (_S, [vp, C.POINTER(GroupedGemvDesc), C.POINTER(Stream), C.POINTER(vp)]),
    "strix_grouped_gemv_plan_submit": (_S, [vp]),
    "strix_grouped_gemv_plan_destroy": (_S, [vp]),
    "strix_tp_moe_desc_init": (None, [C.POINTER(TpMoeDesc)]),
    "strix_tp_moe_device_desc_init": (None, [C.POINTER(TpMoeDeviceDesc)]),
    "strix_tp_moe_workspace_bytes": (_S, [vp, C.POINTER(TpMoeDesc), C.POINTER(u64)]),
    "strix_tp_moe_split_workspace_bytes": (_S, [vp, C.POINTER(TpMoeDesc), C.POINTER(u64)]),
    "strix_tp_moe_plan_create": (_S, [vp, C.POINTER(TpMoeDesc), C.POINTER(Stream), C.POINTER(vp)]),
    "strix_tp_moe_plan_create_split": (_S, [vp, C.POINTER(TpMoeDesc), C.POINTER(Stream), C.POINTER(vp)]),
    "strix_tp_moe_plan_create_device": (_S, [vp, C.POINTER(TpMoeDeviceDesc), C.POINTER(Stream), C.POINTER(vp)]),
    "strix_tp_moe_plan_create_device_split": (_S, [vp, C.POINTER(TpMoeDeviceDesc), C.POINTER(Stream),
                                                   C.POINTER(vp)]),
    "strix_tp_moe_plan_submit": (_S, [vp]),
    "strix_tp_moe_plan_gate_up": (_S, [vp]),
    "strix_tp_moe_plan_down": (_S, [vp]),
    "strix_tp_moe_plan_down_core": (_S, [vp]),
    "strix_tp_moe_plan_down_finish": (_S, [vp]),
    "strix_tp_moe_plan_down_reference_core": (_S, [vp]),
    "strix_tp_moe_plan_destroy": (_S, [vp]),
    "strix_amd_decode": (_S, [vp, vp, u64, C.POINTER(Stream)]),
    "strix_amd_input_stage": (_S, [vp, vp, u64, vp, u64, C.POINTER(Stream)]),
    "strix_amd_output_stage": (_S, [vp, vp, u64, vp, u64, f32, f32, C.POINTER(Stream)]),
    "strix_amd_gemv_shape": (_S, [vp, C.POINTER(u32), C.POINTER(u32)]),
    "strix_amd_plan_launches": (_S, [vp, C.POINTER(u32)]),
    "strix_amd_gemm_splits": (_S, [vp, u64, C.POINTER(u32)]),
    "strix_amd_swiglu": (_S, [vp, vp, vp, vp, u64, C.POINTER(Stream)]),
    "strix_amd_tp_moe_device_workspace_bytes": (_S, [vp, C.POINTER(TpMoeDeviceDesc), u32, C.POINTER(u64)]),
    "strix_amd_set_gemm_handoff": (_S, [vp, u32]),
    "strix_amd_set_gemv_poll_limit": (_S, [vp, u32]),
    "strix_amd_set_plan_state_reuse": (_S, [vp, u32]),
    "strix_amd_plan_status": (_S, [vp, u32, C.POINTER(u32)]),
    "strix_amd_grouped_plan_status": (_S, [vp, u32, C.POINTER(u32)]),
    "strix_amd_stream_read": (_S, [vp, vp, u64, u32, vp, C.POINTER(Stream)]),
    "strix_amd_stream_read_shaped": (_S, [vp, vp, u64, u32, u32, u32, vp, C.POINTER(Stream)]),
    "strix_amd_gemv_noalloc": (_S, [vp, C.POINTER(MatmulDesc), C.POINTER(Stream)]),
    "strix_amd_set_grouped_fold": (_S, [vp, u32]),
    "strix_amd_grouped_plan_fold": (_S, [vp, C.POINTER(u32)]),
    "strix_tp_dense_plan_create": (_S, [vp, C.POINTER(MatmulDesc), C.POINTER(Stream), C.POINTER(vp)]),
    "strix_tp_dense_plan_create_tiled": (_S, [vp, C.POINTER(MatmulDesc), C.POINTER(Stream), u32, C.POINTER(vp)]),
    "strix_tp_dense_plan_create_splitk": (_S, [vp, C.POINTER(MatmulDesc), C.POINTER(Stream), u32, u32,
                                               C.POINTER(vp)]),
    "strix_tp_dense_plan_create_r1": (_S, [vp, C.POINTER(MatmulDesc), C.POINTER(Stream), u32, u32, C.POINTER(vp)]),
    "strix_tp_dense_workspace_bytes": (_S, [vp, C.POINTER(MatmulDesc), u32, C.POINTER(u64)]),
    "strix_tp_dense_plan_submit": (_S, [vp]),
    "strix_tp_dense_plan_destroy": (_S, [vp]),
    "strix_tp_dense_pair_desc_init": (None, [C.POINTER(TpDensePairDesc)]),
    "strix_tp_swiglu_desc_init": (None, [C.POINTER(TpSwigluDesc)]),
    "strix_tp_dense_pair_plan_create": (_S, [vp, C.POINTER(TpDensePairDesc), C.POINTER(Stream), C.POINTER(vp)]),
    "strix_tp_dense_pair_plan_create_r1": (_S, [vp, C.POINTER(TpDensePairDesc), C.POINTER(Stream), u32,
                                                C.POINTER(vp)]),
    "strix_tp_dense_pair_plan_submit": (_S, [vp]),
    "strix_tp_dense_pair_plan_destroy": (_S, [vp]),
    "strix_tp_swiglu_plan_create": (_S, [vp, C.POINTER(TpSwigluDesc), C.POINTER(Stream), C.POINTER(vp)]),
    "strix_tp_swiglu_plan_submit": (_S, [vp]),
    "strix_tp_swiglu_plan_destroy": (_S, [vp]),
}

GEMV_POLL_DEFAULT = 1 << 22
GEMV_GAVE_UP = 1
GEMV_NOALLOC_SCRATCH_BYTES = 4 << 20
FOLD_AUTO, FOLD_SPLIT, FOLD_OWNER = 0, 1, 2

_lib = None


def load(path=None):
    """Open the native library once; raise if it has not been built."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    # STRIX_TRELLIS_LIB selects another build of the same library (a path to a .so).
    p = Path(path) if path else Path(os.environ.get("STRIX_TRELLIS_LIB", LIB_PATH))
    if not p.exists():
        raise RuntimeError(f"libstrix_trellis.so not built at {p}; run strix-trellis_amd/build.py")
    lib = C.CDLL(str(p))
    for name, (res, args) in _PROTOTYPES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if path is None:
        _lib = lib
    return lib


class StrixError(RuntimeError):
    def __init__(self, status, what=""):
        self.status = status
        self.name = STATUS.get(status, f"UNKNOWN({status})")
        super().__init__(f"{what}: STRIX_{self.name}" if what else f"STRIX_{self.name}")


def check(status, what=""):
    if status != 0:
        raise StrixError(status, what)
    return status
