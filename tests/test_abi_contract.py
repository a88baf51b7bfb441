"""CPU checks of the C ABI boundary: the library loads, exports every function
include/strix_trellis.h declares, and its struct layouts agree with the C
compiler's and with the ctypes mirror.  No GPU work is issued here."""
import ctypes as C
import re
import subprocess
from pathlib import Path

import pytest

from strix_trellis import abi

ROOT = Path(__file__).resolve().parents[1]
HEADERS = [ROOT / "include" / "strix_trellis.h", ROOT / "include" / "strix_trellis_amd.h"]


def _declared(header):
    text = header.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(strix_[a-z0-9_]+)\s*\(", text)))


def test_reference_abi_function_count():
    # reference include/strix_trellis.h:264-523 declares 58 functions
    assert len(_declared(HEADERS[0])) == 58


def test_library_exports_every_declared_function():
    lib = abi.load()
    out = subprocess.run(["nm", "-D", "--defined-only", str(abi.LIB_PATH)], capture_output=True, text=True,
                         check=True).stdout
    exported = set(re.findall(r" T (strix_[a-z0-9_]+)", out))
    for h in HEADERS:
        for name in _declared(h):
            assert name in exported, name
            assert hasattr(lib, name)


def test_stage_clock_only_in_the_instrumented_build():
    # The phase-clock hook is compiled only with STX_STAGE_CLOCK=1 (build.py --stage-clock).
    out = subprocess.run(["nm", "-D", "--defined-only", str(abi.LIB_PATH)], capture_output=True, text=True,
                         check=True).stdout
    assert "strix_amd_debug_stage_clock" not in out
    clock = abi.LIB_PATH.with_name("libstrix_trellis_clock.so")
    if not clock.exists():
        pytest.skip("instrumented library not built")
    out = subprocess.run(["nm", "-D", "--defined-only", str(clock)], capture_output=True, text=True, check=True).stdout
    assert " T strix_amd_debug_stage_clock" in out


STRUCTS = {
    "strix_exl3_metadata_v1": abi.Metadata, "strix_exl3_transport_desc": abi.TransportDesc,
    "strix_host_region": abi.HostRegion, "strix_exl3_parts_desc": abi.PartsDesc, "strix_stream": abi.Stream,
    "strix_context_desc": abi.ContextDesc, "strix_tensor_desc": abi.TensorDesc, "strix_matmul_desc": abi.MatmulDesc,
    "strix_grouped_moe_desc": abi.GroupedMoeDesc, "strix_grouped_gemv_desc": abi.GroupedGemvDesc,
    "strix_tp_expert_desc": abi.TpExpertDesc, "strix_tp_moe_desc": abi.TpMoeDesc,
    "strix_tp_moe_device_desc": abi.TpMoeDeviceDesc, "strix_tp_dense_pair_member": abi.TpDensePairMember,
    "strix_tp_dense_pair_desc": abi.TpDensePairDesc, "strix_tp_swiglu_desc": abi.TpSwigluDesc,
}


def test_struct_layouts_match_c_compiler(tmp_path):
    src = tmp_path / "sizes.c"
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "strix_trellis.h"', "int main(void){"]
    for name in STRUCTS:
        lines.append(f'printf("{name} %zu\\n", sizeof({name}));')
    lines.append('printf("strix_matmul_desc.alpha %zu\\n", offsetof(strix_matmul_desc, alpha));')
    lines.append('printf("strix_tp_moe_desc.alpha %zu\\n", offsetof(strix_tp_moe_desc, alpha));')
    lines.append("return 0;}")
    src.write_text("\n".join(lines))
    exe = tmp_path / "sizes"
    subprocess.run(["gcc", "-std=c11", "-Wall", "-Werror", f"-I{ROOT / 'include'}", str(src), "-o", str(exe)],
                   check=True)
    got = dict(l.split() for l in subprocess.run([str(exe)], capture_output=True, text=True).stdout.splitlines())
    for name, ct in STRUCTS.items():
        assert int(got[name]) == C.sizeof(ct), name
    assert int(got["strix_matmul_desc.alpha"]) == abi.MatmulDesc.alpha.offset
    assert int(got["strix_tp_moe_desc.alpha"]) == abi.TpMoeDesc.alpha.offset


def test_status_strings_and_initialisers():
    lib = abi.load()
    assert lib.strix_get_abi_version() == 1
    names = {0: b"success", 1: b"invalid argument", 2: b"ABI mismatch", 3: b"unsupported format",
             4: b"unsupported device", 5: b"insufficient buffer", 6: b"out of memory", 7: b"HIP/backend error",
             8: b"not implemented", 99: b"unknown status"}
    for code, text in names.items():
        assert lib.strix_status_string(code) == text
    d = abi.MatmulDesc()
    d.alpha = 7.0
    d.workspace_bytes = 3
    lib.strix_matmul_desc_init(C.byref(d))
    assert d.struct_size == C.sizeof(abi.MatmulDesc) and d.abi_version == 1
    assert d.alpha == 1.0 and d.beta == 0.0 and d.workspace_bytes == 0
    assert d.input.dtype == abi.DTYPE_F32 and d.output.struct_size == C.sizeof(abi.TensorDesc)
    m = abi.TpMoeDesc()
    lib.strix_tp_moe_desc_init(C.byref(m))
    assert m.alpha == 1.0 and m.struct_size == C.sizeof(abi.TpMoeDesc)


def test_context_header_validation_without_device():
    lib = abi.load()
    h = C.c_void_p(1234)
    assert lib.strix_context_create(None, C.byref(h)) == abi.STATUS_CODE["INVALID_ARGUMENT"]
    assert h.value is None                     # output cleared on failure
    d = abi.header(abi.ContextDesc)
    d.struct_size -= 4
    assert lib.strix_context_create(C.byref(d), C.byref(h)) == abi.STATUS_CODE["ABI_MISMATCH"]
    d = abi.header(abi.ContextDesc, flags=1)
    assert lib.strix_context_create(C.byref(d), C.byref(h)) == abi.STATUS_CODE["INVALID_ARGUMENT"]
    d = abi.header(abi.ContextDesc)
    d.reserved[2] = 1
    assert lib.strix_context_create(C.byref(d), C.byref(h)) == abi.STATUS_CODE["INVALID_ARGUMENT"]
    assert lib.strix_context_destroy(None) == abi.STATUS_CODE["INVALID_ARGUMENT"]
    assert lib.strix_weights_destroy(None) == abi.STATUS_CODE["INVALID_ARGUMENT"]
    assert lib.strix_linear_plan_submit(None) == abi.STATUS_CODE["INVALID_ARGUMENT"]


def test_tp_entry_points_validate_without_device():
    lib = abi.load()
    out = C.c_void_p(99)
    # no context: rejected, output handle cleared
    assert lib.strix_tp_dense_plan_create(None, None, None, C.byref(out)) == abi.STATUS_CODE["INVALID_ARGUMENT"]
    assert out.value is None
    # the integer-A8 MoE identity is not provided
    out = C.c_void_p(99)
    assert lib.strix_tp_moe_plan_create_a8r(None, None, None, C.byref(out)) == abi.STATUS_CODE["NOT_IMPLEMENTED"]
    assert out.value is None
