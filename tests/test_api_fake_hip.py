"""CPU contract test of the C ABI layer against a fake HIP runtime.

The real host sources of the library (api*.cpp, dispatch.cpp, policy.cpp) are
compiled unchanged with ``tests/contract/fake/hip/hip_runtime.h`` in place of
the HIP header, linked with a fake runtime (failure knobs, allocation
tracking, call counters) and fake kernel launchers, and run under
AddressSanitizer and UndefinedBehaviorSanitizer (host code only; no GPU code
is built).  The driver ``tests/contract/contract_main.cpp`` checks:

- each injected HIP failure (device properties, allocation, copy, stream
  synchronisation, launch, free) maps to the documented status;
- a failed call leaves no device allocation behind and drains the stream
  before freeing (reference src/api.hip:240-246);
- plan submission allocates, copies, synchronises and queries nothing
  (reference docs/API.md:230-295);
- every launcher receives device buffers sized by its own policy, and the
  single-launch GEMV receives an initialised state;
- the decomposition policy (GEMV splits, GEMM passes, K splits, tile widths,
  handoff, MoE splits) covers every layer of a sweep of shapes within the
  kernels' limits and follows its documented choice rules.
"""
import os
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
CSRC = ROOT / "strix-trellis_amd" / "csrc"
CONTRACT = ROOT / "tests" / "contract"
HOST_SOURCES = sorted(p.name for p in CSRC.glob("api*.cpp")) + ["dispatch.cpp", "policy.cpp"]
FAKE_SOURCES = ["fake_hip.cpp", "fake_launch.cpp", "contract_main.cpp"]


def _clang():
    rocm = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
    for c in (rocm / "llvm" / "bin" / "clang++", shutil.which("clang++")):
        if c and Path(c).exists():
            return str(c)
    return None


def _build(tmp_path, sanitize):
    cxx = _clang()
    if cxx is None:
        pytest.skip("no clang++ for the host-only contract build")
    exe = tmp_path / "contract"
    cmd = [cxx, "-std=c++20", "-O1", "-g", "-fno-omit-frame-pointer", "-ffp-contract=off", "-Wall", "-Wextra",
           "-Werror", f"-I{CONTRACT / 'fake'}", f"-I{CONTRACT}", f"-I{ROOT / 'include'}", f"-I{CSRC}"]
    if sanitize:
        cmd += ["-fsanitize=address,undefined", "-fno-sanitize-recover=undefined"]
    cmd += [str(CSRC / s) for s in HOST_SOURCES] + [str(CONTRACT / s) for s in FAKE_SOURCES]
    cmd += ["-o", str(exe)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    assert res.returncode == 0, res.stdout + res.stderr
    return exe


@pytest.mark.parametrize("sanitize", [True, False], ids=["asan_ubsan", "plain"])
def test_api_contract_fake_hip(tmp_path, sanitize):
    exe = _build(tmp_path, sanitize)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    res = subprocess.run([str(exe)], capture_output=True, text=True, env=env, timeout=300)
    assert res.returncode == 0, res.stdout + res.stderr
    assert "checks passed" in res.stdout
