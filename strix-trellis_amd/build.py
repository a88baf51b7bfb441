"""Build libstrix_trellis.so for gfx950 in-tree.

Device translation units (csrc/*.hip) are compiled with hipcc for gfx950 only;
host translation units (csrc/*.cpp, the C ABI layer) with the same compiler in
host mode.  The shared library lands in strix_trellis/_native/, where the
Python package and the tests load it.

    python strix-trellis_amd/build.py            # full rebuild
    python strix-trellis_amd/build.py --changed  # only stale objects
    python strix-trellis_amd/build.py --stage-clock
        # instrumented copy, libstrix_trellis_clock.so: the wide GEMM kernel
        # records per-wave phase cycles (bench.py --stage-clock reads them)
"""
import argparse
import concurrent.futures as cf
import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
OBJ = PKG / "_build"
OUT = PKG / "strix_trellis" / "_native" / "libstrix_trellis.so"
CLOCK_OBJ = PKG / "_build_clock"
CLOCK_OUT = PKG / "strix_trellis" / "_native" / "libstrix_trellis_clock.so"
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
HIPCC = str(ROCM / "bin" / "hipcc")
ARCH = "gfx950"

COMMON = ["-O3", "-std=c++20", "-fPIC", "-ffp-contract=off", "-Wall", "-Wextra",
          f"-I{ROOT / 'include'}", f"-I{CSRC}"]
# Packed FP32 VALU ops are kept out of all device code.  Leading scalar
# kernel arguments are preloaded into SGPRs by the dispatcher (the GEMV passes
# its first-needed fields that way).
DEVICE = [f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
          "-fno-gpu-flush-denormals-to-zero", "-mllvm", "-amdgpu-kernarg-preload-count=16"]
HOST = ["-x", "c++", "-D__HIP_PLATFORM_AMD__", f"-I{ROCM / 'include'}"]


def _sources():
    return sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cpp"))


def _headers_mtime():
    hs = list(CSRC.glob("*.hpp")) + list((ROOT / "include").glob("*.h"))
    return max((h.stat().st_mtime for h in hs), default=0.0)


def _compile(src, changed_only, hdr_mtime, obj_dir=OBJ, defines=()):
    obj = obj_dir / (src.name + ".o")
    if changed_only and obj.exists() and obj.stat().st_mtime >= max(src.stat().st_mtime, hdr_mtime):
        return obj, None
    if src.suffix == ".hip":
        cmd = [HIPCC, *COMMON, *defines, *DEVICE, "-c", str(src), "-o", str(obj)]
    else:
        cmd = [HIPCC, *COMMON, *defines, *HOST, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in (res.stdout + res.stderr).splitlines() if noise not in l)
    if res.returncode != 0:
        return obj, f"compile failed: {src.name}\n{' '.join(cmd)}\n{err}"
    return obj, None


def build(changed_only=False, jobs=None, stage_clock=False):
    """Compile and link the library; with stage_clock, the instrumented copy
    (STX_STAGE_CLOCK=1) into its own object folder and file."""
    obj_dir, out = (CLOCK_OBJ, CLOCK_OUT) if stage_clock else (OBJ, OUT)
    defines = ("-DSTX_STAGE_CLOCK=1",) if stage_clock else ()
    obj_dir.mkdir(parents=True, exist_ok=True)
    out.parent.mkdir(parents=True, exist_ok=True)
    jobs = jobs or min(8, os.cpu_count() or 4)
    hdr = _headers_mtime()
    srcs = _sources()
    with cf.ThreadPoolExecutor(jobs) as ex:
        results = list(ex.map(lambda s: _compile(s, changed_only, hdr, obj_dir, defines), srcs))
    errors = [e for _, e in results if e]
    if errors:
        raise RuntimeError("\n\n".join(errors))
    objs = [str(o) for o, _ in results]
    tmp = out.with_suffix(".so.tmp")
    cmd = [HIPCC, "-shared", "-fPIC", f"--offload-arch={ARCH}", *objs, "-o", str(tmp),
           f"-Wl,-rpath,{ROCM / 'lib'}", "-Wl,--no-undefined"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed\n{' '.join(cmd)}\n{res.stdout}{res.stderr}")
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--changed", action="store_true", help="rebuild only stale objects")
    ap.add_argument("-j", "--jobs", type=int, default=None)
    ap.add_argument("--stage-clock", action="store_true", help="build the phase-clock instrumented copy")
    args = ap.parse_args()
    try:
        print(build(args.changed, args.jobs, args.stage_clock))
    except RuntimeError as exc:
        print(exc, file=sys.stderr)
        sys.exit(1)
