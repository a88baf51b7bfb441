"""The Python package without PyTorch (CPU): a child interpreter in which
``import torch`` fails imports strix_trellis, loads an EXL3 group from a
safetensors file, builds the call descriptors from HIP-runtime arrays and
streams, and reaches Exl3Tensor.matmul's argument checks -- without importing
torch.  (The GPU run of the same path is tests/test_gpu_python.py.)"""
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

safetensors_numpy = pytest.importorskip("safetensors.numpy")

ROOT = Path(__file__).resolve().parents[1]
MUL1 = 0x83DCD12D

CHILD = r'''
import sys
sys.modules["torch"] = None              # any "import torch" now raises ImportError
sys.path[:0] = [{pkg!r}]
import numpy as np
import strix_trellis
from strix_trellis import abi, device, runtime, load_exl3

t = load_exl3({path!r}, "layer")
assert (t.input_size, t.output_size, t.bits, t.codebook) == (256, 384, 4.0, "mul1")

# the default stream is the device's NULL stream; a HIP stream passes through
assert runtime.stream_desc(None).hip_stream is None
class FakeStream:                          # the attribute a device.Stream carries
    cuda_stream = 0x1234
assert runtime.stream_desc(FakeStream()).hip_stream == 0x1234

# F32 descriptors from device arrays (no allocation: a stand-in for a
# DeviceArray's surface at a made-up address)
class FakeArray(device.DeviceArray):
    def __init__(self, shape):
        self.shape, self.dtype, self.device, self._ptr = tuple(shape), np.dtype(np.float32), 0, 0x10000
        self.nbytes = int(np.prod(shape)) * 4
    def __del__(self):
        pass
d = runtime.tensor_desc(FakeArray((3, 256)))
assert (d.rank, d.shape[0], d.shape[1], d.strides[0], d.strides[1]) == (2, 3, 256, 256, 1)
assert d.data == 0x10000 and d.buffer_bytes == 3 * 256 * 4 and d.dtype == abi.DTYPE_F32
d1 = runtime.tensor_desc(FakeArray((384,)))
assert (d1.rank, d1.shape[0], d1.strides[0]) == (1, 384, 1)
try:
    bad = FakeArray((2, 256)); bad.dtype = np.dtype(np.float16)
    runtime.tensor_desc(bad)
    raise SystemExit("float16 accepted")
except ValueError:
    pass

# matmul: the FP64 reference form is not part of the library; shapes are
# checked before any device work
try:
    t.matmul(np.zeros(256, np.float32))
    raise SystemExit("production=False ran")
except NotImplementedError:
    pass
try:
    t.matmul(np.zeros((2, 255), np.float32), production=True)
    raise SystemExit("bad shape accepted")
except ValueError:
    pass
assert t.matmul(np.zeros((0, 256), np.float32), production=True).shape == (0, 384)

# the HIP runtime loads (it answers with no device here)
assert device.device_count() >= 0
assert sys.modules.get("torch") is None, "torch was imported"
print("ok")
'''


def write_group(path, I=256, N=384, K=4, seed=91):
    g = np.random.Generator(np.random.PCG64(seed))
    tensors = {
        "layer.trellis": g.integers(-32768, 32768, (I // 16, N // 16, 16 * K), dtype=np.int16),
        "layer.suh": g.choice(np.array([-1.0, 1.0]), I).astype(np.float16),
        "layer.svh": (g.choice(np.array([-1.0, 1.0]), N) * g.uniform(0.5, 1.5, N)).astype(np.float16),
        "layer.bias": g.standard_normal(N).astype(np.float32),
        "layer.mul1": np.array([MUL1], np.uint32).view(np.int32).reshape(()),
    }
    safetensors_numpy.save_file(tensors, str(path))
    return tensors


def test_package_runs_without_torch(tmp_path):
    path = tmp_path / "layer.safetensors"
    write_group(path)
    code = CHILD.format(pkg=str(ROOT / "strix-trellis_amd"), path=str(path))
    res = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120)
    assert res.returncode == 0 and res.stdout.strip().endswith("ok"), res.stdout + res.stderr
