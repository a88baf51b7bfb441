"""The reference's Python entry point on the GPU:
``load_exl3(path, prefix).matmul(x, production=True)`` (reference
python/strix_trellis/container.py:112-115) runs strix_gemv (1-8 rows) or
strix_gemm (more rows) on NumPy arrays, with device memory and streams from the
HIP runtime.  Its outputs meet the staged FP32 oracle (reference GPU gate),
equal the torch-buffer calls of the same library bit for bit, and a child
interpreter in which ``import torch`` fails computes the same bits."""
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

import synth
from oracle import linear

torch = pytest.importorskip("torch")
safetensors_numpy = pytest.importorskip("safetensors.numpy")
pytestmark = pytest.mark.gpu

from strix_trellis import load_exl3, runtime  # noqa: E402
from test_python_no_torch import write_group  # noqa: E402

ROOT = Path(__file__).resolve().parents[1]
DEV = "cuda:0"
ROWS = (1, 3, 8, 40)

CHILD = r'''
import sys
sys.modules["torch"] = None
sys.path[:0] = [{pkg!r}]
import numpy as np
from strix_trellis import load_exl3
t = load_exl3({path!r}, "layer")
x = np.load({xpath!r})
out = {{}}
for rows in {rows!r}:
    xr = x[0] if rows == 1 else x[:rows]
    out[str(rows)] = t.matmul(xr, production=True)
np.savez({opath!r}, **out)
assert sys.modules.get("torch") is None
print("ok")
'''


@pytest.fixture(scope="module")
def ctx():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    c = runtime.Context(0)
    yield c
    torch.cuda.synchronize()


def test_exl3_tensor_matmul_production(ctx, tmp_path):
    print("Exl3Tensor.matmul(production=True) 256x384 K4, rows 1/3/8/40", flush=True)
    path = tmp_path / "layer.safetensors"
    src = write_group(path)
    t = load_exl3(path, "layer")
    x = synth.activations(max(ROWS), t.input_size, 92)
    tr = src["layer.trellis"].view(np.uint16)
    w = runtime.Weights(ctx, tr, src["layer.suh"], src["layer.svh"], src["layer.bias"], "mul1")
    got = {}
    for rows in ROWS:
        xr = x[0] if rows == 1 else x[:rows]
        y = t.matmul(xr, production=True, context=ctx)
        assert y.dtype == np.float32 and y.shape == xr.shape[:-1] + (t.output_size,)
        ref = linear.matmul_fp32(np.atleast_2d(xr), tr, src["layer.suh"], src["layer.svh"], 4, "mul1",
                                 src["layer.bias"])
        synth.gate(np.atleast_2d(y), ref)
        # the same call through torch buffers: the same bits
        yt = torch.full((rows, t.output_size), float("nan"), device=DEV)
        (runtime.gemv if rows <= 8 else runtime.gemm)(w, torch.from_numpy(np.atleast_2d(xr).copy()).to(DEV), yt)
        torch.cuda.synchronize()
        assert np.array_equal(np.atleast_2d(y).view(np.uint32), yt.cpu().numpy().view(np.uint32)), rows
        got[str(rows)] = y
    w.destroy()

    # a child interpreter without torch
    xpath, opath = tmp_path / "x.npy", tmp_path / "out.npz"
    np.save(xpath, x)
    code = CHILD.format(pkg=str(ROOT / "strix-trellis_amd"), path=str(path), xpath=str(xpath), opath=str(opath),
                        rows=ROWS)
    print("child interpreter without torch", flush=True)
    res = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=180)
    assert res.returncode == 0 and res.stdout.strip().endswith("ok"), res.stdout + res.stderr
    child = np.load(opath)
    for rows in ROWS:
        assert np.array_equal(child[str(rows)].view(np.uint32), got[str(rows)].view(np.uint32)), rows
