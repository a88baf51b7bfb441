"""The allocation-free GEMV entry point (strix_amd_gemv_noalloc) against strix_gemv.

strix_amd_gemv_noalloc runs strix_gemv's kernels with the split partial
planes in the library's static device scratch instead of a workspace, so its
output must carry strix_gemv's exact bits.  Two calls in a row, the second on
a smaller layer (the scratch keeps the first call's planes), then the limits:
planes beyond the scratch, more than 8 rows, a workspace in the descriptor.
"""
import numpy as np
import pytest

import synth

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

from strix_trellis import abi, runtime  # noqa: E402

DEV = "cuda:0"


@pytest.fixture(scope="module")
def ctx():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    c = runtime.Context(0)
    yield c
    torch.cuda.synchronize()


def _bits(t):
    return t.view(torch.int32).cpu().numpy()


def _case(ctx, I, N, K, R, seed, alpha=1.0, beta=0.0):
    print(f"noalloc {I}x{N} K{K} R{R} alpha={alpha} beta={beta}", flush=True)
    tr, suh, svh, b = synth.layer(I, N, K, seed, bias=True)
    w = runtime.Weights(ctx, tr, suh, svh, b, "mul1")
    x = torch.from_numpy(synth.activations(R, I, seed + 1)).to(DEV)
    y0 = torch.from_numpy(synth.activations(R, N, seed + 2)).to(DEV)
    ref, got = y0.clone(), y0.clone()
    runtime.gemv(w, x, ref, alpha, beta)
    runtime.gemv_noalloc(w, x, got, alpha, beta)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(_bits(got), _bits(ref))
    w.destroy()


def test_noalloc_matches_strix_gemv_twice(ctx):
    # First the larger planes (8 splits x 8 rows x 12288), then a smaller call.
    _case(ctx, 4096, 12288, 5, 8, synth.BASE_SEED + 90)
    _case(ctx, 4096, 4096, 4, 2, synth.BASE_SEED + 91, alpha=0.5, beta=0.25)


def test_noalloc_limits(ctx):
    print("noalloc limits 5120x40960 K1", flush=True)
    I, N = 5120, 40960
    tr, suh, svh, _ = synth.layer(I, N, 1, synth.BASE_SEED + 92)
    w = runtime.Weights(ctx, tr, suh, svh, None, "mul1")
    bps, splits = w.gemv_shape()
    assert splits * 8 * N * 4 > abi.GEMV_NOALLOC_SCRATCH_BYTES
    x = torch.from_numpy(synth.activations(8, I, 7)).to(DEV)
    y = torch.empty((8, N), device=DEV)
    with pytest.raises(abi.StrixError) as e:
        runtime.gemv_noalloc(w, x, y)
    assert e.value.name == "INSUFFICIENT_BUFFER"
    ref = torch.empty((2, N), device=DEV)
    y2 = torch.empty((2, N), device=DEV)
    runtime.gemv(w, x[:2].contiguous(), ref)
    runtime.gemv_noalloc(w, x[:2].contiguous(), y2)   # two rows fit
    torch.cuda.synchronize()
    np.testing.assert_array_equal(_bits(y2), _bits(ref))
    x9 = torch.zeros((9, I), device=DEV)
    y9 = torch.empty((9, N), device=DEV)
    with pytest.raises(abi.StrixError) as e:
        runtime.gemv_noalloc(w, x9, y9)
    assert e.value.name == "UNSUPPORTED_FORMAT"
    ws = torch.empty(1 << 20, dtype=torch.uint8, device=DEV)
    d = runtime.matmul_desc(w, x[:2].contiguous(), y2, workspace=ws)
    st = ctx.lib.strix_amd_gemv_noalloc(ctx.handle, runtime.C.byref(d), runtime.C.byref(runtime.stream_desc()))
    assert abi.STATUS.get(st) == "INVALID_ARGUMENT"
    w.destroy()
