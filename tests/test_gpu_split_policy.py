"""GEMV layers whose split count comes from the one-poll-round rule.

`gemv_shape` replaces a split count above 17 by the split count with the most
workgroups among those of at most 17 parts, when that keeps at least 384
workgroups and half the splits and loads the busiest CU no more.  Besides the
benchmark's 5120^2 (C2 tests), these layers change with the rule and are
checked here:
  * the split count the library reports is the rule's (against a restatement
    of the rule on the host);
  * the prepared single-launch plan at R1 and R8, and plain calls at R3, against
    the staged FP32 oracle with the reference GPU gate on two 256-column slices
    (the first and the last; the output stage acts per 128 columns, so a slice
    of whole 128-column groups is a layer of its own);
  * the plan's rows equal 1-row strix_gemv calls bit for bit.
"""
import numpy as np
import pytest

import synth
from oracle import codec, linear

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

from strix_trellis import runtime  # noqa: E402

DEV = "cuda:0"


@pytest.fixture(scope="module")
def ctx():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    c = runtime.Context(0)
    yield c
    torch.cuda.synchronize()


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def _bits(t):
    return t.view(torch.int32).cpu().numpy()


def _rule(I, N):
    """(bps, splits) by the documented policy, restated on the host."""
    nb, nc = I // 16, N // 128
    units = nb // 8
    best = (16, nb // 16) if units % 2 == 0 and nc * (nb // 16) >= 128 else (8, nb // 8)
    for m in range(1, 17):
        if units % m == 0 and nc * (nb // (8 * m)) >= 512:
            best = (8 * m, nb // (8 * m))
    if best[1] > 17:
        w0 = nc * best[1]
        for m in range(1, 17):
            s = nb // (8 * m)
            w1 = nc * s
            if units % m == 0 and s <= 17 and 2 * s >= best[1] and w1 >= 384 and \
                    -(-w1 // 256) * w0 <= -(-w0 // 256) * w1:
                return 8 * m, s
    return best


def _slice(layer, c0, c1):
    tr, suh, svh, b = layer
    return tr[:, c0 // 16:c1 // 16], suh, svh[c0:c1], None if b is None else b[c0:c1]


# (I, N, K, splits before the rule -> after)
@pytest.mark.parametrize("I,N,K,before,after", [(2304, 6144, 4, 18, 9), (4608, 4096, 5, 18, 12),
                                                (9216, 4096, 4, 18, 12), (3840, 4096, 6, 30, 15)])
def test_one_round_split_layers(ctx, I, N, K, before, after):
    print(f"GEMV {I}x{N} K={K}: S {before} -> {after}", flush=True)
    assert _rule(I, N)[1] == after
    layer = synth.layer(I, N, K, 4800 + I // 128 + K, bias=True)
    w = runtime.Weights(ctx, *layer, "mul1")
    assert w.gemv_shape() == _rule(I, N)
    x8 = synth.activations(8, I, 4900 + K)
    xd = _dev(x8)
    slices = [(0, 256), (N - 256, N)]
    qs = [codec.dequantize_rotated(_slice(layer, c0, c1)[0], K, "mul1") for c0, c1 in slices]

    def check(y, x):
        for (c0, c1), q in zip(slices, qs):
            tr, suh, svh, b = _slice(layer, c0, c1)
            ref = linear.matmul_fp32_stages(x, tr, suh, svh, K, "mul1", b, rotated=q)["output_fp32"]
            synth.gate(y[:, c0:c1], ref)

    for R in (1, 8):
        x = xd[:R].contiguous()
        y = torch.full((R, N), float("nan"), device=DEV)
        plan = runtime.LinearPlan(w, x, y)
        plan.submit()
        torch.cuda.synchronize()
        plan.destroy()
        for r in range(R):
            y1 = torch.full((N,), float("nan"), device=DEV)
            runtime.gemv(w, xd[r].contiguous(), y1)
            np.testing.assert_array_equal(_bits(y1), _bits(y[r]), err_msg=f"plan R{R} row {r} vs 1-row strix_gemv")
        check(y.cpu().numpy(), x8[:R])
    y3 = torch.full((3, N), float("nan"), device=DEV)
    runtime.gemv(w, xd[:3].contiguous(), y3)
    torch.cuda.synchronize()
    check(y3.cpu().numpy(), x8[:3])
    w.destroy()
