"""GPU tests of the tensor-parallel dense plans (strix_tp_dense_*, pair, SwiGLU).

Every variant runs the library's decode GEMV on row views, so the bar is
bit-identity with strix_gemv on the same rows (which the GEMV parity tests pin
to the oracle), plus the SwiGLU activation bit-exact to the oracle's.
"""
import numpy as np
import pytest

import synth
from oracle import moe

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


def _w(ctx, I, N, K, seed, bias=False):
    tr, suh, svh, b = synth.layer(I, N, K, seed, bias)
    return runtime.Weights(ctx, tr, suh, svh, b, "mul1")


def _gemv_rows(w, x_rows):
    out = []
    for r in range(x_rows.shape[0]):
        y = torch.empty((w.output,), device=DEV)
        runtime.gemv(w, x_rows[r].contiguous(), y)
        out.append(y)
    torch.cuda.synchronize()
    return torch.stack(out)


@pytest.mark.parametrize("variant,param,strategy", [("plain", 0, 0), ("tiled", 2, 0), ("splitk", 0, 1), ("r1", 1, 0)])
def test_dense_plan_on_row_views_matches_gemv(ctx, variant, param, strategy):
    I, N, K, R = 1280, 512, 5, 4
    w = _w(ctx, I, N, K, 600, bias=True)
    # x is the second half of a wider activation; y likewise
    xa = torch.from_numpy(synth.activations(R, 2 * I, 601)).to(DEV)
    ya = torch.full((R, 2 * N + 64), float("nan"), device=DEV)
    x, y = xa[:, I:], ya[:, N:2 * N]
    old = torch.from_numpy(synth.rng(602).standard_normal((R, N)).astype(np.float32)).to(DEV)
    y.copy_(old)
    plan = runtime.TpDensePlan(w, x, y, alpha=0.5, beta=-1.0, variant=variant, param=param, strategy=strategy)
    plan.submit()
    torch.cuda.synchronize()
    base = _gemv_rows(w, x)
    ref = (np.float32(0.5) * base.cpu().numpy()).astype(np.float32)
    ref = (ref + (np.float32(-1.0) * old.cpu().numpy()).astype(np.float32)).astype(np.float32)
    np.testing.assert_array_equal(y.cpu().numpy().view(np.uint32), ref.view(np.uint32))
    # columns outside the view are untouched
    assert torch.isnan(ya[:, :N]).all() and torch.isnan(ya[:, 2 * N:]).all()
    plan.destroy()
    w.destroy()


def test_dense_plan_rank1_and_validation(ctx):
    I, N, K = 512, 256, 4
    w = _w(ctx, I, N, K, 610)
    x = torch.from_numpy(synth.activations(1, I, 611)).to(DEV)
    y = torch.empty((1, N), device=DEV)
    plan = runtime.TpDensePlan(w, x, y, rank=1)
    plan.submit()
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int32), _gemv_rows(w, x).view(torch.int32))
    # retained weights cannot be destroyed
    assert ctx.lib.strix_weights_destroy(w.handle) != 0
    plan.destroy()
    # 9 rows is not a TP dense shape; rows_per_block above R is rejected
    x9 = torch.zeros((9, I), device=DEV)
    y9 = torch.zeros((9, N), device=DEV)
    with pytest.raises(abi.StrixError):
        runtime.TpDensePlan(w, x9, y9)
    with pytest.raises(abi.StrixError):
        runtime.TpDensePlan(w, x.expand(2, I).contiguous(), torch.zeros((2, N), device=DEV), variant="tiled",
                            param=3)
    w.destroy()


def test_pair_plan_matches_two_gemvs(ctx):
    I, R = 1024, 3
    w0 = _w(ctx, I, 384, 4, 620)
    w1 = _w(ctx, I, 128, 5, 621, bias=True)
    x = torch.from_numpy(synth.activations(R, I, 622)).to(DEV)
    y0 = torch.empty((R, 384), device=DEV)
    y1 = torch.empty((R, 128), device=DEV)
    plan = runtime.TpPairPlan(w0, w1, x, y0, y1)
    for _ in range(2):
        y0.fill_(float("nan"))
        y1.fill_(float("nan"))
        plan.submit()
        torch.cuda.synchronize()
        assert torch.equal(y0.view(torch.int32), _gemv_rows(w0, x).view(torch.int32))
        assert torch.equal(y1.view(torch.int32), _gemv_rows(w1, x).view(torch.int32))
    plan.destroy()
    w0.destroy()
    w1.destroy()


def test_swiglu_plan(ctx):
    I, H, R = 1024, 256, 2
    g = _w(ctx, I, H, 4, 630)
    u = _w(ctx, I, H, 4, 631)
    x = torch.from_numpy(synth.activations(R, I, 632)).to(DEV)
    hidden = torch.full((R, H), float("nan"), device=DEV)
    dg = torch.empty((R, H), device=DEV)
    du = torch.empty((R, H), device=DEV)
    plan = runtime.TpSwigluPlan(g, u, x, hidden, dg, du)
    plan.submit()
    torch.cuda.synchronize()
    gg, uu = _gemv_rows(g, x), _gemv_rows(u, x)
    assert torch.equal(dg.view(torch.int32), gg.view(torch.int32))
    assert torch.equal(du.view(torch.int32), uu.view(torch.int32))
    ref = moe.swiglu(gg.cpu().numpy(), uu.cpu().numpy())
    np.testing.assert_array_equal(hidden.cpu().numpy().view(np.uint32), ref.view(np.uint32))
    plan.destroy()
    # without diagnostic buffers: same hidden
    h2 = torch.full((R, H), float("nan"), device=DEV)
    plan = runtime.TpSwigluPlan(g, u, x, h2)
    plan.submit()
    torch.cuda.synchronize()
    assert torch.equal(h2.view(torch.int32), hidden.view(torch.int32))
    plan.destroy()
    g.destroy()
    u.destroy()
