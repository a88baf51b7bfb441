"""Parity at the benchmark's remaining full-size configurations.

Every cell the benchmark times is also checked here against the staged FP32
oracle with the reference GPU gate (maxabs <= 5e-4 * max(1, max|ref|),
nrmse <= 3e-5; reference docs/GPU_TESTS.md:129-130), on all outputs where the
oracle finishes in seconds and on sampled rows otherwise, plus identities that
hold over the whole output:

  * C2 GEMV 5120^2 and 4096 -> 12288 at K4/K5/K6: R1 and R8 outputs of the
    prepared plan (the path bench.py times) against the oracle, every output;
    the plan equals 1-row strix_gemv calls bitwise; the rows of 2- and 4-row
    calls equal 1-row calls.
  * C3 prefill GEMM, every cell (M = 128, 512, 2048 x 5120^2 and
    4096 -> 12288 x K4/K5/K6): sampled rows against the oracle; a row's bits
    depend only on its row class, so a call on the rows in reverse order
    returns the same rows in reverse order, bit for bit.
  * C4 grouped o_a plan (16 x 4096 -> 1024, K5) at R1 and R8, both folds
    (split and owner): every output of four sampled groups against the
    oracle, all groups finite; for every row count 1-8 the owner-fold plan,
    the split plan and per-group 1-row strix_gemv calls agree bit for bit.
  * TP plans at the reference's own shapes (src/tp_split_api.inc:86-100): the
    q_a || kv pair (5120 -> 1280 and 5120 -> 512) and the SwiGLU pair
    (5120 -> 1152) against the oracle.
"""
import numpy as np
import pytest

import synth
from oracle import codec, linear, moe

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


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def _bits(t):
    return t.view(torch.int32).cpu().numpy()


def _oracle(x, layer, K, q):
    tr, suh, svh, b = layer
    return linear.matmul_fp32_stages(x, tr, suh, svh, K, "mul1", b, rotated=q)["output_fp32"]


@pytest.mark.parametrize("K", [4, 5, 6])
def test_c2_gemv_5120(ctx, K):
    I = N = 5120
    print(f"C2 GEMV {I}x{N} K={K} R1/R2/R4/R8", flush=True)
    layer = synth.layer(I, N, K, 4700 + K, bias=True)
    w = runtime.Weights(ctx, *layer, "mul1")
    q = codec.dequantize_rotated(layer[0], K, "mul1")
    x8 = synth.activations(8, I, 4710 + K)
    xd = _dev(x8)
    ones = []
    for r in range(8):
        y1 = torch.full((N,), float("nan"), device=DEV)
        runtime.gemv(w, xd[r].contiguous(), y1)
        ones.append(y1)
    ones = torch.stack(ones)
    for R in (1, 8):
        x = xd[:R].contiguous()
        y = torch.full((R, N), float("nan"), device=DEV)
        plan = runtime.LinearPlan(w, x, y)
        plan.submit()
        torch.cuda.synchronize()
        plan.destroy()
        np.testing.assert_array_equal(_bits(y), _bits(ones[:R]), err_msg=f"plan R{R} vs 1-row strix_gemv")
        synth.gate(y.cpu().numpy(), _oracle(x8[:R], layer, K, q))
    for R in (2, 4):
        y = torch.full((R, N), float("nan"), device=DEV)
        runtime.gemv(w, xd[:R].contiguous(), y)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(_bits(y), _bits(ones[:R]), err_msg=f"R{R} rows vs 1-row calls")
    w.destroy()


@pytest.mark.parametrize("K", [4, 5, 6])
def test_c2_gemv_4096_to_12288(ctx, K):
    I, N = 4096, 12288
    print(f"C2 GEMV {I}x{N} K={K} R1/R8", flush=True)
    layer = synth.layer(I, N, K, 4750 + K, bias=True)
    w = runtime.Weights(ctx, *layer, "mul1")
    q = codec.dequantize_rotated(layer[0], K, "mul1")
    x8 = synth.activations(8, I, 4760 + K)
    xd = _dev(x8)
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
        synth.gate(y.cpu().numpy(), _oracle(x8[:R], layer, K, q))
    w.destroy()


@pytest.mark.parametrize("I,N,K", [(4096, 12288, 4), (4096, 12288, 5), (4096, 12288, 6),
                                   (5120, 5120, 4), (5120, 5120, 5), (5120, 5120, 6)])
def test_c3_gemm(ctx, I, N, K):
    # Every C3 cell: M = 128, 512, 2048 on this layer.  Sampled rows (ends,
    # the middle, a 256-row tile boundary) against the oracle; the call on the
    # rows in reverse order returns the same rows in reverse, bit for bit.
    layer = synth.layer(I, N, K, 4800 + I // 1024 + K, bias=False)
    w = runtime.Weights(ctx, *layer, "mul1")
    q = codec.dequantize_rotated(layer[0], K, "mul1")
    for M in (128, 512, 2048):
        print(f"C3 GEMM M={M} {I}x{N} K={K}", flush=True)
        x = synth.activations(M, I, 4810 + M + K + I // 1024)
        y = torch.full((M, N), float("nan"), device=DEV)
        runtime.gemm(w, _dev(x), y)
        yr = torch.full((M, N), float("nan"), device=DEV)
        runtime.gemm(w, _dev(x[::-1]), yr)
        torch.cuda.synchronize()
        got = y.cpu().numpy()
        np.testing.assert_array_equal(yr.cpu().numpy()[::-1].view(np.uint32), got.view(np.uint32),
                                      err_msg=f"M={M}: row bits depend on the other rows")
        sel = np.unique(np.r_[0, 1, M // 2 - 1, M // 2, min(255, M - 1), min(256, M - 1), M - 2, M - 1])
        synth.gate(got[sel], _oracle(x[sel], layer, K, q))
        assert np.isfinite(got).all()
        del y, yr
    w.destroy()


@pytest.mark.parametrize("fold", ["split", "owner"])
@pytest.mark.parametrize("R", [1, 8])
def test_c4_grouped_oa(ctx, R, fold):
    G, I, N, K = 16, 4096, 1024, 5
    print(f"C4 grouped {G} x {I}->{N} K={K} R={R} fold={fold}", flush=True)
    layers = [synth.layer(I, N, K, 4900 + g) for g in range(G)]
    ws = [runtime.Weights(ctx, *L, "mul1") for L in layers]
    x = synth.activations(R, G * I, 4950 + R)
    y = torch.full((R, G * N), float("nan"), device=DEV)
    ctx.set_grouped_fold(abi.FOLD_OWNER if fold == "owner" else abi.FOLD_SPLIT)
    try:
        plan = runtime.GroupedGemvPlan(ws, _dev(x), y, R, igs=I, ogs=N, irs=G * I, ors=G * N)
    finally:
        ctx.set_grouped_fold(abi.FOLD_AUTO)
    assert plan.fold() == (abi.FOLD_OWNER if fold == "owner" else abi.FOLD_SPLIT)
    plan.submit()
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    assert np.isfinite(got).all()
    for g in (0, 5, 10, 15):
        q = codec.dequantize_rotated(layers[g][0], K, "mul1")
        synth.gate(got[:, g * N:(g + 1) * N], _oracle(x[:, g * I:(g + 1) * I], layers[g], K, q))
    plan.destroy()
    for w in ws:
        w.destroy()


@pytest.mark.parametrize("G,I,N,K,bias", [(16, 4096, 1024, 5, False), (3, 2048, 384, 4, True),
                                           (2, 1024, 640, 6, True)])
def test_grouped_folds_bit_identical(ctx, G, I, N, K, bias):
    print(f"grouped folds {G} x {I}->{N} K={K} bias={bias} R=1..8", flush=True)
    ws = [runtime.Weights(ctx, *synth.layer(I, N, K, 5100 + g, bias=bias), "mul1") for g in range(G)]
    x = synth.activations(8, G * I, 5150)
    xd = _dev(x)
    ref = torch.empty((8, G * N), device=DEV)
    for g in range(G):
        for r in range(8):
            y1 = torch.empty((N,), device=DEV)
            runtime.gemv(ws[g], xd[r, g * I:(g + 1) * I].contiguous(), y1)
            ref[r, g * N:(g + 1) * N] = y1
    for R in range(1, 9):
        outs = {}
        for fold in (abi.FOLD_SPLIT, abi.FOLD_OWNER):
            y = torch.full((R, G * N), float("nan"), device=DEV)
            ctx.set_grouped_fold(fold)
            try:
                plan = runtime.GroupedGemvPlan(ws, xd[:R].contiguous(), y, R, igs=I, ogs=N, irs=G * I, ors=G * N)
            finally:
                ctx.set_grouped_fold(abi.FOLD_AUTO)
            assert plan.fold() == fold
            for _ in range(2):
                plan.submit()
            torch.cuda.synchronize()
            plan.destroy()
            outs[fold] = y
        np.testing.assert_array_equal(_bits(outs[abi.FOLD_OWNER]), _bits(outs[abi.FOLD_SPLIT]), err_msg=f"R{R}")
        np.testing.assert_array_equal(_bits(outs[abi.FOLD_SPLIT]), _bits(ref[:R]), err_msg=f"R{R} vs strix_gemv")
    for w in ws:
        w.destroy()


def test_tp_pair_reference_shapes(ctx):
    # q_a (5120 -> 1280) || kv (5120 -> 512), K4/K5 as the reference's site table
    I, R = 5120, 4
    print("TP pair 5120->1280 K4 || 5120->512 K5", flush=True)
    la = synth.layer(I, 1280, 4, 5001, bias=True)
    lb = synth.layer(I, 512, 5, 5002)
    wa, wb = runtime.Weights(ctx, *la, "mul1"), runtime.Weights(ctx, *lb, "mul1")
    x = synth.activations(R, I, 5003)
    ya = torch.full((R, 1280), float("nan"), device=DEV)
    yb = torch.full((R, 512), float("nan"), device=DEV)
    plan = runtime.TpPairPlan(wa, wb, _dev(x), ya, yb)
    plan.submit()
    torch.cuda.synchronize()
    synth.gate(ya.cpu().numpy(), _oracle(x, la, 4, codec.dequantize_rotated(la[0], 4, "mul1")))
    synth.gate(yb.cpu().numpy(), _oracle(x, lb, 5, codec.dequantize_rotated(lb[0], 5, "mul1")))
    plan.destroy()
    wa.destroy()
    wb.destroy()


def test_tp_swiglu_reference_shape(ctx):
    # gate and up 5120 -> 1152 (the reference's SwiGLU pair shape)
    I, H, R = 5120, 1152, 3
    print("TP SwiGLU 5120->1152 K4", flush=True)
    lg, lu = synth.layer(I, H, 4, 5011), synth.layer(I, H, 4, 5012)
    g, u = runtime.Weights(ctx, *lg, "mul1"), runtime.Weights(ctx, *lu, "mul1")
    x = synth.activations(R, I, 5013)
    hidden = torch.full((R, H), float("nan"), device=DEV)
    dg = torch.empty((R, H), device=DEV)
    du = torch.empty((R, H), device=DEV)
    plan = runtime.TpSwigluPlan(g, u, _dev(x), hidden, dg, du)
    plan.submit()
    torch.cuda.synchronize()
    rg = _oracle(x, lg, 4, codec.dequantize_rotated(lg[0], 4, "mul1"))
    ru = _oracle(x, lu, 4, codec.dequantize_rotated(lu[0], 4, "mul1"))
    synth.gate(dg.cpu().numpy(), rg)
    synth.gate(du.cpu().numpy(), ru)
    # the activation of the GPU's own projections is bit-exact; the whole
    # pair meets twice the single-linear nrmse bar against the oracle chain
    np.testing.assert_array_equal(hidden.cpu().numpy().view(np.uint32),
                                  moe.swiglu(dg.cpu().numpy(), du.cpu().numpy()).view(np.uint32))
    href = moe.swiglu(rg, ru).astype(np.float64)
    a = hidden.cpu().numpy().astype(np.float64)
    nrmse = np.sqrt(np.sum((a - href) ** 2) / np.sum(href ** 2))
    assert np.max(np.abs(a - href)) <= 5e-4 * max(1.0, np.max(np.abs(href))) and nrmse <= 6e-5, nrmse
    plan.destroy()
    g.destroy()
    u.destroy()
