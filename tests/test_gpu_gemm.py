"""GPU parity of the MFMA prefill GEMM (strix_gemm / GEMM plans) through the C ABI.

Bars: the full operator meets the reference GPU gate against the oracle's
staged FP32 layer (reference docs/GPU_TESTS.md:124-143); the core is within
max-rel-err 1e-3 of the FP64 product of the same FP16 operands; a row's bits
do not depend on the other rows of the call, only on its class: M below 256
(the split-K narrow path, S fixed by the layer), a wide pass whose tiles fill
at most half the CUs (K split in S planes, S fixed by the layer and the number
of 256-row blocks), or one K pass per tile -- and not on the tile shape or
split-tile handoff that computes it.
"""
import ctypes

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


GEMM_CASES = [
    # (M, I, N, K, codebook, bias)
    (16, 256, 256, 4, "mul1", False),
    (129, 512, 384, 5, "mul1", True),
    (300, 256, 640, 6, "mul1", False),
    (512, 1024, 256, 4, "mul1", True),
    (64, 384, 256, 3, "mcg", False),
    (40, 256, 128, 2, "3inst", True),
    (33, 128, 256, 8, "mul1", False),
    (260, 768, 512, 1, "mul1", False),
]


@pytest.mark.parametrize("M,I,N,K,codebook,bias", GEMM_CASES)
def test_gemm_matches_oracle(ctx, M, I, N, K, codebook, bias):
    print(f"gemm M={M} {I}x{N} K={K} {codebook} bias={bias}", flush=True)
    tr, suh, svh, b = synth.layer(I, N, K, 3000 + M + K, bias)
    w = runtime.Weights(ctx, tr, suh, svh, b, codebook)
    x = synth.activations(M, I, 91)
    y = torch.full((M, N), float("nan"), device=DEV)
    runtime.gemm(w, torch.from_numpy(x).to(DEV), y)
    torch.cuda.synchronize()
    q = codec.dequantize_rotated(tr, K, codebook)
    ref = linear.matmul_fp32_stages(x, tr, suh, svh, K, codebook, b, rotated=q)["output_fp32"]
    synth.gate(y.cpu().numpy(), ref)
    w.destroy()


def test_gemm_core_within_fp64_tolerance(ctx):
    M, I, N, K = 256, 2048, 512, 4
    tr, _, _, _ = synth.layer(I, N, K, 41)
    suh = np.ones(I, np.float16)
    svh = np.ones(N, np.float16)
    w = runtime.Weights(ctx, tr, suh, svh, None, "mul1")
    x = synth.activations(M, I, 42)
    y = torch.empty((M, N), device=DEV)
    runtime.gemm(w, torch.from_numpy(x).to(DEV), y)
    got = y.cpu().numpy().astype(np.float64)
    a = linear.input_stages_fp32(x, suh)["core_input_fp16"].astype(np.float64)
    exact = a @ codec.dequantize_rotated(tr, K).astype(np.float64)
    rel = np.max(np.abs(linear.hadamard(got) - exact)) / np.max(np.abs(exact))
    assert rel <= 1e-3, rel
    w.destroy()


def test_gemm_rows_independent_of_batch_and_alpha_beta(ctx):
    # The core's accumulation order depends on the layer and on the row class
    # (below 256: K split in S planes, S fixed by the layer; from 256 on this
    # eight-stage layer: one K pass per tile), never on the other rows.
    I, N, K = 512, 512, 5
    tr, suh, svh, b = synth.layer(I, N, K, 77, bias=True)
    w = runtime.Weights(ctx, tr, suh, svh, b, "mul1")
    x = torch.from_numpy(synth.activations(300, I, 78)).to(DEV)
    y_all = torch.empty((300, N), device=DEV)
    runtime.gemm(w, x, y_all)
    y256 = torch.empty((256, N), device=DEV)
    runtime.gemm(w, x[44:].contiguous(), y256)
    assert torch.equal(y256.view(torch.int32), y_all[44:].view(torch.int32))
    y200 = torch.empty((200, N), device=DEV)
    runtime.gemm(w, x[:200].contiguous(), y200)
    y16 = torch.empty((16, N), device=DEV)
    runtime.gemm(w, x[:16].contiguous(), y16)
    assert torch.equal(y16.view(torch.int32), y200[:16].view(torch.int32))
    y1 = torch.empty((1, N), device=DEV)
    runtime.gemm(w, x[199:200].contiguous(), y1)
    assert torch.equal(y1.view(torch.int32), y200[199:200].view(torch.int32))
    # both classes within the reference gate of the same staged oracle
    q = codec.dequantize_rotated(tr, K, "mul1")
    ref = linear.matmul_fp32_stages(x[:200].cpu().numpy(), tr, suh, svh, K, "mul1", b, rotated=q)["output_fp32"]
    synth.gate(y200.cpu().numpy(), ref)
    synth.gate(y_all[:200].cpu().numpy(), ref)
    # alpha / beta epilogue on top of the same core
    old = torch.from_numpy(synth.rng(5).standard_normal((300, N)).astype(np.float32)).to(DEV)
    y_ab = old.clone()
    runtime.gemm(w, x, y_ab, alpha=-0.5, beta=2.0)
    ref = linear.apply_alpha_beta(y_all.cpu().numpy(), old.cpu().numpy(), -0.5, 2.0)
    np.testing.assert_array_equal(y_ab.cpu().numpy().view(np.uint32), ref.view(np.uint32))
    # a GEMM plan replays the same bits
    yp = torch.empty((300, N), device=DEV)
    plan = runtime.LinearPlan(w, x, yp, operation="gemm")
    for _ in range(2):
        yp.fill_(float("nan"))
        plan.submit()
        torch.cuda.synchronize()
        assert torch.equal(yp.view(torch.int32), y_all.view(torch.int32))
    plan.destroy()
    w.destroy()


@pytest.mark.parametrize("N", [8448, 8192])
def test_gemm_tile_widths_agree(ctx, N):
    # M = 2048 over N = 8448 runs 32 column blocks as 256 x 256 tiles and the
    # last as 256 x 128 tiles; N = 8192 fills the 256 CUs with 256 x 256 tiles
    # only.  256 rows run as 256 x 128 tiles: every row has the same bits
    # whichever tile computes it.
    I, K, M = 256, 4, 2048
    print(f"gemm tile widths M={M} {I}x{N} K={K}", flush=True)
    tr, suh, svh, b = synth.layer(I, N, K, 90 + N, bias=True)
    w = runtime.Weights(ctx, tr, suh, svh, b, "mul1")
    x = torch.from_numpy(synth.activations(M, I, 93)).to(DEV)
    y = torch.full((M, N), float("nan"), device=DEV)
    runtime.gemm(w, x, y)
    yr = torch.full((256, N), float("nan"), device=DEV)
    runtime.gemm(w, x[M - 256:].contiguous(), yr)
    assert torch.equal(yr.view(torch.int32), y[M - 256:].view(torch.int32))
    torch.cuda.synchronize()
    sel = np.r_[0:24, 1000:1016, M - 24:M]
    q = codec.dequantize_rotated(tr, K, "mul1")
    ref = linear.matmul_fp32_stages(x.cpu().numpy()[sel], tr, suh, svh, K, "mul1", b, rotated=q)["output_fp32"]
    synth.gate(y.cpu().numpy()[sel], ref)
    w.destroy()


@pytest.mark.parametrize("I,N,K,codebook,splits", [(2432, 512, 4, "mul1", 4), (1280, 256, 5, "3inst", 2),
                                                    (1024, 8192, 4, "mcg", 2)])
def test_gemm_wide_k_split(ctx, I, N, K, codebook, splits):
    # 256 and 300 rows (1 and 2 row blocks) leave most of the 256 CUs idle, so
    # each tile's K splits in S planes of at least eight 64-channel stages
    # (I = 2432: 38 stages as 9 + 10 + 9 + 10): N = 512 and 256 run 256 x 128
    # tiles, N = 8192 (32 and 64 tiles) 256 x 256 ones.  Both calls fall in the
    # same class, so shared rows keep their bits; the planes fold in ascending
    # split order before the output stage.
    print(f"gemm wide K split {I}x{N} K={K} {codebook} S={splits}", flush=True)
    tr, suh, svh, b = synth.layer(I, N, K, 190 + I, bias=True)
    w = runtime.Weights(ctx, tr, suh, svh, b, codebook)
    for rows in (256, 300):
        got = ctypes.c_uint32()
        assert ctx.lib.strix_amd_gemm_splits(w.handle, rows, ctypes.byref(got)) == 0
        assert got.value == splits, (rows, got.value)
    x = torch.from_numpy(synth.activations(300, I, 191)).to(DEV)
    y = torch.full((300, N), float("nan"), device=DEV)
    runtime.gemm(w, x, y)
    y256 = torch.full((256, N), float("nan"), device=DEV)
    runtime.gemm(w, x[44:].contiguous(), y256)
    assert torch.equal(y256.view(torch.int32), y[44:].view(torch.int32))
    yp = torch.full((300, N), float("nan"), device=DEV)
    plan = runtime.LinearPlan(w, x, yp, operation="gemm")
    for _ in range(2):
        yp.fill_(float("nan"))
        plan.submit()
        torch.cuda.synchronize()
        assert torch.equal(yp.view(torch.int32), y.view(torch.int32))
    plan.destroy()
    sel = np.r_[0:8, 120:136, 292:300]
    q = codec.dequantize_rotated(tr, K, codebook)
    xs = x.cpu().numpy()[sel]
    st = linear.matmul_fp32_stages(xs, tr, suh, svh, K, codebook, b, rotated=q)
    synth.gate(y.cpu().numpy()[sel], st["output_fp32"])
    # alpha / beta on the folded planes: the wide split (300 rows) and the
    # narrow one (100 rows), each on top of its own alpha = 1, beta = 0 core
    for rows in (300, 100):
        xr = x[:rows].contiguous()
        base = torch.empty((rows, N), device=DEV)
        runtime.gemm(w, xr, base)
        old = torch.from_numpy(synth.rng(192 + rows).standard_normal((rows, N)).astype(np.float32)).to(DEV)
        y_ab = old.clone()
        runtime.gemm(w, xr, y_ab, alpha=-0.5, beta=2.0)
        ref = linear.apply_alpha_beta(base.cpu().numpy(), old.cpu().numpy(), -0.5, 2.0)
        np.testing.assert_array_equal(y_ab.cpu().numpy().view(np.uint32), ref.view(np.uint32))
    w.destroy()


@pytest.mark.parametrize("I,N", [(256, 12288), (384, 8448)])
@pytest.mark.parametrize("take_over", [0, 1])
def test_gemm_split_tile_handoff(ctx, I, N, take_over):
    # M = 2048: 384 (12288 columns) or 264 (8448) 256 x 256 tiles, so 128 or 8
    # of them are split at half of K between two workgroups (I = 384: six K
    # stages, split 3 + 3).  With take_over the second workgroup always
    # recomputes the first half itself (the late-head path).  Either way each
    # row keeps the bits of unsplit tiles: those of the same rows run as 256
    # rows (256 x 128 tiles).
    K, M = 4, 2048
    print(f"gemm handoff M={M} {I}x{N} take_over={take_over}", flush=True)
    assert ctx.lib.strix_amd_set_gemm_handoff(ctx.handle, take_over) == 0
    try:
        tr, suh, svh, b = synth.layer(I, N, K, 170 + I, bias=True)
        w = runtime.Weights(ctx, tr, suh, svh, b, "mul1")
        x = torch.from_numpy(synth.activations(M, I, 171)).to(DEV)
        y = torch.full((M, N), float("nan"), device=DEV)
        runtime.gemm(w, x, y)
        plan_y = torch.full((M, N), float("nan"), device=DEV)
        plan = runtime.LinearPlan(w, x, plan_y, operation="gemm")
        for _ in range(2):
            plan_y.fill_(float("nan"))
            plan.submit()
            torch.cuda.synchronize()
            assert torch.equal(plan_y.view(torch.int32), y.view(torch.int32))
        plan.destroy()
        for r0, rows in ((1792, 256), (0, 256), (1000, 256)):
            yr = torch.full((rows, N), float("nan"), device=DEV)
            runtime.gemm(w, x[r0:r0 + rows].contiguous(), yr)
            assert torch.equal(yr.view(torch.int32), y[r0:r0 + rows].view(torch.int32)), (r0, rows)
        torch.cuda.synchronize()
        sel = np.r_[0:8, 1020:1028, M - 8:M]
        q = codec.dequantize_rotated(tr, K, "mul1")
        ref = linear.matmul_fp32_stages(x.cpu().numpy()[sel], tr, suh, svh, K, "mul1", b, rotated=q)["output_fp32"]
        synth.gate(y.cpu().numpy()[sel], ref)
        w.destroy()
    finally:
        assert ctx.lib.strix_amd_set_gemm_handoff(ctx.handle, 0) == 0
