"""Parity at the benchmark's full sizes: C2 decode GEMV, C3 prefill GEMM, C5 MoE.

The oracle cannot produce every output at these sizes in test time, so each
case combines a sample checked against the staged FP32 oracle (the reference
GPU gate, reference docs/GPU_TESTS.md:129-130) with identities that hold over
the whole output whatever its size:
  * GEMV: every row of an 8-row call carries the bits of a 1-row call;
  * GEMM: the last 1024 rows of a 2048-row call (split-tile handoff) carry the
    bits of a 1024-row call (one K pass per tile);
  * MoE: a token's output does not depend on the other tokens (bitwise); the
    hidden of two slots of every token, every token's output from the GPU's
    own hidden, and one token's whole chain meet the oracle.
"""
import numpy as np
import pytest

import synth
from oracle import codec, linear, moe

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


def test_c2_gemv_4096_to_12288_k6_r8(ctx):
    I, N, K, R = 4096, 12288, 6, 8
    print(f"full-size GEMV {I}x{N} K={K} R={R}", flush=True)
    tr, suh, svh, b = synth.layer(I, N, K, 4401, bias=True)
    w = runtime.Weights(ctx, tr, suh, svh, b, "mul1")
    x = _dev(synth.activations(R, I, 4402))
    y = torch.full((R, N), float("nan"), device=DEV)
    runtime.gemv(w, x, y)
    for r in range(R):
        y1 = torch.full((N,), float("nan"), device=DEV)
        runtime.gemv(w, x[r].contiguous(), y1)
        assert torch.equal(y1.view(torch.int32), y[r].view(torch.int32)), r
    q = codec.dequantize_rotated(tr, K, "mul1")
    ref = linear.matmul_fp32_stages(x.cpu().numpy(), tr, suh, svh, K, "mul1", b, rotated=q)["output_fp32"]
    synth.gate(y.cpu().numpy(), ref)
    w.destroy()


def test_c3_gemm_m2048_4096_to_12288_k5(ctx):
    M, I, N, K = 2048, 4096, 12288, 5
    print(f"full-size GEMM M={M} {I}x{N} K={K}", flush=True)
    tr, suh, svh, b = synth.layer(I, N, K, 4501, bias=False)
    w = runtime.Weights(ctx, tr, suh, svh, b, "mul1")
    x = _dev(synth.activations(M, I, 4502))
    y = torch.full((M, N), float("nan"), device=DEV)
    runtime.gemm(w, x, y)
    y_half = torch.full((1024, N), float("nan"), device=DEV)
    runtime.gemm(w, x[1024:].contiguous(), y_half)
    assert torch.equal(y_half.view(torch.int32), y[1024:].view(torch.int32))
    sel = np.r_[0:16, 1016:1032, M - 16:M]
    q = codec.dequantize_rotated(tr, K, "mul1")
    ref = linear.matmul_fp32_stages(x.cpu().numpy()[sel], tr, suh, svh, K, "mul1", b, rotated=q)["output_fp32"]
    synth.gate(y.cpu().numpy()[sel], ref)
    w.destroy()


def test_c5_moe_64_experts_top8(ctx):
    E, I, H, R, k = 64, 4096, 1536, 8, 8
    print(f"full-size MoE E={E} I={I} H={H} R={R} k={k}", flush=True)
    bank = synth.moe_bank(E, I, H, 2, 4601)
    ids, sc = synth.routes(R, E, k, 4602)
    x = synth.activations(R, I, 4603)
    ws = []
    for e in bank:
        ws.append(tuple(runtime.Weights(ctx, *e[p][:4], "mul1") for p in ("gate", "up", "down")))

    def run(rows):
        y = torch.full((len(rows), I), float("nan"), device=DEV)
        plan = runtime.MoePlan(ctx, ws, _dev(x[rows]), y, device_ids=_dev(ids[rows].astype(np.int32)),
                               device_scores=_dev(sc[rows]))
        plan.submit()
        torch.cuda.synchronize()
        out, hidden = y.cpu().numpy(), plan.hidden.cpu().numpy()
        plan.destroy()
        return out, hidden

    y, hidden = run(np.arange(R))
    assert np.isfinite(y).all()
    for r in range(R):
        yr, _ = run(np.array([r]))
        assert np.array_equal(yr[0].view(np.uint32), y[r].view(np.uint32)), r
    # the hidden of every token's first and last slot against the oracle (gate
    # and up of up to 16 experts; twice the single-linear nrmse bar for SwiGLU
    # of two projections), every token's output from the GPU's own hidden (all
    # 64 down projections; the single-linear gate), and token 5's whole chain
    # from x (max-rel-err <= 1e-3 of the output's scale)
    cache = {}
    for r in range(R):
        for s in (0, k - 1):
            e = int(ids[r, s])
            g = moe.projection(x[r:r + 1], bank[e]["gate"], cache, (e, "gate"))
            u = moe.projection(x[r:r + 1], bank[e]["up"], cache, (e, "up"))
            href = moe.swiglu(g, u)[0].astype(np.float64)
            a = hidden[r, s].astype(np.float64)
            nrmse = np.sqrt(np.sum((a - href) ** 2) / np.sum(href ** 2))
            assert np.max(np.abs(a - href)) <= 5e-4 * max(1.0, np.max(np.abs(href))) and nrmse <= 6e-5, (r, s, nrmse)
    synth.gate(y, moe.down_combine(hidden, bank, ids, sc, cache=cache))
    chain, _ = moe.moe_block(x[5:6], bank, ids[5:6], sc[5:6], cache=cache)
    assert np.max(np.abs(y[5] - chain[0])) <= 1e-3 * np.max(np.abs(chain[0]))
    for t in ws:
        for w in t:
            w.destroy()
