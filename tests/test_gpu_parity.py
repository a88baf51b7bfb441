"""GPU parity of the HIP path against the CPU oracle, through the C ABI.

Bars (from the north star and reference docs/GPU_TESTS.md:96-143):
  * decoded Q, the FP16 core input and the output stage from a known core are
    bit-exact with the oracle (signed zeros included);
  * the full operator meets the reference GPU gate (maxabs <= 5e-4*max(1,max|ref|),
    nrmse <= 3e-5) against the oracle's staged FP32 layer, and its core is within
    max-rel-err 1e-3 of the FP64 product of the same FP16 operands;
  * rows, plans and groups of one geometry are bit-identical to single-row GEMV.
"""
import numpy as np
import pytest

import synth
from oracle import codec, linear

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


def _weights(ctx, I, N, K, seed, codebook="mul1", bias=False, blob=False):
    tr, suh, svh, b = synth.layer(I, N, K, seed, bias)
    w = runtime.Weights(ctx, tr, suh, svh, b, codebook, blob=blob)
    return w, (tr, suh, svh, b)


def _h16(a):
    return np.ascontiguousarray(a).view(np.uint16)


# --------------------------------------------------------------------------- decode
@pytest.mark.parametrize("codebook", ["mul1", "mcg", "3inst"])
@pytest.mark.parametrize("K", [1, 2, 3, 4, 5, 6, 7, 8])
def test_decode_bit_exact(ctx, K, codebook):
    I, N = 256, 384
    print(f"decode K={K} {codebook} {I}x{N}", flush=True)
    w, (tr, *_rest) = _weights(ctx, I, N, K, 100 + K, codebook)
    q = w.decode().cpu().numpy()
    ref = codec.dequantize_rotated(tr, K, codebook)
    np.testing.assert_array_equal(_h16(q), _h16(ref))
    w.destroy()


def test_decode_covers_every_state_k4(ctx):
    # 16.7M states: every 16-bit state value occurs (~256 times each).
    I = N = 4096
    print("decode K=4 mul1 4096x4096", flush=True)
    w, (tr, *_rest) = _weights(ctx, I, N, 4, synth.BASE_SEED)
    q = w.decode().cpu().numpy()
    states = codec.unpack_states(tr, 4)
    assert np.unique(states).size == 65536
    np.testing.assert_array_equal(_h16(q), _h16(codec.dequantize_rotated(tr, 4)))
    w.destroy()


# --------------------------------------------------------------------------- stages
def _special_x(R, I, seed):
    x = synth.activations(R, I, seed)
    g = synth.rng(seed + 1)
    # ties, subnormals, signed zeros and large values through the RN16 boundary
    specials = np.array([0.0, -0.0, 6e-8, -6e-8, 1e-5, 65504.0 / 4, 0.2001299113035202, 1.0 + 2 ** -11,
                         1.0 + 3 * 2 ** -11, -(2 ** -14)], dtype=np.float32)
    idx = g.choice(I, size=min(I, len(specials) * 4), replace=False)
    x[0, idx] = np.resize(specials, idx.size)
    return x


@pytest.mark.parametrize("R", [1, 3, 8])
def test_input_stage_bit_exact(ctx, R):
    I, N = 512, 256
    print(f"input stage R={R}", flush=True)
    w, (tr, suh, svh, b) = _weights(ctx, I, N, 4, 7)
    x = _special_x(R, I, 11)
    a = w.input_stage(torch.from_numpy(x).to(DEV)).cpu().numpy()
    ref = linear.input_stages_fp32(x, suh)["core_input_fp16"]
    np.testing.assert_array_equal(_h16(a), _h16(ref))
    w.destroy()


@pytest.mark.parametrize("bias", [False, True])
@pytest.mark.parametrize("alpha,beta", [(1.0, 0.0), (0.75, 0.0), (-1.5, 0.5), (0.0, -2.0)])
def test_output_stage_from_known_core_bit_exact(ctx, bias, alpha, beta):
    I, N, R = 256, 512, 3
    print(f"output stage bias={bias} alpha={alpha} beta={beta}", flush=True)
    w, (tr, suh, svh, b) = _weights(ctx, I, N, 5, 13, bias=bias)
    core = synth.rng(5).standard_normal((R, N)).astype(np.float32) * 40
    old = synth.rng(6).standard_normal((R, N)).astype(np.float32)
    y = torch.from_numpy(old.copy()).to(DEV)
    w.output_stage(torch.from_numpy(core).to(DEV), y, alpha, beta)
    ref = linear.apply_alpha_beta(linear.output_stages_fp32(core, svh, b)["output_fp32"], old, alpha, beta)
    np.testing.assert_array_equal(y.cpu().numpy().view(np.uint32), ref.view(np.uint32))
    w.destroy()


# --------------------------------------------------------------------------- full operator
def _oracle(x, tr, suh, svh, b, K, codebook="mul1"):
    q = codec.dequantize_rotated(tr, K, codebook)
    st = linear.matmul_fp32_stages(x, tr, suh, svh, K, codebook, b, rotated=q)
    return st, q


GEMV_CASES = [
    # (I, N, K, codebook, bias)
    (128, 256, 4, "mul1", False),      # one split: workgroup finishes from LDS
    (512, 384, 4, "mul1", True),
    (1024, 1024, 5, "mul1", False),
    (2048, 1280, 6, "mul1", True),
    (4096, 4096, 4, "mul1", False),    # north-star shape
    (768, 512, 2, "mul1", False),
    (512, 256, 3, "mcg", False),
    (512, 256, 3, "3inst", True),
    (256, 512, 8, "mul1", False),
    (384, 256, 1, "mul1", False),
]


@pytest.mark.parametrize("I,N,K,codebook,bias", GEMV_CASES)
@pytest.mark.parametrize("R", [1, 8])
def test_gemv_matches_oracle(ctx, I, N, K, codebook, bias, R):
    print(f"gemv R={R} {I}x{N} K={K} {codebook} bias={bias}", flush=True)
    w, (tr, suh, svh, b) = _weights(ctx, I, N, K, 1000 + I + N + K, codebook, bias)
    x = synth.activations(R, I, 77)
    xt = torch.from_numpy(x).to(DEV)
    y = torch.full((R, N), float("nan"), device=DEV)   # beta = 0 never reads old output
    runtime.gemv(w, xt, y)
    got = y.cpu().numpy()
    st, q = _oracle(x, tr, suh, svh, b, K, codebook)
    synth.gate(got, st["output_fp32"])
    w.destroy()


def test_gemv_core_within_fp64_tolerance(ctx):
    # Core isolation: with suh = svh = 1 and no bias, the output stage is an
    # exact H32 of the core; invert it in FP64 and compare with A @ Q.
    I, N, K, R = 2048, 1024, 4, 4
    tr, _, _, _ = synth.layer(I, N, K, 31)
    suh = np.ones(I, np.float16)
    svh = np.ones(N, np.float16)
    w = runtime.Weights(ctx, tr, suh, svh, None, "mul1")
    x = synth.activations(R, I, 32)
    y = torch.empty((R, N), device=DEV)
    runtime.gemv(w, torch.from_numpy(x).to(DEV), y)
    got = y.cpu().numpy().astype(np.float64)
    a = linear.input_stages_fp32(x, suh)["core_input_fp16"].astype(np.float64)
    q = codec.dequantize_rotated(tr, K).astype(np.float64)
    exact_core = a @ q
    core_est = linear.hadamard(got)           # H is an involution over the reals
    scale = np.max(np.abs(exact_core))
    rel = np.max(np.abs(core_est - exact_core)) / scale
    assert rel <= 1e-3, rel
    w.destroy()


@pytest.mark.parametrize("I,N,K", [(4096, 4096, 4), (1024, 512, 5), (128, 256, 6)])
def test_rows_plans_and_entry_points_bit_identical(ctx, I, N, K):
    print(f"row invariance {I}x{N} K={K}", flush=True)
    w, (tr, suh, svh, b) = _weights(ctx, I, N, K, 5 + K, bias=True)
    # RN16 ties, subnormals and signed zeros in row 0 and, reversed, in rows 1
    # and 5: the 2- and 8-row templates take even rows in lanes 0-31 and odd
    # rows in lanes 32-63, so both halves see them.
    xs = _special_x(8, I, 3)
    xs[1] = xs[0][::-1]
    xs[5] = xs[0][::-1]
    x = torch.from_numpy(np.ascontiguousarray(xs)).to(DEV)
    y8 = torch.empty((8, N), device=DEV)
    runtime.gemv(w, x, y8)
    singles = []
    for r in range(8):
        y1 = torch.empty((N,), device=DEV)
        runtime.gemv(w, x[r].contiguous(), y1)
        singles.append(y1)
    ys = torch.stack(singles)
    assert torch.equal(y8.view(torch.int32), ys.view(torch.int32))
    # single-launch plan, submitted repeatedly (counters reset by the last workgroup)
    yp = torch.empty((8, N), device=DEV)
    plan = runtime.LinearPlan(w, x, yp)
    for _ in range(3):
        yp.fill_(float("nan"))
        plan.submit()
        torch.cuda.synchronize()
        assert torch.equal(yp.view(torch.int32), y8.view(torch.int32))
    assert plan.launches() == 1
    plan.destroy()
    # 2 rows (2-row template), 3 rows (4-row template with a dead row) and 5, 6
    # or 7 rows (8-row template with dead rows) keep their bits
    for rows in (2, 3, 5, 6, 7):
        yr = torch.empty((rows, N), device=DEV)
        runtime.gemv(w, x[:rows].contiguous(), yr)
        assert torch.equal(yr.view(torch.int32), y8[:rows].view(torch.int32)), rows
    # x only 4-byte aligned, which is all the ABI asks of it: the same bits
    for rows in (8, 6, 2, 1):
        buf = torch.empty(rows * I + 1, device=DEV)
        xm = buf[1:].view(rows, I)
        xm.copy_(x[:rows])
        assert xm.data_ptr() % 16 == 4
        ym = torch.empty((rows, N), device=DEV)
        runtime.gemv(w, xm, ym)
        assert torch.equal(ym.view(torch.int32), y8[:rows].view(torch.int32)), rows
    w.destroy()


def test_alpha_beta_and_blob_prepare(ctx):
    I, N, K = 512, 256, 4
    w, (tr, suh, svh, b) = _weights(ctx, I, N, K, 9, bias=True, blob=True)
    x = synth.activations(2, I, 4)
    old = synth.rng(8).standard_normal((2, N)).astype(np.float32)
    y = torch.from_numpy(old.copy()).to(DEV)
    runtime.gemv(w, torch.from_numpy(x).to(DEV), y, alpha=0.5, beta=-1.25)
    base = torch.empty((2, N), device=DEV)
    runtime.gemv(w, torch.from_numpy(x).to(DEV), base)
    ref = linear.apply_alpha_beta(base.cpu().numpy(), old, 0.5, -1.25)
    np.testing.assert_array_equal(y.cpu().numpy().view(np.uint32), ref.view(np.uint32))
    w.destroy()


def test_grouped_gemv_equals_individual(ctx):
    I, N, K, G, R = 1024, 256, 5, 4, 3
    ws, xs = [], []
    for g in range(G):
        w, _ = _weights(ctx, I, N, K, 50 + g)
        ws.append(w)
    x = torch.from_numpy(synth.activations(R, G * I, 12)).to(DEV)
    y = torch.empty((R, G * N), device=DEV)
    plan = runtime.GroupedGemvPlan(ws, x, y, R, igs=I, ogs=N, irs=G * I, ors=G * N)
    for _ in range(2):
        y.fill_(float("nan"))
        plan.submit()
        torch.cuda.synchronize()
        for g in range(G):
            for r in range(R):
                y1 = torch.empty((N,), device=DEV)
                runtime.gemv(ws[g], x[r, g * I:(g + 1) * I].contiguous(), y1)
                assert torch.equal(y[r, g * N:(g + 1) * N].view(torch.int32), y1.view(torch.int32))
    plan.destroy()
    for w in ws:
        w.destroy()


@pytest.mark.parametrize("I,N,K,G,R", [(2048, 1024, 5, 16, 1), (4096, 1024, 5, 16, 1), (4096, 1024, 5, 16, 2),
                                       (4096, 1024, 4, 16, 5)])
def test_grouped_large_grids_equal_individual(ctx, I, N, K, G, R):
    # Grouped plans at the benchmark shape (16 x 4096 -> 1024: 4096 workgroups
    # at R = 1, several rounds of resident workgroups): each group's rows stay
    # bit-identical to strix_gemv on that layer alone.
    print(f"grouped large grid {G}x {I}x{N} K={K} R={R}", flush=True)
    ws = [_weights(ctx, I, N, K, 700 + g, bias=(g % 3 == 0))[0] for g in range(G)]
    x = torch.from_numpy(synth.activations(R, G * I, 13)).to(DEV)
    y = torch.empty((R, G * N), device=DEV)
    plan = runtime.GroupedGemvPlan(ws, x, y, R, igs=I, ogs=N, irs=G * I, ors=G * N)
    ref = torch.empty((R, G * N), device=DEV)
    for g in range(G):
        yg = torch.empty((R, N), device=DEV)
        runtime.gemv(ws[g], x[:, g * I:(g + 1) * I].contiguous(), yg)
        ref[:, g * N:(g + 1) * N] = yg
    for _ in range(3):
        y.fill_(float("nan"))
        plan.submit()
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int32), ref.view(torch.int32))
    plan.destroy()
    for w in ws:
        w.destroy()


def test_errors_and_empty_rows(ctx):
    lib = ctx.lib
    w, _ = _weights(ctx, 256, 128, 4, 1)
    x = torch.empty((0, 256), device=DEV)
    y = torch.empty((0, 128), device=DEV)
    assert runtime.workspace_bytes(w, x, y) == 0
    d = runtime.matmul_desc(w, x, y)
    import ctypes as C
    assert lib.strix_gemv(ctx.handle, C.byref(d), C.byref(runtime.stream_desc())) == 0
    # more than 8 rows is not a GEMV
    x9 = torch.zeros((9, 256), device=DEV)
    y9 = torch.zeros((9, 128), device=DEV)
    ws = runtime.alloc_workspace(runtime.workspace_bytes(w, x9, y9), DEV)
    d = runtime.matmul_desc(w, x9, y9, workspace=ws)
    assert lib.strix_gemv(ctx.handle, C.byref(d), C.byref(runtime.stream_desc())) == abi.STATUS_CODE[
        "UNSUPPORTED_FORMAT"]
    # host memory is not a device buffer
    xh = torch.zeros((2, 256))
    yd = torch.zeros((2, 128), device=DEV)
    ws = runtime.alloc_workspace(1 << 20, DEV)
    d = runtime.matmul_desc(w, xh, yd, workspace=ws)
    assert lib.strix_gemv(ctx.handle, C.byref(d), C.byref(runtime.stream_desc())) == abi.STATUS_CODE[
        "INVALID_ARGUMENT"]
    # destroying weights retained by a plan fails
    xd = torch.zeros((1, 256), device=DEV)
    yd1 = torch.zeros((1, 128), device=DEV)
    plan = runtime.LinearPlan(w, xd, yd1)
    assert lib.strix_weights_destroy(w.handle) == abi.STATUS_CODE["INVALID_ARGUMENT"]
    plan.destroy()
    w.destroy()


@pytest.mark.parametrize("I,N,K", [(3584, 1024, 5), (3072, 1024, 4), (4096, 2048, 4)])
def test_single_launch_plan_with_many_splits(ctx, I, N, K):
    # One row and 17..32 other splits: the last split's workgroup polls the
    # planes with all four waves and folds them from LDS; same bits as the
    # two-launch strix_gemv, on every resubmission.
    w, _ = _weights(ctx, I, N, K, 990 + K, bias=True)
    bps, splits = w.gemv_shape()
    print(f"plan {I}x{N} K={K}: {splits} splits", flush=True)
    assert splits - 1 > 16
    x = torch.from_numpy(synth.activations(1, I, 991)).to(DEV)
    ref = torch.empty((1, N), device=DEV)
    runtime.gemv(w, x, ref)
    y = torch.empty((1, N), device=DEV)
    plan = runtime.LinearPlan(w, x, y)
    for _ in range(3):
        y.fill_(float("nan"))
        plan.submit()
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int32), ref.view(torch.int32))
    plan.destroy()
    w.destroy()
