"""Single-launch GEMV plans: published planes, launch epochs and the sticky, poisoning give-up.

A single-launch plan's finisher waits (bounded) for the other splits' published
partials.  These tests force the give-up path from the host
(strix_amd_set_gemv_poll_limit(ctx, 0): every finisher gives up at once, so
every kernel still exits normally) and check that

  * the give-up is reported: NaN outputs and STRIX_AMD_GEMV_GAVE_UP in the
    plan's sticky status word;
  * it poisons the plan: later submissions with the default limit write NaN
    again (no plane is trusted, since a split of the given-up launch may have
    started after the give-up and published into the next launch's planes),
    and the flag stays set;
  * clearing the status re-initialises the state: the next submissions return
    the exact bits of the two-launch strix_gemv;
  * many submissions in a row, with inputs rewritten between them, each carry
    the bits of strix_gemv (the epoch advances every launch);
  * a plan created after another was destroyed starts clean, whether it takes
    a fresh state (the default) or the destroyed plan's (opt-in reuse).

The interleavings a forced give-up cannot produce on the GPU (a split that
starts after its finisher gave up) are covered by the CPU model in
tests/test_gemv_protocol.py.

Also the call-floor kernel (strix_amd_stream_read): every workgroup's XOR of
its slice of the source.
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
    c.set_gemv_poll_limit(abi.GEMV_POLL_DEFAULT)
    torch.cuda.synchronize()


def _bits(t):
    return t.view(torch.int32).cpu().numpy()


@pytest.mark.parametrize("R", [1, 3, 8])
def test_linear_plan_give_up_then_exact(ctx, R):
    I, N, K = 4096, 4096, 4
    print(f"plan give-up R={R} {I}x{N} K{K}", flush=True)
    tr, suh, svh, b = synth.layer(I, N, K, synth.BASE_SEED + 40 + R, bias=True)
    w = runtime.Weights(ctx, tr, suh, svh, b, "mul1")
    assert w.gemv_shape()[1] > 1
    x = torch.from_numpy(synth.activations(R, I, synth.BASE_SEED + 50 + R)).to(DEV)
    y = torch.empty((R, N), device=DEV)
    ref = torch.empty((R, N), device=DEV)
    runtime.gemv(w, x, ref)
    plan = runtime.LinearPlan(w, x, y)
    assert plan.launches() == 1
    try:
        plan.submit()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(_bits(y), _bits(ref))
        assert plan.status() == 0

        ctx.set_gemv_poll_limit(0)
        y.fill_(0.0)
        plan.submit()
        torch.cuda.synchronize()
        assert torch.isnan(y).all(), "a finisher that gives up writes NaN outputs"
        assert plan.status() == abi.GEMV_GAVE_UP

        ctx.set_gemv_poll_limit(abi.GEMV_POLL_DEFAULT)
        for rep in range(2):
            y.fill_(0.0)
            plan.submit()
            torch.cuda.synchronize()
            assert torch.isnan(y).all(), f"submission {rep} after the give-up trusts a poisoned plane set"
        assert plan.status() == abi.GEMV_GAVE_UP, "the status is sticky"
        assert plan.status(clear=True) == abi.GEMV_GAVE_UP
        assert plan.status() == 0
        for rep in range(3):
            y.fill_(0.0)
            plan.submit()
            torch.cuda.synchronize()
            np.testing.assert_array_equal(_bits(y), _bits(ref), err_msg=f"submission {rep} after the clear")
        assert plan.status() == 0
    finally:
        ctx.set_gemv_poll_limit(abi.GEMV_POLL_DEFAULT)
        plan.destroy()
        w.destroy()


def test_linear_plan_many_submissions(ctx):
    # 64 launches, inputs rewritten in place between them: each equals strix_gemv.
    I, N, K, R = 5120, 5120, 5, 2
    print(f"plan epochs {I}x{N} K{K} R{R}", flush=True)
    tr, suh, svh, _ = synth.layer(I, N, K, synth.BASE_SEED + 60)
    w = runtime.Weights(ctx, tr, suh, svh, None, "mul1")
    x = torch.empty((R, I), device=DEV)
    y = torch.empty((R, N), device=DEV)
    ref = torch.empty((R, N), device=DEV)
    plan = runtime.LinearPlan(w, x, y)
    try:
        g = torch.Generator(device=DEV).manual_seed(7)
        for rep in range(64):
            x.copy_(torch.randn((R, I), device=DEV, generator=g).half().float())
            plan.submit()
            runtime.gemv(w, x, ref)
            torch.cuda.synchronize()
            np.testing.assert_array_equal(_bits(y), _bits(ref), err_msg=f"submission {rep}")
        assert plan.status() == 0
    finally:
        plan.destroy()
        w.destroy()


def test_grouped_plan_give_up_then_exact(ctx):
    G, I, N, K, R = 4, 4096, 1024, 5, 2
    print(f"grouped give-up G={G} {I}->{N} K{K} R{R}", flush=True)
    ws = []
    for g in range(G):
        tr, suh, svh, _ = synth.layer(I, N, K, synth.BASE_SEED + 70 + g)
        ws.append(runtime.Weights(ctx, tr, suh, svh, None, "mul1"))
    x = torch.from_numpy(synth.activations(R, G * I, synth.BASE_SEED + 80)).to(DEV)
    y = torch.empty((R, G * N), device=DEV)
    ref = torch.empty((R, G * N), device=DEV)
    for g in range(G):
        yg = torch.empty((R, N), device=DEV)
        runtime.gemv(ws[g], x[:, g * I:(g + 1) * I].contiguous(), yg)
        ref[:, g * N:(g + 1) * N] = yg
    plan = runtime.GroupedGemvPlan(ws, x, y, R, igs=I, ogs=N, irs=G * I, ors=G * N)
    try:
        plan.submit()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(_bits(y), _bits(ref))
        ctx.set_gemv_poll_limit(0)
        plan.submit()
        torch.cuda.synchronize()
        assert torch.isnan(y).all()
        assert plan.status() == abi.GEMV_GAVE_UP
        ctx.set_gemv_poll_limit(abi.GEMV_POLL_DEFAULT)
        y.fill_(0.0)
        plan.submit()
        torch.cuda.synchronize()
        assert torch.isnan(y).all(), "a poisoned grouped plan trusts no plane until cleared"
        assert plan.status(clear=True) == abi.GEMV_GAVE_UP
        assert plan.status() == 0
        y.fill_(0.0)
        plan.submit()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(_bits(y), _bits(ref))
    finally:
        ctx.set_gemv_poll_limit(abi.GEMV_POLL_DEFAULT)
        plan.destroy()
        for w in ws:
            w.destroy()


@pytest.mark.parametrize("reuse", [False, True])
def test_plan_after_destroy_starts_clean(ctx, reuse):
    # A plan created after a poisoned plan on the same weights was destroyed
    # starts clean: by default with a state of its own (the destroyed plan's
    # stays allocated with the weights), with reuse enabled with the destroyed
    # plan's block, initialised again.  Either way it neither inherits the
    # sticky give-up nor folds stale partials.
    I, N, K, R = 4096, 4096, 4, 2
    print(f"plan after destroy {I}x{N} K{K} R{R} reuse={reuse}", flush=True)
    tr, suh, svh, _ = synth.layer(I, N, K, synth.BASE_SEED + 90)
    w = runtime.Weights(ctx, tr, suh, svh, None, "mul1")
    x = torch.from_numpy(synth.activations(R, I, synth.BASE_SEED + 91)).to(DEV)
    y = torch.empty((R, N), device=DEV)
    ref = torch.empty((R, N), device=DEV)
    runtime.gemv(w, x, ref)
    ctx.set_plan_state_reuse(reuse)
    first = runtime.LinearPlan(w, x, y)
    second = None
    try:
        ctx.set_gemv_poll_limit(0)
        first.submit()
        torch.cuda.synchronize()
        assert first.status() == abi.GEMV_GAVE_UP
        ctx.set_gemv_poll_limit(abi.GEMV_POLL_DEFAULT)
        first.destroy()
        first = None
        second = runtime.LinearPlan(w, x, y)
        assert second.status() == 0
        for rep in range(4):
            y.fill_(0.0)
            second.submit()
            torch.cuda.synchronize()
            np.testing.assert_array_equal(_bits(y), _bits(ref), err_msg=f"submission {rep} of the second plan")
        assert second.status() == 0
    finally:
        ctx.set_gemv_poll_limit(abi.GEMV_POLL_DEFAULT)
        ctx.set_plan_state_reuse(False)
        for plan in (first, second):
            if plan is not None:
                plan.destroy()
        w.destroy()


@pytest.mark.parametrize("nbytes,wgs,threads,depth", [(8 << 20, 512, 256, 4), (1 << 20, 64, 256, 4), (4096, 1, 256, 4),
                                                      (8 << 20, 2048, 64, 16), (8 << 20, 256, 1024, 1),
                                                      (1 << 20, 128, 512, 8), (160, 10, 128, 2)])
def test_stream_read_xor(ctx, nbytes, wgs, threads, depth):
    # Every shape reads each 16-byte word of its slice exactly once (the
    # ring's loads past the slice read nothing).
    print(f"stream read {nbytes} B x {wgs} workgroups x {threads} threads, depth {depth}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(nbytes + wgs + threads + depth)
    src = torch.randint(-2 ** 31, 2 ** 31 - 1, (nbytes // 4,), dtype=torch.int32, device=DEV, generator=g)
    sink = torch.zeros(wgs, dtype=torch.int32, device=DEV)
    runtime.stream_read(ctx, src, nbytes, wgs, sink, threads=threads, depth=depth)
    torch.cuda.synchronize()
    words = src.cpu().numpy().view(np.uint32).reshape(wgs, -1)
    expect = np.bitwise_xor.reduce(words, axis=1)
    np.testing.assert_array_equal(sink.cpu().numpy().view(np.uint32), expect)
