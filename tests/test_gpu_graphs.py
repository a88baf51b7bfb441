"""Prepared linear plans captured into a HIP graph and replayed.

Capture is allowed once a plan exists (reference docs/API.md:271-276): submit
allocates, copies and synchronises nothing, and every piece of state a launch
needs is either re-armed by the launch itself (the single-launch GEMV's EMPTY
planes) or cleared by a kernel of the same submission (the GEMM's split-tile
handoff flags), never by a memset node.  Each replay follows new inputs
written in place, with eager work and synchronisations between replays, and
must reproduce the eager call's bits.
"""
import pytest

import synth

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


def _weights(ctx, I, N, K, seed, bias=True):
    tr, suh, svh, b = synth.layer(I, N, K, seed, bias)
    return runtime.Weights(ctx, tr, suh, svh, b, "mul1")


# (name, I, N, K, rows, operation): a single-launch GEMV, a four-row GEMV,
# the narrow GEMM with its K split, the wide GEMM with its K split (plane
# finish), and the wide GEMM whose last round splits tiles (handoff flags).
CASES = [
    ("gemv_r1", 4096, 4096, 4, 1, "gemv"),
    ("gemv_r4", 4096, 4096, 4, 4, "gemv"),
    ("gemm_narrow", 2432, 512, 4, 100, "gemm"),
    ("gemm_wide_split", 2432, 512, 4, 256, "gemm"),
    ("gemm_handoff", 4096, 12288, 4, 2048, "gemm"),
]


def test_linear_plans_replay_in_graph(ctx):
    stream = torch.cuda.Stream()
    weights, plans, xs, ys, refs = {}, [], [], [], []
    for name, I, N, K, rows, op in CASES:
        key = (I, N, K)
        if key not in weights:
            weights[key] = _weights(ctx, I, N, K, 700 + I % 97 + K)
        w = weights[key]
        x = torch.empty((rows, I), device=DEV)
        y = torch.empty((rows, N), device=DEV)
        inputs = [torch.from_numpy(synth.activations(rows, I, 800 + 10 * len(plans) + v)).to(DEV) for v in range(3)]
        expected = []
        for xin in inputs:
            ye = torch.empty((rows, N), device=DEV)
            (runtime.gemv if op == "gemv" else runtime.gemm)(w, xin, ye, alpha=0.5, beta=0.0)
            assert bool(torch.isfinite(ye).all()), name
            expected.append(ye)
        plans.append(runtime.LinearPlan(w, x, y, alpha=0.5, beta=0.0, stream=stream, operation=op))
        xs.append(inputs)
        ys.append((x, y))
        refs.append(expected)
    torch.cuda.synchronize()
    print(f"capturing {len(plans)} plans", flush=True)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for p in plans:
            p.submit()
    torch.cuda.synchronize()
    for rep in range(6):
        v = rep % 3
        for (x, y), inputs in zip(ys, xs):
            x.copy_(inputs[v])
            y.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for (name, *_), (x, y), expected in zip(CASES, ys, refs):
            assert torch.equal(y.view(torch.int32), expected[v].view(torch.int32)), (name, rep)
        # eager work between replays, on the same weights and buffers
        runtime.gemv(weights[(4096, 4096, 4)], xs[0][v], ys[0][1], alpha=0.5)
        torch.cuda.synchronize()
        assert torch.equal(ys[0][1].view(torch.int32), refs[0][v].view(torch.int32))
    del graph
    for p in plans:
        p.destroy()
    for w in weights.values():
        w.destroy()

