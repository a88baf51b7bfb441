"""GPU runs of the STGPU001 golden fixtures (tests/golden/*.stgpu) through every
route of the C ABI, as the reference's gpu_runtime harness runs its fixtures
(reference tests/gpu_runtime.hip; docs/GPU_TESTS.md:72-108):

* weights prepared three ways -- arrays through strix_weights_prepare_parts,
  and a safetensors file through the loader (borrowed regions, and the blob
  through strix_weights_prepare) -- decode to the fixture's Q bit for bit and
  give bit-identical outputs;
* stage checkpoints bit-exact: the core input from x, the output from the
  fixture's core;
* GEMV (rows 1..8; rank 1 for one row) and GEMM (rows 1..16) within the
  reference gate of the fixture's reference output, for alpha/beta (1, 0),
  (-0.75, 0.25), (0, -0.5) and (1, -0); a zero beta never reads the old
  output, which is NaN-filled.
"""
from pathlib import Path

import numpy as np
import pytest

import synth
from oracle import linear
from strix_trellis import loader
from strix_trellis.fixture import CODEBOOKS, read_stgpu

torch = pytest.importorskip("torch")
safetensors_numpy = pytest.importorskip("safetensors.numpy")
pytestmark = pytest.mark.gpu

from strix_trellis import runtime  # noqa: E402

DEV = "cuda:0"
GOLDEN = sorted((Path(__file__).parent / "golden").glob("*.stgpu"))
ALPHA_BETA = [(1.0, 0.0), (-0.75, 0.25), (0.0, -0.5), (1.0, -0.0)]


@pytest.fixture(scope="module")
def ctx():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    c = runtime.Context(0)
    yield c
    torch.cuda.synchronize()


def _safetensors(tmp_path, meta, f):
    cb = CODEBOOKS[meta["codebook"]]
    tensors = {"layer.trellis": f["trellis"].view(np.int16), "layer.suh": f["suh"], "layer.svh": f["svh"]}
    if cb != "3inst":
        tensors["layer." + cb] = np.array([meta["marker"]], np.uint32).view(np.int32).reshape(())
    if meta["bias"]:
        tensors["layer.bias"] = f["bias"]
    path = tmp_path / "layer.safetensors"
    safetensors_numpy.save_file(tensors, str(path))
    return path


@pytest.mark.parametrize("path", GOLDEN, ids=lambda p: p.stem)
def test_fixture_routes(ctx, tmp_path, path):
    meta, f = read_stgpu(path)
    cb = CODEBOOKS[meta["codebook"]]
    print(f"fixture {path.name}: {meta}", flush=True)
    bias = f["bias"] if meta["bias"] else None
    group = loader.load_exl3(_safetensors(tmp_path, meta, f), "layer")
    ws = [runtime.Weights(ctx, f["trellis"], f["suh"], f["svh"], bias, cb),
          group.prepare(ctx), group.prepare(ctx, blob=True)]
    try:
        x = torch.from_numpy(np.ascontiguousarray(f["x"])).to(DEV)
        R, N = meta["rows"], meta["N"]
        for w in ws:
            q = w.decode()
            torch.cuda.synchronize()
            np.testing.assert_array_equal(q.cpu().numpy().view(np.uint16), f["q"].view(np.uint16))
        w = ws[0]
        a = w.input_stage(x)
        y = w.output_stage(torch.from_numpy(np.ascontiguousarray(f["core"])).to(DEV))
        torch.cuda.synchronize()
        np.testing.assert_array_equal(a.cpu().numpy().view(np.uint16), f["a"].view(np.uint16))
        np.testing.assert_array_equal(y.cpu().numpy().view(np.uint32), f["ref"].view(np.uint32))
        old = torch.from_numpy(np.ascontiguousarray(f["old"])).to(DEV)
        for alpha, beta in ALPHA_BETA:
            ref = linear.apply_alpha_beta(f["ref"], f["old"], alpha, beta)
            for rows in range(1, 9):
                outs = []
                for w in ws:
                    yg = old[:rows].clone() if beta != 0 else torch.full((rows, N), float("nan"), device=DEV)
                    if rows == 1:
                        yv = yg[0]
                        runtime.gemv(w, x[0].contiguous(), yv, alpha=alpha, beta=beta)
                    else:
                        runtime.gemv(w, x[:rows].contiguous(), yg, alpha=alpha, beta=beta)
                    outs.append(yg)
                torch.cuda.synchronize()
                for o in outs[1:]:
                    assert torch.equal(o.view(torch.int32), outs[0].view(torch.int32))
                synth.gate(outs[0].cpu().numpy(), ref[:rows])
            for rows in (1, 2, 8, R):
                yg = old[:rows].clone() if beta != 0 else torch.full((rows, N), float("nan"), device=DEV)
                runtime.gemm(ws[1], x[:rows].contiguous(), yg, alpha=alpha, beta=beta)
                torch.cuda.synchronize()
                synth.gate(yg.cpu().numpy(), ref[:rows])
    finally:
        for w in ws:
            w.destroy()


@pytest.mark.parametrize("site", ["shared_gate", "shared_down"])
def test_tp_rank_views_on_device(ctx, site):
    # Two-rank views prepared through the loader's transport: output halves
    # concatenate to the whole layer's output, input halves (bias on rank 0)
    # sum to it, within the reference gate of the whole-layer GPU result.
    from strix_trellis.tp import SITES, rank_partition
    I, N, axis, _ = SITES[site]
    tr, suh, svh, b = synth.layer(I, N, 4, 880, bias=True)
    g = loader.Exl3Tensor(tr.view(np.int16), suh, svh, 4.0, "mul1", b, "mem", site)
    full = g.prepare(ctx)
    ranks = [rank_partition(g, site, r).prepare(ctx) for r in (0, 1)]
    try:
        x = torch.from_numpy(synth.activations(4, I, 881)).to(DEV)
        y = torch.empty((4, N), device=DEV)
        runtime.gemv(full, x, y)
        if axis == "output":
            parts = [torch.empty((4, N // 2), device=DEV) for _ in ranks]
            for w, p in zip(ranks, parts):
                runtime.gemv(w, x, p)
            got = torch.cat(parts, dim=1)
        else:
            parts = [torch.empty((4, N), device=DEV) for _ in ranks]
            for r, (w, p) in enumerate(zip(ranks, parts)):
                runtime.gemv(w, x[:, r * I // 2:(r + 1) * I // 2].contiguous(), p)
            got = parts[0] + parts[1]
        torch.cuda.synchronize()
        synth.gate(got.cpu().numpy(), y.cpu().numpy())
    finally:
        for w in [full] + ranks:
            w.destroy()
