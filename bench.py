"""Benchmark of the EXL3 trellis hot path on one MI355X.

Headline (`value`): decode GEMV, R = 1, K4 mul1, I = N = 4096 (the north-star
configuration), through a prepared single-launch plan, as packed-weight GB/s
over a cold rotation of >= 1 GiB of distinct weight copies (more than 4x the
256 MB MALL), inputs resident in HBM.  One step = one GEMV call = one launch.

Also reported on the same JSON line:
  sweep_gemv     decode GEMV, R = 1, 2, 4, 8 x {5120^2, 4096 -> 12288} x K4-6
  sweep_gemm     prefill GEMM, M = 128, 512, 2048 x the same shapes x K4-6
  grouped_o_a    16 groups x (4096 -> 1024) K5, R = 1..8, the split and the
                 owner-fold grouped plan (cells carry "fold")
  moe_k2         64 experts (4096 <-> 1536, K2), 8 tokens, top-8, device routes
  roofline       the headline kernel: packed bytes / its mean launch time
  fp16_library   per GEMV/GEMM cell: the same product on dense FP16 weights
                 through torch.matmul (hipBLASLt / rocBLAS), random-normal
                 operands, same rotation and timing -- the vendor library's
                 speed on the unquantised layer, for comparison
  cpu_baseline   the NumPy oracle on the host cores, bounded sample

Timing: each rotation pass (one launch per weight copy) is captured once into
a HIP graph and replayed; exactly --steps launches are timed (whole passes plus
one partial pass, submitted directly when it is short) right behind the
warm-up passes (at least max(--warmup, 512) launches), with no host
synchronisation between them, HIP events on the kernels' own stream bracket
the region, and the time per step is the timed region over the steps.  Every
cell also reports median_pass_us, the median over 11 further whole passes
(an event per pass), whatever --steps is.  Replayed outputs are checked
bit-for-bit against an untimed eager call before the warm-up, after the timed
region and after the passes (`replay_matches_eager`); the headline's output is
also checked against the NumPy oracle (reference GPU gate) before and after
(`oracle_pass`, `oracle_maxabs`, `oracle_nrmse`).

read_ceiling: the fastest of 105 launch shapes (threads x loads in flight per
lane x workgroups) of a streaming-read kernel reading 1 GiB in one launch (4x
the MALL, so cold).  call_floor: for each cell's packed bytes, the fastest of
60 such shapes over a cold rotation of >= 1 GiB (one graph of >= 1024
launches per shape) -- the cost of one launch that moves those bytes and does
nothing else.  Each GEMV,
grouped and MoE cell reports its time as a percentage of that floor and its
bandwidth as a percentage of the read ceiling, beside its percentage of HBM
peak.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--quick] [--no-cpu]
    python bench.py --pmc-workload     # headline plan + a plain copy, for rocprofv3 --pmc
"""
import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for p in (str(ROOT), str(ROOT / "strix-trellis_amd"), str(ROOT / "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)

HBM_PEAK_GBPS = 8000.0
FP16_PEAK_TFLOPS = 2500.0
METRIC = "GEMV R1 µs & HBM GB/s (% peak); prefill GEMM TFLOP/s (% MFMA peak)"
ROTATION_BYTES = 1 << 30
TRAFFIC_FILE = ROOT / "profiles" / "traffic.json"
HEADLINE_KERNEL = "stx::gemv_kernel<4, 2, 1>"


def log(msg):
    print(msg, file=sys.stderr, flush=True)


class Rotation:
    """Distinct device copies of one layer (or one group set), one prepared plan each.

    One pass over the copies is captured into a HIP graph so that the timed
    region measures the GPU, not Python's launch rate.  The copies share x, y
    and the workspace (their calls are ordered on one stream), so after any
    number of passes y holds the result of one call.
    """

    def __init__(self, ctx, I, N, K, R, seed, op="gemv", groups=1, min_bytes=ROTATION_BYTES, fold=None):
        import torch
        import synth
        from strix_trellis import runtime
        self.groups = groups
        layers = [synth.layer(I, N, K, seed + g) for g in range(groups)]
        packed = groups * I * N * K // 8
        self.copies = max(2, -(-min_bytes // packed))
        self.packed = packed
        self.stream = torch.cuda.Stream()
        self.x = torch.from_numpy(synth.activations(R, groups * I, seed + 100)).to("cuda:0")
        self.y = torch.empty((R, groups * N), device="cuda:0")
        self.weights, self.plans = [], []
        ws = None
        for _ in range(self.copies):
            wl = [runtime.Weights(ctx, tr, suh, svh, None, "mul1") for (tr, suh, svh, _) in layers]
            self.weights.extend(wl)
            if op == "grouped":
                # a grouped plan keeps its weight table in its own workspace
                if fold is not None:
                    ctx.set_grouped_fold(fold)
                try:
                    plan = runtime.GroupedGemvPlan(wl, self.x, self.y, R, igs=I, ogs=N, irs=groups * I,
                                                   ors=groups * N, stream=self.stream)
                finally:
                    if fold is not None:
                        ctx.set_grouped_fold(0)
                self.fold = plan.fold()
            else:
                if ws is None:
                    ws = runtime.alloc_workspace(runtime.workspace_bytes(wl[0], self.x, self.y), "cuda:0")
                plan = runtime.LinearPlan(wl[0], self.x, self.y, workspace=ws, stream=self.stream, operation=op)
            self.plans.append(plan)
        self.workspace = ws
        self.launches = self.plans[0].launches() if op != "grouped" else 1
        torch.cuda.synchronize()
        self.plans[0].submit()
        torch.cuda.synchronize()
        self.expected = self.y.clone()
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph, stream=self.stream):
            for p in self.plans:
                p.submit()
        torch.cuda.synchronize()

    def check(self):
        """The replayed plans reproduce the untimed call bit for bit."""
        import torch
        torch.cuda.synchronize()
        return bool(torch.equal(self.y.view(torch.int32), self.expected.view(torch.int32)))

    def partial(self, n):
        """A HIP graph of the first n submissions of a pass (captured once per n)."""
        return capture_partial(self, n)

    def close(self):
        del self.graph
        self.__dict__.pop("_partials", None)
        for p in self.plans:
            p.destroy()
        for w in self.weights:
            w.destroy()


def capture_partial(rot, n):
    import torch
    cache = rot.__dict__.setdefault("_partials", {})
    if n not in cache:
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=rot.stream):
            for p in rot.plans[:n]:
                p.submit()
        torch.cuda.synchronize()
        cache[n] = g
    return cache[n]


PASSES = 11   # whole rotation passes behind every cell's median_pass_us
# A partial pass of at most this many launches is submitted directly: the
# host enqueues it while the GPU still runs the pass before it, so the timed
# region holds no graph-launch boundary (measured on the headline at 20
# steps: 7.2-7.3 us per launch this way, 7.6-7.8 us as a 20-launch graph).
DIRECT_MAX = 64
# Warm-up launches before every timed region: at least this many, whatever
# --warmup asks (which is the minimum), so the timed steps run at the clocks a
# sustained stream of calls reaches.
MIN_WARMUP = 512


def time_rotation(rot, steps, warmup, passes=PASSES):
    """Time exactly `steps` launches (whole rotation passes, then a partial
    pass) right behind >= `warmup` untimed ones, with no host synchronisation
    between the warm-up and the timed region; HIP events on the plans' stream.
    ms = timed region / steps.  Then, separately, `passes` whole passes with an
    event per pass: median_pass_ms = their median per launch, whatever `steps`
    is.  The output is checked against the untimed eager call before the
    warm-up, after the timed region and after the passes."""
    import torch
    full, rem = divmod(steps, rot.copies)
    part = rot.partial(rem) if rem > DIRECT_MAX else None
    with torch.cuda.stream(rot.stream):
        rot.graph.replay()
    ok_before = rot.check()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(full + 2)]
    warm_passes = max(1, -(-max(warmup, MIN_WARMUP) // rot.copies))
    with torch.cuda.stream(rot.stream):
        for _ in range(warm_passes):
            rot.graph.replay()
        ev[0].record(rot.stream)
        for i in range(full):
            rot.graph.replay()
            ev[i + 1].record(rot.stream)
        if part is not None:
            part.replay()
        else:
            for p in rot.plans[:rem]:
                p.submit()
        ev[full + 1].record(rot.stream)
    torch.cuda.synchronize()
    total = ev[0].elapsed_time(ev[full + 1])
    ok_after = rot.check()
    pe = [torch.cuda.Event(enable_timing=True) for _ in range(passes + 1)]
    with torch.cuda.stream(rot.stream):
        rot.graph.replay()
        pe[0].record(rot.stream)
        for i in range(passes):
            rot.graph.replay()
            pe[i + 1].record(rot.stream)
    torch.cuda.synchronize()
    per_pass = [pe[i].elapsed_time(pe[i + 1]) / rot.copies for i in range(passes)]
    ok_passes = rot.check()
    return {"ms": total / steps, "median_pass_ms": statistics.median(per_pass), "timed_steps": steps,
            "warmup_launches": warm_passes * rot.copies, "passes": passes,
            "output_check": ok_before and ok_after and ok_passes}


# Launch shapes of the streaming-read kernel (threads, loads in flight per
# lane, workgroups): the call floor of a byte count is the fastest of
# FLOOR_SHAPES over a cold rotation; the read ceiling the fastest of
# CEILING_SHAPES reading 1 GiB.
FLOOR_SHAPES = [(t, d, w) for t in (256, 512, 1024) for d in (2, 4, 8, 16) for w in (256, 512, 1024, 2048, 4096)]
CEILING_SHAPES = [(t, d, w) for t in (256, 512, 1024) for d in (1, 2, 4, 8, 16)
                  for w in (256, 512, 1024, 2048, 4096, 8192, 16384)]
CEILING_BYTES = 1 << 30


class FloorRotation:
    """Distinct device buffers of `nbytes` each (>= 1 GiB in all); a pass = one
    streaming-read launch per buffer, captured in a HIP graph per launch shape
    and replayed like the plan rotations."""

    def __init__(self, ctx, nbytes, min_bytes=ROTATION_BYTES):
        import torch
        self.ctx, self.nbytes = ctx, nbytes
        self.copies = max(2, -(-min_bytes // nbytes))
        self.stream = torch.cuda.Stream()
        self.bufs = [torch.full((nbytes,), 0x5A, dtype=torch.uint8, device="cuda:0") for _ in range(self.copies)]
        self.sink = torch.zeros(max(w for _, _, w in FLOOR_SHAPES), dtype=torch.int32, device="cuda:0")

    def time_shape(self, shape, launches=1024):
        """Per-launch us of one graph of >= `launches` launches (whole passes)
        in `shape`, replayed once untimed and once timed, so the graph-launch
        boundary is spread over that many launches."""
        import torch
        from strix_trellis import runtime
        threads, depth, wgs = shape
        passes = max(1, -(-launches // self.copies))
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=self.stream):
            for _ in range(passes):
                for b in self.bufs:
                    runtime.stream_read(self.ctx, b, self.nbytes, wgs, self.sink, stream=self.stream,
                                        threads=threads, depth=depth)
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
        with torch.cuda.stream(self.stream):
            graph.replay()
            ev[0].record(self.stream)
            graph.replay()
            ev[1].record(self.stream)
        torch.cuda.synchronize()
        del graph
        return ev[0].elapsed_time(ev[1]) * 1e3 / (passes * self.copies)

    def close(self):
        self.bufs = None


_FLOORS = {}


def call_floor(ctx, nbytes):
    """Call floor of one launch that reads `nbytes` cold: the fastest shape of
    FLOOR_SHAPES whose workgroups split the bytes into whole 16-byte loads.
    Returns {"us", "shape": [threads, depth, workgroups], "shapes"}; cached."""
    if nbytes in _FLOORS:
        return _FLOORS[nbytes]
    rot = FloorRotation(ctx, nbytes)
    best, tried = None, 0
    try:
        for shape in FLOOR_SHAPES:
            if nbytes % (16 * shape[2]):
                continue
            us = rot.time_shape(shape)
            tried += 1
            if best is None or us < best[0]:
                best = (us, shape)
    finally:
        rot.close()
    _FLOORS[nbytes] = {"us": round(best[0], 3), "shape": list(best[1]), "shapes": tried}
    return _FLOORS[nbytes]


_CEILING = {}


def read_ceiling(ctx, passes=3):
    """Sustained HBM read ceiling: the fastest shape of CEILING_SHAPES reading
    CEILING_BYTES (1 GiB, 4x the MALL, so every read is cold) in one launch;
    median of `passes` launches per shape.  Cached."""
    import torch
    from strix_trellis import runtime
    if _CEILING:
        return _CEILING
    buf = torch.full((CEILING_BYTES,), 0x3C, dtype=torch.uint8, device="cuda:0")
    sink = torch.zeros(max(w for _, _, w in CEILING_SHAPES), dtype=torch.int32, device="cuda:0")
    stream = torch.cuda.Stream()
    best = None
    for shape in CEILING_SHAPES:
        threads, depth, wgs = shape
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(passes + 1)]
        with torch.cuda.stream(stream):
            runtime.stream_read(ctx, buf, CEILING_BYTES, wgs, sink, stream=stream, threads=threads, depth=depth)
            ev[0].record(stream)
            for i in range(passes):
                runtime.stream_read(ctx, buf, CEILING_BYTES, wgs, sink, stream=stream, threads=threads, depth=depth)
                ev[i + 1].record(stream)
        torch.cuda.synchronize()
        ms = statistics.median(ev[i].elapsed_time(ev[i + 1]) for i in range(passes))
        gbps = CEILING_BYTES / (ms * 1e-3) / 1e9
        if best is None or gbps > best[0]:
            best = (gbps, shape, ms)
    del buf
    _CEILING.update({"GBps": round(best[0], 1), "pct_hbm_peak": round(100 * best[0] / HBM_PEAK_GBPS, 1),
                     "shape": list(best[1]), "us": round(best[2] * 1e3, 1), "bytes": CEILING_BYTES,
                     "shapes": len(CEILING_SHAPES)})
    return _CEILING


def floor_fields(ctx, us, packed, launch_bytes):
    """% of read ceiling and of the best-shape call floor for a cell of `us`
    per step reading `packed` bytes in launches of `launch_bytes` each."""
    ceil = read_ceiling(ctx)
    floors = [call_floor(ctx, b) for b in launch_bytes]
    floor_us = sum(f["us"] for f in floors)
    gbps = packed / (us * 1e-6) / 1e9
    out = {"call_floor_us": round(floor_us, 3), "pct_call_floor": round(100 * floor_us / us, 1),
           "call_floor_shape": [f["shape"] for f in floors] if len(floors) > 1 else floors[0]["shape"],
           "pct_read_ceiling": round(100 * gbps / ceil["GBps"], 1)}
    return out


_LIBRARY = {}


def library_fp16(M, I, N, passes=5):
    """The same product, y[M][N] = x[M][I] @ W[I][N], on dense FP16 weights
    through torch.matmul (hipBLASLt / rocBLAS), random-normal operands: weight
    copies rotated over >= ROTATION_BYTES, one pass captured in a HIP graph,
    median pass time over HIP events.  Cached per shape."""
    import torch
    key = (M, I, N)
    if key in _LIBRARY:
        return _LIBRARY[key]
    dev = "cuda:0"
    g = torch.Generator(device=dev).manual_seed(M * 131 + I * 7 + N)
    copies = max(2, -(-ROTATION_BYTES // (2 * I * N)))
    ws = [torch.randn((I, N), device=dev, dtype=torch.float16, generator=g) for _ in range(copies)]
    x = torch.randn((M, I), device=dev, dtype=torch.float16, generator=g)
    ys = [torch.empty((M, N), device=dev, dtype=torch.float16) for _ in range(2)]
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        for i in range(copies):
            torch.matmul(x, ws[i], out=ys[i & 1])
    torch.cuda.synchronize()
    expected = [ys[(copies - 2) & 1].clone(), ys[(copies - 1) & 1].clone()]
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for i in range(copies):
            torch.matmul(x, ws[i], out=ys[i & 1])
    graph.replay()
    torch.cuda.synchronize()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(passes + 1)]
    with torch.cuda.stream(stream):
        ev[0].record(stream)
        for i in range(passes):
            graph.replay()
            ev[i + 1].record(stream)
    torch.cuda.synchronize()
    ms = statistics.median(ev[i].elapsed_time(ev[i + 1]) / copies for i in range(passes))
    same = all(torch.equal(ys[(copies - 2 + j) & 1], expected[j]) for j in range(2)) if copies >= 2 else True
    del graph, ws
    out = {"us": round(ms * 1e3, 3), "replay_matches_eager": bool(same)}
    _LIBRARY[key] = out
    return out


def oracle_gate(got, ref):
    """The reference GPU gate (maxabs <= 5e-4 * max(1, max|ref|), nrmse <= 3e-5)."""
    import synth
    maxabs, nrmse = synth.gate_values(got, ref)
    bound = 5e-4 * max(1.0, float(abs(ref).max()))
    return {"maxabs": float(f"{maxabs:.3e}"), "nrmse": float(f"{nrmse:.3e}"),
            "pass": bool(maxabs <= bound and nrmse <= 3e-5)}


def bench_gemv(ctx, I, N, K, R, steps, warmup, seed, oracle=False):
    rot = Rotation(ctx, I, N, K, R, seed, "gemv")
    gate = {}
    try:
        if oracle:
            from oracle import linear
            import synth
            tr, suh, svh, _ = synth.layer(I, N, K, seed)
            ref = linear.matmul_fp32(rot.x.cpu().numpy(), tr, suh, svh, K, "mul1")
            gate["before"] = oracle_gate(rot.expected.cpu().numpy(), ref)
        t = time_rotation(rot, steps, warmup)
        if oracle:
            gate["after"] = oracle_gate(rot.y.cpu().numpy(), ref)
    finally:
        rot.close()
    gbps = rot.packed / (t["ms"] * 1e-3) / 1e9
    lib = library_fp16(R, I, N)
    out = {"I": I, "N": N, "K": K, "R": R, "us": round(t["ms"] * 1e3, 3), "packed_GBps": round(gbps, 1),
           "pct_hbm_peak": round(100 * gbps / HBM_PEAK_GBPS, 1),
           "median_pass_us": round(t["median_pass_ms"] * 1e3, 3), "passes": t["passes"],
           **floor_fields(ctx, t["ms"] * 1e3, rot.packed, [rot.packed]), "launches": rot.launches,
           "rotation_copies": rot.copies, "timed_steps": t["timed_steps"], "warmup_launches": t["warmup_launches"],
           "replay_matches_eager": t["output_check"],
           "fp16_library_us": lib["us"], "speedup_vs_fp16_library": round(lib["us"] / (t["ms"] * 1e3), 2)}
    if oracle:
        out["oracle_gate"] = gate
        out["oracle_pass"] = gate["before"]["pass"] and gate["after"]["pass"]
        out["oracle_maxabs"] = max(gate["before"]["maxabs"], gate["after"]["maxabs"])
        out["oracle_nrmse"] = max(gate["before"]["nrmse"], gate["after"]["nrmse"])
    return out


def bench_gemm(ctx, M, I, N, K, steps, warmup, seed):
    rot = Rotation(ctx, I, N, K, M, seed, "gemm")
    try:
        t = time_rotation(rot, steps, warmup)
    finally:
        rot.close()
    tflops = 2.0 * M * I * N / (t["ms"] * 1e-3) / 1e12
    lib = library_fp16(M, I, N)
    lib_tflops = 2.0 * M * I * N / (lib["us"] * 1e-6) / 1e12
    return {"M": M, "I": I, "N": N, "K": K, "us": round(t["ms"] * 1e3, 2), "TFLOPs": round(tflops, 1),
            "pct_fp16_peak": round(100 * tflops / FP16_PEAK_TFLOPS, 1),
            "median_pass_us": round(t["median_pass_ms"] * 1e3, 2), "passes": t["passes"], "launches": rot.launches,
            "rotation_copies": rot.copies, "timed_steps": t["timed_steps"], "replay_matches_eager": t["output_check"],
            "fp16_library_us": lib["us"], "fp16_library_pct_peak": round(100 * lib_tflops / FP16_PEAK_TFLOPS, 1),
            "speedup_vs_fp16_library": round(lib["us"] / (t["ms"] * 1e3), 2)}


def bench_grouped(ctx, G, I, N, K, R, steps, warmup, seed, fold=None):
    """fold: None (the library's choice), 1 (split plan) or 2 (owner-fold plan)."""
    rot = Rotation(ctx, I, N, K, R, seed, "grouped", groups=G, fold=fold)
    try:
        t = time_rotation(rot, steps, warmup)
    finally:
        rot.close()
    gbps = rot.packed / (t["ms"] * 1e-3) / 1e9
    return {"groups": G, "I": I, "N": N, "K": K, "R": R, "fold": {1: "split", 2: "owner"}[rot.fold],
            "us": round(t["ms"] * 1e3, 3), "median_pass_us": round(t["median_pass_ms"] * 1e3, 3),
            "passes": t["passes"], "packed_GBps": round(gbps, 1), "pct_hbm_peak": round(100 * gbps / HBM_PEAK_GBPS, 1),
            **floor_fields(ctx, t["ms"] * 1e3, rot.packed, [rot.packed]),
            "rotation_copies": rot.copies, "timed_steps": t["timed_steps"], "replay_matches_eager": t["output_check"]}


class MoeRotation:
    """Copies of a whole expert bank, one device-route MoE plan each, all
    reading the same device routes, x and y; one pass captured in a HIP graph."""

    def __init__(self, ctx, E, I, H, K, R, k, seed, min_bytes=ROTATION_BYTES):
        import numpy as np
        import torch
        import synth
        from strix_trellis import runtime
        bank = synth.moe_bank(E, I, H, K, seed)
        ids, scores = synth.routes(R, E, k, seed + 1)
        self.distinct = len(set(ids.ravel().tolist()))
        per_expert = (2 * I * H + H * I) * K // 8
        self.packed = self.distinct * per_expert
        self.copies = max(2, -(-min_bytes // (E * per_expert)))
        self.stream = torch.cuda.Stream()
        self.x = torch.from_numpy(synth.activations(R, I, seed + 2)).to("cuda:0")
        self.y = torch.empty((R, I), device="cuda:0")
        self.ids = torch.from_numpy(ids.astype(np.int32)).to("cuda:0")
        self.scores = torch.from_numpy(scores).to("cuda:0")
        self.weights, self.plans = [], []
        for _ in range(self.copies):
            ws = [tuple(runtime.Weights(ctx, *e[p][:4], "mul1") for p in ("gate", "up", "down")) for e in bank]
            self.weights.extend(w for t in ws for w in t)
            self.plans.append(runtime.MoePlan(ctx, ws, self.x, self.y, device_ids=self.ids,
                                              device_scores=self.scores, stream=self.stream))
        torch.cuda.synchronize()
        self.plans[0].submit()
        torch.cuda.synchronize()
        self.expected = self.y.clone()
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph, stream=self.stream):
            for p in self.plans:
                p.submit()
        torch.cuda.synchronize()

    check = Rotation.check
    partial = Rotation.partial

    def close(self):
        del self.graph
        self.__dict__.pop("_partials", None)
        for p in self.plans:
            p.destroy()
        for w in self.weights:
            w.destroy()


def bench_moe(ctx, steps, warmup, seed):
    """C5: 64 experts (gate/up 4096 -> 1536, down 1536 -> 4096, K2), 8 tokens, top-8."""
    E, I, H, K, R, k = 64, 4096, 1536, 2, 8, 8
    rot = MoeRotation(ctx, E, I, H, K, R, k, seed)
    try:
        t = time_rotation(rot, steps, warmup)
    finally:
        rot.close()
    gbps = rot.packed / (t["ms"] * 1e-3) / 1e9
    per = (2 * I * H + H * I) * K // 8
    gu, dn = rot.distinct * per * 2 // 3, rot.distinct * per // 3
    return {"experts": E, "I": I, "H": H, "K": K, "rows": R, "top_k": k, "distinct_experts": rot.distinct,
            "packed_bytes": rot.packed, "us": round(t["ms"] * 1e3, 2),
            "median_pass_us": round(t["median_pass_ms"] * 1e3, 2), "passes": t["passes"],
            "packed_GBps": round(gbps, 1), "pct_hbm_peak": round(100 * gbps / HBM_PEAK_GBPS, 1),
            **floor_fields(ctx, t["ms"] * 1e3, rot.packed, [gu, dn]),
            "call_floor_launches": "gate/up bytes, then down bytes, each in its fastest shape", "launches": 3,
            "rotation_copies": rot.copies, "timed_steps": t["timed_steps"],
            "replay_matches_eager": t["output_check"]}


def cpu_baseline(sample_seconds=12.0):
    """NumPy oracle (decode + staged FP32 layer) on the north-star layer, host cores.

    Phases timed separately: (i) vectorized decode of the packed layer, (ii)
    the staged FP32 path from x to y given the decoded weights -- together the
    reported rate; NumPy's elementwise work runs on one thread -- and (iii) the
    FP64 algebraic product with a BLAS matmul, on all of BLAS's threads and on
    one.
    """
    import numpy as np
    import synth
    from oracle import codec, linear
    I = N = 4096
    K = 4
    tr, suh, svh, _ = synth.layer(I, N, K, synth.BASE_SEED)
    x = synth.activations(1, I, synth.BASE_SEED + 1)
    dec, stg = [], []
    t0 = time.perf_counter()
    while True:
        a = time.perf_counter()
        q = codec.dequantize_rotated(tr, K)
        b = time.perf_counter()
        linear.matmul_fp32_stages(x, tr, suh, svh, K, rotated=q)
        c = time.perf_counter()
        dec.append(b - a)
        stg.append(c - b)
        if c - t0 >= sample_seconds and len(dec) >= 5:
            break
    layer = statistics.median(d + s for d, s in zip(dec, stg))
    packed = I * N * K // 8

    def blas_ms():
        t = []
        for _ in range(5):
            a = time.perf_counter()
            linear.matmul(x, tr, suh, svh, K, rotated=q)
            t.append(time.perf_counter() - a)
        return round(statistics.median(t) * 1e3, 2)
    blas_threads, fp64_all, fp64_one = None, blas_ms(), None
    try:
        import threadpoolctl
        blas_threads = max((i.get("num_threads", 0) for i in threadpoolctl.threadpool_info()
                            if i.get("user_api") == "blas"), default=None)
        with threadpoolctl.threadpool_limits(1, user_api="blas"):
            fp64_one = blas_ms()
    except ImportError:
        pass
    return {"value": round(packed / layer / 1e9, 6), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"{len(dec)} full R1 K4 mul1 4096x4096 layers (vectorized decode + staged FP32 path), "
                      f"median {layer * 1e3:.0f} ms per layer",
            "decode_ms": round(statistics.median(dec) * 1e3, 1), "staged_ms": round(statistics.median(stg) * 1e3, 1),
            "us_per_call": round(layer * 1e6, 1), "cpu_model": _cpu_model(), "os_cpu_count": os.cpu_count(),
            "fp64_blas_ms": fp64_all, "fp64_blas_ms_1_thread": fp64_one, "blas_threads": blas_threads}


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _traffic():
    """HBM bytes per headline launch from the committed rocprofv3 --pmc passes, if present."""
    try:
        t = json.loads(TRAFFIC_FILE.read_text())
        return t.get(HEADLINE_KERNEL, {}).get("hbm_bytes_per_launch")
    except (OSError, ValueError):
        return None


def pmc_workload(ctx, launches, which="gemv"):
    """Fixed workload for counter passes, launched directly (no graph).

    gemv: the headline plan over its rotation, then the read-only call-floor
    kernel over 512 MiB (two launches, 1024 workgroups) and a plain 256 MiB
    device copy, whose FETCH_SIZE / WRITE_SIZE calibrate the counters against
    known bytes.  gemm: the M = 2048, 4096 -> 12288 K4 prefill plan.  moe: the
    C5 routed-expert plan."""
    import torch
    import synth
    if which == "moe":
        rot = MoeRotation(ctx, 64, 4096, 1536, 2, 8, 8, synth.BASE_SEED + 4)
    elif which == "gemm":
        rot = Rotation(ctx, 4096, 12288, 4, 2048, synth.BASE_SEED + 2, "gemm")
    else:
        rot = Rotation(ctx, 4096, 4096, 4, 1, synth.BASE_SEED, "gemv")
    for i in range(launches):
        rot.plans[i % rot.copies].submit()
    torch.cuda.synchronize()
    ok = rot.check()
    rot.close()
    if which != "gemv":
        log(f"pmc workload {which}: {launches} launches (replay_matches_eager={ok})")
        return
    from strix_trellis import runtime
    big = torch.empty(128 << 20, dtype=torch.float32, device="cuda:0").fill_(1.0)
    sink = torch.empty(1024, dtype=torch.int32, device="cuda:0")
    for _ in range(2):
        runtime.stream_read(ctx, big, big.numel() * 4, 1024, sink)
    src = torch.empty(64 << 20, dtype=torch.float32, device="cuda:0").fill_(1.0)
    dst = torch.empty_like(src)
    for _ in range(4):
        dst.copy_(src)
    torch.cuda.synchronize()
    log(f"pmc workload: {launches} headline launches (replay_matches_eager={ok}), 2 reads of {big.numel() * 4} "
        f"bytes, 4 copies of {src.numel() * 4} bytes")


STAGE_PHASES = ("mfma_decode", "store_issue", "a_wait", "barrier")
CLOCK_LIB = ROOT / "strix-trellis_amd" / "strix_trellis" / "_native" / "libstrix_trellis_clock.so"


def stage_clock(ctx, cells):
    """Per-stage phase cycles of the wide GEMM kernel from the instrumented
    library (build.py --stage-clock; main() points the loader at it).

    Each cell (M, I, N, K) is called directly six times; the records of the
    last call are summarised: per kind of work item (whole tile, handoff head,
    handoff tail), the mean cycles per K stage of each loop phase, the
    prologue and epilogue, and the shader clock (s_memtime cycles over
    s_memrealtime at 100 MHz).  Prints one JSON line per cell."""
    import ctypes as C
    import numpy as np
    import torch
    import synth
    from strix_trellis import abi, runtime
    lib = abi.load()
    if not hasattr(lib, "strix_amd_debug_stage_clock"):
        raise RuntimeError(f"the loaded library is not {CLOCK_LIB.name}; run strix-trellis_amd/build.py --stage-clock")
    rec = torch.zeros(8192 * 8 * 16, dtype=torch.int64, device="cuda:0")
    lib.strix_amd_debug_stage_clock(C.c_void_p(rec.data_ptr()))
    kinds = {0: "whole", 1: "head", 2: "tail"}
    for (M, I, N, K) in cells:
        tr, suh, svh, _ = synth.layer(I, N, K, synth.BASE_SEED + 2)
        w = runtime.Weights(ctx, tr, suh, svh, None, "mul1")
        x = torch.from_numpy(synth.activations(M, I, synth.BASE_SEED + 102)).to("cuda:0")
        y = torch.empty((M, N), device="cuda:0")
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
        for _ in range(6):
            rec.zero_()
            ev[0].record()
            runtime.gemm(w, x, y)
            ev[1].record()
        torch.cuda.synchronize()
        d = rec.view(-1, 16).cpu().numpy().astype(np.float64)
        d = d[d[:, 10] > 0]                       # waves that ran K stages
        st = d[:, 10]
        ghz = (d[:, 8] - d[:, 6]) / ((d[:, 9] - d[:, 7]) * 10.0)
        rt0 = d[:, 7].min()
        beg, end = (d[:, 7] - rt0) / 100.0, (d[:, 9] - rt0) / 100.0
        cell = {"M": M, "I": I, "N": N, "K": K, "call_us": round(ev[0].elapsed_time(ev[1]) * 1e3, 2),
                "workgroups": int(len(d) // 8), "clock_ghz_p10_p50_p90": [round(float(np.percentile(ghz, q)), 2)
                                                                           for q in (10, 50, 90)],
                "last_end_us": round(float(end.max()), 1), "items": {}}
        low = np.arange(len(d)) % 8 < 4           # waves 0..3, one per SIMD; 4..7 share the SIMDs

        def phase_mean(sel, i):
            return round(float((d[sel, i] / st[sel]).mean()))

        for kind, name in kinds.items():
            m = d[:, 11] == kind
            if not m.any():
                continue
            per = {ph: phase_mean(m, i) for i, ph in enumerate(STAGE_PHASES)}
            per["loop"] = int(sum(per[ph] for ph in STAGE_PHASES))
            cell["items"][name] = {
                "workgroups": int(m.sum() // 8), "stages": round(float(st[m].mean()), 1),
                "cycles_per_stage": per,
                "cycles_per_stage_waves_0_3_4_7": {ph: [phase_mean(m & low, i), phase_mean(m & ~low, i)]
                                                   for i, ph in enumerate(STAGE_PHASES)},
                "prologue_cycles": round(float(d[m, 4].mean())), "epilogue_cycles": round(float(d[m, 5].mean())),
                "duration_us": round(float((end - beg)[m].mean()), 1)}
        print(json.dumps(cell), flush=True)
        w.destroy()
    lib.strix_amd_debug_stage_clock(None)


def run_section(ctx, which, steps, warmup):
    """One section of the default run with the same cells and step counts."""
    import synth
    small_steps, small_warm = max(256, steps // 8), max(32, warmup // 8)
    cells = []
    if which == "gemv":
        cells.append(bench_gemv(ctx, 4096, 4096, 4, 1, steps, warmup, synth.BASE_SEED))
        for (I, N) in ((5120, 5120), (4096, 12288)):
            for K in (4, 5, 6):
                for R in (1, 2, 4, 8):
                    cells.append(bench_gemv(ctx, I, N, K, R, small_steps, small_warm, synth.BASE_SEED + 1))
    elif which == "gemm":
        for (I, N) in ((4096, 12288), (5120, 5120)):
            for K in (4, 5, 6):
                for M in (128, 512, 2048):
                    cells.append(bench_gemm(ctx, M, I, N, K, 48, 8, synth.BASE_SEED + 2))
    elif which == "grouped":
        for R in range(1, 9):
            for fold in (1, 2):
                cells.append(bench_grouped(ctx, 16, 4096, 1024, 5, R, small_steps, small_warm, synth.BASE_SEED + 3,
                                           fold))
    else:
        cells.append(bench_moe(ctx, max(64, steps // 32), max(8, warmup // 32), synth.BASE_SEED + 4))
    for c in cells:
        print(json.dumps(c), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=4096)
    ap.add_argument("--warmup", type=int, default=512)
    ap.add_argument("--quick", action="store_true", help="headline only (no sweeps)")
    ap.add_argument("--only", choices=("gemv", "gemm", "grouped", "moe"), default=None,
                    help="run one section (for profiling); prints that section's cells only")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--pmc-workload", nargs="?", const="gemv", choices=("gemv", "gemm", "moe"), default=None)
    ap.add_argument("--stage-clock", action="store_true",
                    help="per-stage phase cycles of the M = 2048 GEMMs (instrumented library)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (every box here has one MI355X); --gpus {args.gpus} "
              "is not supported", file=sys.stderr)
        sys.exit(2)

    if args.stage_clock:
        os.environ["STRIX_TRELLIS_LIB"] = str(CLOCK_LIB)
    import torch
    from strix_trellis import runtime
    import synth
    ctx = runtime.Context(0)
    props = torch.cuda.get_device_properties(0)
    log(f"device {props.name} {getattr(props, 'gcnArchName', '')} CUs={props.multi_processor_count}")
    if args.stage_clock:
        stage_clock(ctx, ((2048, 4096, 12288, 4), (2048, 5120, 5120, 4)))
        return
    if args.pmc_workload:
        pmc_workload(ctx, {"gemv": 256, "gemm": 16, "moe": 16}[args.pmc_workload], args.pmc_workload)
        return

    if args.only:
        run_section(ctx, args.only, args.steps, args.warmup)
        return

    # The read ceiling first: a second of full-bandwidth reads also brings the
    # GPU to its sustained clocks before the headline.
    ceil = read_ceiling(ctx)
    log(f"read ceiling: {json.dumps(ceil)}")
    log("headline: GEMV R1 K4 4096x4096")
    head = bench_gemv(ctx, 4096, 4096, 4, 1, args.steps, args.warmup, synth.BASE_SEED, oracle=True)
    log(json.dumps(head))
    small_steps, small_warm = max(256, args.steps // 8), max(32, args.warmup // 8)
    sweep, gemm, grouped, moe_cell = [], [], [], None
    if not args.quick:
        for (I, N) in ((5120, 5120), (4096, 12288)):
            for K in (4, 5, 6):
                for R in (1, 2, 4, 8):
                    cell = bench_gemv(ctx, I, N, K, R, small_steps, small_warm, synth.BASE_SEED + 1)
                    log(json.dumps(cell))
                    sweep.append(cell)
        for (I, N) in ((4096, 12288), (5120, 5120)):
            for K in (4, 5, 6):
                for M in (128, 512, 2048):
                    cell = bench_gemm(ctx, M, I, N, K, 48, 8, synth.BASE_SEED + 2)
                    log(json.dumps(cell))
                    gemm.append(cell)
        for R in range(1, 9):
            for fold in (1, 2):
                cell = bench_grouped(ctx, 16, 4096, 1024, 5, R, small_steps, small_warm, synth.BASE_SEED + 3, fold)
                log(json.dumps(cell))
                grouped.append(cell)
        moe_cell = bench_moe(ctx, max(64, args.steps // 32), max(8, args.warmup // 32), synth.BASE_SEED + 4)
        log(json.dumps(moe_cell))
    cpu = None if args.no_cpu else cpu_baseline()
    if cpu:
        log(json.dumps(cpu))
    ms = head["us"] / 1e3
    achieved = head["packed_GBps"]
    out = {
        "metric": METRIC,
        "value": head["packed_GBps"],
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": head["timed_steps"],
        "warmup": args.warmup,
        "ms_per_step": round(ms, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u16 trellis decode -> fp16 operands, f32 accumulation",
        "data": f"synthetic: PCG64 seed {synth.BASE_SEED} (+ config index) trellis/suh/svh/x per BASELINE configs",
        "config": {"workload": "decode GEMV R1, EXL3 K4 mul1, I=N=4096, prepared single-launch plan, "
                               f"cold rotation over {head['rotation_copies']} weight copies (>=1 GiB)",
                   "us_per_call": head["us"], "median_pass_us": head["median_pass_us"], "passes": head["passes"],
                   "warmup_launches": head["warmup_launches"],
                   "pct_hbm_peak": head["pct_hbm_peak"], "pct_read_ceiling": head["pct_read_ceiling"],
                   "replay_matches_eager": head["replay_matches_eager"],
                   "oracle_pass": head["oracle_pass"], "oracle_maxabs": head["oracle_maxabs"],
                   "oracle_nrmse": head["oracle_nrmse"],
                   "call_floor_us": head["call_floor_us"], "call_floor_shape": head["call_floor_shape"],
                   "pct_call_floor": head["pct_call_floor"], "read_ceiling_GBps": ceil["GBps"],
                   "fp16_library_us": head["fp16_library_us"],
                   "speedup_vs_fp16_library": head["speedup_vs_fp16_library"]},
        "oracle_pass": head["oracle_pass"],
        "oracle_maxabs": head["oracle_maxabs"],
        "oracle_nrmse": head["oracle_nrmse"],
        "oracle_gate": head.get("oracle_gate"),
        "median_pass_us": head["median_pass_us"],
        "read_ceiling": ceil,
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": _traffic(),
                     "kernel": HEADLINE_KERNEL, "algorithmic_bytes_per_launch": 4096 * 4096 * 4 // 8,
                     "launch_us": head["us"], "median_pass_us": head["median_pass_us"],
                     "read_ceiling_GBps": ceil["GBps"],
                     "frac_of_read_ceiling": round(achieved / ceil["GBps"], 4),
                     "call_floor_us": head["call_floor_us"]},
        "cpu_baseline": cpu,
        "sweep_gemv": sweep,
        "sweep_gemm": gemm,
        "grouped_o_a": grouped,
        "moe_k2": moe_cell,
    }
    if gemm:
        best, lib = {}, {}
        for c in gemm:
            if c["M"] == 2048:
                best[f"{c['I']}x{c['N']} K{c['K']}"] = c["pct_fp16_peak"]
                lib[f"{c['I']}x{c['N']}"] = c["fp16_library_pct_peak"]
        out["prefill_m2048_pct_fp16_peak"] = best
        out["prefill_m2048_fp16_library_pct_peak"] = lib
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
