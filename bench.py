"""Benchmark of the EXL3 trellis hot path on one MI355X.

Headline (`value`): decode GEMV, R = 1, K4 mul1, I = N = 4096 (the north-star
configuration), through a prepared single-launch plan, as packed-weight GB/s
over a cold rotation of >= 1 GiB of distinct weight copies (more than 4x the
256 MB MALL), inputs resident in HBM.  One step = one GEMV call.

Also reported (same JSON line): the decode GEMV sweep of BASELINE configs[1]
(R = 1, 2, 4, 8 x {5120^2, 4096 -> 12288} x K4-6), `roofline` for the GEMV
kernel and `cpu_baseline` (the NumPy oracle on the host, bounded sample).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-sweep] [--no-cpu]
"""
import argparse
import json
import os
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


def log(msg):
    print(msg, file=sys.stderr, flush=True)


class Rotation:
    """Distinct device copies of one layer, each with its own prepared plan.

    One pass over the copies is captured into a HIP graph (one plan submission
    per copy) so that the timed region measures the GPU, not Python's launch
    rate.  The copies share x, y and the workspace (their calls are ordered on
    one stream).
    """

    def __init__(self, ctx, I, N, K, R, seed, op="gemv", min_bytes=ROTATION_BYTES):
        import torch
        import synth
        from strix_trellis import runtime
        tr, suh, svh, _ = synth.layer(I, N, K, seed)
        packed = I * N * K // 8
        self.copies = max(2, -(-min_bytes // packed))
        self.packed = packed
        self.stream = torch.cuda.Stream()
        self.x = torch.from_numpy(synth.activations(R, I, seed + 1)).to("cuda:0")
        self.y = torch.empty((R, N), device="cuda:0")
        self.weights, self.plans = [], []
        ws = None
        for _ in range(self.copies):
            w = runtime.Weights(ctx, tr, suh, svh, None, "mul1")
            if ws is None:
                ws = runtime.alloc_workspace(runtime.workspace_bytes(w, self.x, self.y), "cuda:0")
            self.weights.append(w)
            self.plans.append(runtime.LinearPlan(w, self.x, self.y, workspace=ws, stream=self.stream, operation=op))
        self.workspace = ws
        self.launches = self.plans[0].launches()
        torch.cuda.synchronize()
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph, stream=self.stream):
            for p in self.plans:
                p.submit()
        torch.cuda.synchronize()

    def run(self, steps, start=0):
        """Replay whole passes; `steps` is rounded up to a multiple of the copy count."""
        for _ in range(-(-steps // self.copies)):
            self.graph.replay()
        return -(-steps // self.copies) * self.copies

    def close(self):
        del self.graph
        for p in self.plans:
            p.destroy()
        for w in self.weights:
            w.destroy()


def time_steps(run, steps, warmup, stream):
    """HIP events on the stream the kernels run on; returns ms per step."""
    import torch
    run(warmup)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        start.record(stream)
        done = run(steps)
        end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) / done, done


def bench_gemv(ctx, I, N, K, R, steps, warmup, seed):
    rot = Rotation(ctx, I, N, K, R, seed, "gemv")
    try:
        ms, steps = time_steps(rot.run, steps, warmup, rot.stream)
    finally:
        rot.close()
    us = ms * 1e3
    gbps = rot.packed / (ms * 1e-3) / 1e9
    return {"I": I, "N": N, "K": K, "R": R, "us": round(us, 3), "packed_GBps": round(gbps, 1),
            "pct_hbm_peak": round(100 * gbps / HBM_PEAK_GBPS, 1), "launches": rot.launches,
            "rotation_copies": rot.copies, "timed_steps": steps}


def bench_gemm(ctx, M, I, N, K, steps, warmup, seed):
    rot = Rotation(ctx, I, N, K, M, seed, "gemm", min_bytes=ROTATION_BYTES // 4)
    try:
        ms, steps = time_steps(rot.run, steps, warmup, rot.stream)
    finally:
        rot.close()
    tflops = 2.0 * M * I * N / (ms * 1e-3) / 1e12
    return {"M": M, "I": I, "N": N, "K": K, "us": round(ms * 1e3, 2), "TFLOPs": round(tflops, 1),
            "pct_fp16_peak": round(100 * tflops / FP16_PEAK_TFLOPS, 1), "launches": rot.launches,
            "rotation_copies": rot.copies, "timed_steps": steps}


def cpu_baseline(sample_seconds=12.0):
    """NumPy oracle (decode + staged FP32 layer) on the north-star layer, host cores."""
    import numpy as np
    import synth
    from oracle import codec, linear
    I = N = 4096
    K = 4
    tr, suh, svh, _ = synth.layer(I, N, K, synth.BASE_SEED)
    x = synth.activations(1, I, synth.BASE_SEED + 1)
    runs, t0 = 0, time.perf_counter()
    while True:
        q = codec.dequantize_rotated(tr, K)
        linear.matmul_fp32_stages(x, tr, suh, svh, K, rotated=q)
        runs += 1
        if time.perf_counter() - t0 >= sample_seconds:
            break
    dt = (time.perf_counter() - t0) / runs
    packed = I * N * K // 8
    return {"value": round(packed / dt / 1e9, 6), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"{runs} full R1 K4 4096x4096 layers (vectorized decode + staged FP32 path), "
                      f"{dt * 1e3:.0f} ms each", "cpu_model": _cpu_model(), "os_cpu_count": os.cpu_count()}


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=4000)
    ap.add_argument("--warmup", type=int, default=400)
    ap.add_argument("--no-sweep", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (every box here has one MI355X); --gpus {args.gpus} "
              "is not supported", file=sys.stderr)
        sys.exit(2)

    import torch
    from strix_trellis import runtime
    import synth
    ctx = runtime.Context(0)
    props = torch.cuda.get_device_properties(0)
    log(f"device {props.name} {getattr(props, 'gcnArchName', '')} CUs={props.multi_processor_count}")

    log("headline: R1 K4 4096x4096")
    head = bench_gemv(ctx, 4096, 4096, 4, 1, args.steps, args.warmup, synth.BASE_SEED)
    log(json.dumps(head))
    sweep = []
    if not args.no_sweep:
        for (I, N) in ((5120, 5120), (4096, 12288)):
            for K in (4, 5, 6):
                for R in (1, 2, 4, 8):
                    cell = bench_gemv(ctx, I, N, K, R, max(200, args.steps // 8), max(20, args.warmup // 8),
                                      synth.BASE_SEED + 1)
                    log(json.dumps(cell))
                    sweep.append(cell)
    cpu = None if args.no_cpu else cpu_baseline()
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
        "dtype": "fp16 operands, f32 accumulation (K4 mul1 trellis)",
        "data": "synthetic: PCG64 seed 20261201 trellis/suh/svh/x per BASELINE configs",
        "config": {"workload": "decode GEMV R1, EXL3 K4 mul1, I=N=4096, prepared single-launch plan, "
                               f"cold rotation over {head['rotation_copies']} weight copies (>=1 GiB)",
                   "us_per_call": head["us"], "pct_hbm_peak": head["pct_hbm_peak"]},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": None,
                     "kernel": "stx::gemv_kernel<4,2,1>",
                     "algorithmic_bytes_per_launch": 4096 * 4096 * 4 // 8},
        "cpu_baseline": cpu,
        "sweep_gemv": sweep,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
