"""Write the STGPU001 parity fixtures tests/golden/*.stgpu from the oracle.

Each case follows the reference's fixture recipe (docs/GPU_TESTS.md:22-35):
F16 scales with signs, zeros, negative zero and magnitudes 0.0625..2; odd bit
widths carry an F32 bias and even ones none; the first row holds asymmetric
impulses at lane and H128-block boundaries, the other rows are random.  Every
stage is the oracle's (oracle/linear.py, oracle/codec.py): scaled, inh and a
from the input stages, q from the vectorized decode, core from the scalar
ascending-I product and ref from the output stages.

    python tests/golden/make_stgpu.py        # rewrites the fixtures in place
"""
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path[:0] = [str(ROOT), str(ROOT / "strix-trellis_amd")]

from oracle import codec, linear  # noqa: E402
from strix_trellis.fixture import CODEBOOKS, MARKERS, write_stgpu  # noqa: E402

# (name, I, N, bits, codebook, rows, seed)
CASES = [
    ("k5_mul1_bias_256x128", 256, 128, 5, "mul1", 16, 11),
    ("k4_mcg_128x256", 128, 256, 4, "mcg", 16, 12),
    ("k2_3inst_128x128", 128, 128, 2, "3inst", 16, 13),
    ("k3_mul1_bias_128x256", 128, 256, 3, "mul1", 16, 14),
]


def scales(g, n):
    special = np.array([0.0, -0.0, 0.0625, -0.0625, 2.0, -2.0, 1.0, -0.5], dtype=np.float32)
    values = g.choice([-1.0, 1.0], n) * g.uniform(0.0625, 2.0, n)
    pick = g.random(n) < 0.125
    values[pick] = g.choice(special, int(pick.sum()))
    return values.astype(np.float16)


def case(I, N, K, codebook, rows, seed):
    g = np.random.Generator(np.random.PCG64(seed))
    trellis = g.integers(0, 65536, (I // 16, N // 16, 16 * K), dtype=np.uint16)
    suh, svh = scales(g, I), scales(g, N)
    bias = g.standard_normal(N).astype(np.float32) if K % 2 else None
    x = g.standard_normal((rows, I)).astype(np.float16).astype(np.float32)
    x[0] = 0.0
    for pos, v in zip((0, 63, 64, 127, 128 % I, I - 1), (1.0, -2.0, 0.5, 3.0, -0.25, 1.5)):
        x[0, pos] += v
    old = g.standard_normal((rows, N)).astype(np.float32)
    ins = linear.input_stages_fp32(x, suh)
    q = codec.dequantize_rotated(trellis, K, codebook)
    core = linear.core_dot_fp32(ins["core_input_fp16"], q)
    ref = linear.output_stages_fp32(core, svh, bias)["output_fp32"]
    meta = {"I": I, "N": N, "bits": K, "codebook": CODEBOOKS.index(codebook),
            "marker": MARKERS[CODEBOOKS.index(codebook)], "rows": rows, "bias": int(bias is not None), "seed": seed}
    arrays = {"trellis": trellis, "suh": suh, "svh": svh,
              "bias": bias if bias is not None else np.zeros(0, np.float32), "x": x, "old": old,
              "scaled": ins["scaled_fp16"], "inh": ins["input_hadamard_fp32"], "a": ins["core_input_fp16"],
              "q": q, "core": core, "ref": ref}
    return meta, arrays


def main():
    for name, I, N, K, codebook, rows, seed in CASES:
        meta, arrays = case(I, N, K, codebook, rows, seed)
        path = HERE / f"{name}.stgpu"
        write_stgpu(path, meta, arrays)
        print(f"{path.name}: {path.stat().st_size} bytes")


if __name__ == "__main__":
    main()
