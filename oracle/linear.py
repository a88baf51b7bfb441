"""EXL3 linear-layer oracle: FP64 algebra and the staged FP32 contract.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Restates python/strix_trellis/linear.py and docs/NUMERICS.md:30-126:

    W = diag(suh) H_I Q H_O diag(svh);   Y = ((X*suh) H_I) Q H_O * svh + bias

Staged FP32 production contract (every op IEEE RNE, no FMA, no FTZ):

    scaled_fp32         = RN32(RN32(X) * f32(RN16(suh)))
    scaled_fp16         = RN16(scaled_fp32)
    input_hadamard_fp32 = H32(scaled_fp16)
    core_input_fp16     = RN16(input_hadamard_fp32)
    core_fp32           = sum_i A_i * Q_io   (FP32, i ascending, from +0)
    output_hadamard     = H32(core_fp32)
    scaled_output_fp32  = RN32(output_hadamard * f32(RN16(svh)))
    output_fp32         = scaled_output_fp32 [+ RN32(bias)]

H32 = Sylvester butterflies with strides 1, 2, ..., 64 (each add/sub RN32),
then one multiply by RN32(1/sqrt(128)).

The library's operator additionally applies ``alpha`` / ``beta`` after the
bias (include/strix_trellis.h:147-154; reference src/transforms.hpp:44-49):
``y = RN32(output_fp32 * alpha)`` and, only when ``beta != 0``,
``y = RN32(y + RN32(beta * old))`` -- ``apply_alpha_beta`` below.

Parity pinning (tests/test_oracle_linear.py): prescale regression 0x1D6A of
tests/test_numerics.py:46-54; impulse Hadamards equal to the parity matrix
times RN32(1/sqrt(128)) bitwise; half ties and subnormals; the fixed-order
core example of test_numerics.py:115-126; gamma bounds; the explicit dense
matrix algebra of test_reference.py:135-150.
"""
import numpy as np

from .codec import dequantize_rotated

INV_SQRT128_F32 = np.float32(1.0 / np.sqrt(128.0))


def _finite(values, dtype, name):
    raw = np.asarray(values)
    if raw.dtype.kind not in "fiu" or not np.isfinite(raw).all():
        raise ValueError(f"{name} must contain finite real numbers")
    with np.errstate(over="ignore", invalid="ignore"):
        out = raw.astype(dtype)
    if not np.isfinite(out).all():
        raise ValueError(f"{name} overflows {np.dtype(dtype).name}")
    return out


def _finite_stage(values, name):
    if not np.isfinite(values).all():
        raise ValueError(f"Nonfinite result at {name}")
    return values


def _butterflies(blocks, size):
    """In-place ascending-stride Sylvester butterflies on [-1, size] rows."""
    stride = 1
    while stride < size:
        view = blocks.reshape(blocks.shape[0], size // (2 * stride), 2, stride)
        a = view[:, :, 0, :].copy()
        b = view[:, :, 1, :].copy()
        view[:, :, 0, :] = a + b
        view[:, :, 1, :] = a - b
        stride *= 2
    return blocks


def _check_block(block_size):
    if (isinstance(block_size, bool) or not isinstance(block_size, int)
            or block_size <= 0 or block_size & (block_size - 1)):
        raise ValueError("block_size must be a positive power of two")


def hadamard(values, block_size=128, axis=-1):
    """Normalized block Sylvester Hadamard in FP64 (linear.py:7-29)."""
    _check_block(block_size)
    data = np.asarray(values, dtype=np.float64)
    if data.ndim == 0 or not -data.ndim <= axis < data.ndim:
        raise ValueError("Invalid transform axis")
    data = np.moveaxis(data, axis, -1).copy()
    if data.shape[-1] % block_size:
        raise ValueError("Transform dimension must be divisible by block_size")
    shape = data.shape
    blocks = _butterflies(data.reshape(-1, block_size), block_size)
    blocks /= np.sqrt(block_size)
    return np.moveaxis(blocks.reshape(shape), -1, axis)


def hadamard_fp32(values, block_size=128, axis=-1):
    """H32: FP32 ascending-stride butterflies, then x RN32(1/sqrt(n)) (linear.py:82-108)."""
    _check_block(block_size)
    data = _finite(values, np.float32, "Hadamard input")
    if data.ndim == 0 or not -data.ndim <= axis < data.ndim:
        raise ValueError("Invalid transform axis")
    data = np.moveaxis(data, axis, -1).copy()
    if not data.shape[-1] or data.shape[-1] % block_size:
        raise ValueError("Transform dimension must be positive and divisible by block_size")
    shape = data.shape
    with np.errstate(over="ignore", invalid="ignore"):
        blocks = _butterflies(data.reshape(-1, block_size), block_size)
        _finite_stage(blocks, "Hadamard butterfly")
        blocks *= np.float32(1.0 / np.sqrt(block_size))
    return np.moveaxis(_finite_stage(blocks.reshape(shape), "Hadamard normalization"), -1, axis)


def input_stages_fp32(x, suh):
    """First five checkpoints of the FP32 contract (linear.py:111-124)."""
    xf = _finite(x, np.float32, "Input")
    u = _finite(suh, np.float16, "suh")
    if xf.ndim < 1 or u.shape != (xf.shape[-1],):
        raise ValueError("suh must match input last dimension")
    with np.errstate(over="ignore", invalid="ignore"):
        scaled = _finite_stage(xf * u.astype(np.float32), "input scale")
    scaled16 = _finite(scaled, np.float16, "Scaled input")
    had = hadamard_fp32(scaled16)
    a16 = _finite(had, np.float16, "Input Hadamard")
    return {"x_fp32": xf, "scaled_fp32": scaled, "scaled_fp16": scaled16,
            "input_hadamard_fp32": had, "core_input_fp16": a16}


def core_dot_fp32(core_input, rotated):
    """FP16 operands, FP32 mul then add, i ascending from +0 (linear.py:127-143)."""
    a = _finite(core_input, np.float16, "Core input").astype(np.float32)
    q = _finite(rotated, np.float16, "Rotated weights").astype(np.float32)
    if a.ndim < 1 or q.ndim != 2 or not q.shape[0] or not q.shape[1] or a.shape[-1] != q.shape[0]:
        raise ValueError("Core shapes must be [..., input] and [input, output]")
    acc = np.zeros(a.shape[:-1] + (q.shape[1],), dtype=np.float32)
    with np.errstate(over="ignore", invalid="ignore"):
        for i in range(q.shape[0]):
            acc += a[..., i, None] * q[i]
    return _finite_stage(acc, "core accumulation")


def output_stages_fp32(core, svh, bias=None):
    """H32, x f32(svh), + bias (linear.py:146-163)."""
    c = _finite(core, np.float32, "Core output")
    v = _finite(svh, np.float16, "svh")
    if c.ndim < 1 or v.shape != (c.shape[-1],):
        raise ValueError("svh must match output last dimension")
    had = hadamard_fp32(c)
    with np.errstate(over="ignore", invalid="ignore"):
        scaled = _finite_stage(had * v.astype(np.float32), "output scale")
    out = scaled.copy()
    if bias is not None:
        b = _finite(bias, np.float32, "Bias")
        if b.shape != v.shape:
            raise ValueError("Bias must match output dimension")
        with np.errstate(over="ignore", invalid="ignore"):
            out = _finite_stage(out + b, "bias addition")
    return {"output_hadamard_fp32": had, "scaled_output_fp32": scaled, "output_fp32": out}


def matmul_fp32_stages(x, trellis, suh, svh, k=None, codebook="mul1", bias=None, rotated=None):
    """All checkpoints of the staged contract (linear.py:166-175).

    ``rotated`` may pass an already decoded Q to skip the decode.
    """
    q = dequantize_rotated(trellis, k, codebook) if rotated is None else rotated
    stages = input_stages_fp32(x, suh)
    if stages["core_input_fp16"].shape[-1] != q.shape[0]:
        raise ValueError("Input last dimension must match trellis input dimension")
    stages["rotated_fp16"] = q
    stages["core_fp32"] = core_dot_fp32(stages["core_input_fp16"], q)
    stages.update(output_stages_fp32(stages["core_fp32"], svh, bias))
    return stages


def matmul_fp32(x, trellis, suh, svh, k=None, codebook="mul1", bias=None):
    """``output_fp32`` of the staged contract (linear.py:178-180)."""
    return matmul_fp32_stages(x, trellis, suh, svh, k, codebook, bias)["output_fp32"]


def apply_alpha_beta(linear_out, old, alpha, beta):
    """Operator epilogue: RN32(lin*alpha), then + RN32(beta*old) iff beta != 0."""
    y = (np.asarray(linear_out, dtype=np.float32) * np.float32(alpha)).astype(np.float32)
    if beta != 0:
        y = (y + (np.asarray(old, dtype=np.float32) * np.float32(beta)).astype(np.float32)).astype(np.float32)
    return y


def _scales(suh, svh, shape):
    left = np.asarray(suh, dtype=np.float64)
    right = np.asarray(svh, dtype=np.float64)
    if left.shape != (shape[0],) or right.shape != (shape[1],):
        raise ValueError("Scale vectors must match input/output dimensions")
    if not np.isfinite(left).all() or not np.isfinite(right).all():
        raise ValueError("Scale vectors must be finite")
    return left, right


def reconstruct_weight(trellis, suh, svh, k=None, codebook="mul1"):
    """W = diag(suh) H Q H diag(svh) in FP64 (linear.py:41-46)."""
    q = dequantize_rotated(trellis, k, codebook).astype(np.float64)
    left, right = _scales(suh, svh, q.shape)
    return left[:, None] * hadamard(hadamard(q, axis=0), axis=1) * right[None, :]


def matmul(x, trellis, suh, svh, k=None, codebook="mul1", bias=None, rotated=None):
    """FP64 algebraic layer without forming W (linear.py:49-62)."""
    q = (dequantize_rotated(trellis, k, codebook) if rotated is None else rotated).astype(np.float64)
    left, right = _scales(suh, svh, q.shape)
    xs = np.asarray(x, dtype=np.float64)
    if xs.ndim < 1 or xs.shape[-1] != q.shape[0]:
        raise ValueError("Input last dimension must match trellis input dimension")
    out = hadamard(hadamard(xs * left) @ q) * right
    if bias is not None:
        b = np.asarray(bias, dtype=np.float64)
        if b.shape != right.shape:
            raise ValueError("Bias must match output dimension")
        out = out + b
    return out


def core_exact_f64(core_input_fp16, rotated_fp16):
    """Exact-operand FP64 product A @ Q used for the core tolerance checks."""
    return np.asarray(core_input_fp16, dtype=np.float64) @ np.asarray(rotated_fp16, dtype=np.float64)


def gamma_bound(core_input_fp16, rotated_fp16, terms_factor=2):
    """gamma_{2I} * (|A| @ |Q|): per-output bound of NUMERICS.md:101-108."""
    a = np.abs(np.asarray(core_input_fp16, dtype=np.float64))
    q = np.abs(np.asarray(rotated_fp16, dtype=np.float64))
    n = terms_factor * q.shape[0]
    u = 2.0 ** -24
    return (n * u / (1 - n * u)) * (a @ q)
