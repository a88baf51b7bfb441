"""Pins the staged FP32 / FP64 layer oracle against the reference's known answers."""
import numpy as np
import pytest

from oracle import codec, linear


def parity_matrix(n):
    return np.array([[1 if bin(i & j).count("1") % 2 == 0 else -1 for j in range(n)]
                     for i in range(n)], dtype=np.float64)


def test_prescale_double_rounding_regression():
    # tests/test_numerics.py:46-54: RN16(RN32(x*s)) = 0x1D6A, while the direct
    # RN16 of the exact product is 0x1D6B.
    x = np.zeros(128, dtype=np.float32)
    s = np.ones(128, dtype=np.float16)
    x[0] = np.float32(0.2001299113035202)
    s[0] = np.float16(0.02642822265625)
    st = linear.input_stages_fp32(x, s)["scaled_fp16"]
    assert int(st.view(np.uint16)[0]) == 0x1D6A
    assert int(np.float16(float(x[0]) * float(s[0])).view(np.uint16)) == 0x1D6B


def test_hadamard_impulses_are_parity_matrix_exactly():
    # tests/test_numerics.py:89-96.
    x = np.eye(128, dtype=np.float32)
    np.testing.assert_array_equal(linear.hadamard_fp32(x),
                                  parity_matrix(128).astype(np.float32) * np.float32(1 / np.sqrt(128)))
    blocks = np.concatenate([x, np.zeros_like(x)], axis=1)
    np.testing.assert_array_equal(linear.hadamard_fp32(blocks)[:, 128:], 0)
    np.testing.assert_array_equal(linear.hadamard_fp32(blocks.T, axis=0), linear.hadamard_fp32(blocks).T)


def test_hadamard_fp64_matches_dense_and_involution():
    # tests/test_reference.py:125-133.
    rng = np.random.default_rng(45)
    for n in (1, 2, 8, 128):
        x = rng.normal(size=(3, 2 * n))
        dense = parity_matrix(n) / np.sqrt(n)
        np.testing.assert_allclose(linear.hadamard(x, n), (x.reshape(3, 2, n) @ dense).reshape(x.shape), atol=2e-14)
        np.testing.assert_allclose(linear.hadamard(linear.hadamard(x, n), n), x, atol=2e-14)


def test_hadamard_fp32_butterfly_order_fixed():
    # The FP32 result must equal an explicit scalar butterfly in ascending stride
    # (catches a reversed stride order, which differs in the last bits).
    rng = np.random.default_rng(3)
    x = rng.normal(size=128).astype(np.float32)
    v = [np.float32(t) for t in x]
    stride = 1
    while stride < 128:
        for base in range(0, 128, 2 * stride):
            for i in range(base, base + stride):
                a, b = v[i], v[i + stride]
                v[i], v[i + stride] = np.float32(a + b), np.float32(a - b)
        stride *= 2
    expected = np.array(v, dtype=np.float32) * np.float32(1 / np.sqrt(128))
    np.testing.assert_array_equal(linear.hadamard_fp32(x), expected)
    rev = x.copy()
    stride = 64
    while stride >= 1:
        view = rev.reshape(-1, 2, stride)
        a, b = view[:, 0].copy(), view[:, 1].copy()
        view[:, 0], view[:, 1] = a + b, a - b
        stride //= 2
    rev *= np.float32(1 / np.sqrt(128))
    assert np.any(rev != expected)  # the order is observable


def test_half_boundaries_ties_subnormals_signed_scales():
    # tests/test_numerics.py:98-113.
    x = np.zeros(128, dtype=np.float32)
    x[:6] = [1 + 2**-11, 1 + 3 * 2**-11, 2**-24, 2**-25, 1.0003, -3.25]
    s = np.ones(128, dtype=np.float16)
    s[4:7] = [-1.5, 0, 2]
    st = linear.input_stages_fp32(x, s)
    np.testing.assert_array_equal(st["scaled_fp32"], x * s.astype(np.float32))
    assert st["scaled_fp16"][0] == 1
    assert st["scaled_fp16"][1] == 1 + 2**-9
    assert st["scaled_fp16"][2] == 2**-24
    assert st["scaled_fp16"][3] == 0
    assert st["scaled_fp16"][5] == 0
    expected = st["scaled_fp16"].astype(np.float64) @ parity_matrix(128) / np.sqrt(128)
    np.testing.assert_allclose(st["input_hadamard_fp32"], expected, rtol=2e-6, atol=2e-7)
    np.testing.assert_array_equal(st["core_input_fp16"], st["input_hadamard_fp32"].astype(np.float16))


def test_core_fixed_order():
    # tests/test_numerics.py:115-126: 0.125 is absorbed by the FP32 partial sum.
    a = np.array([[2048, 1, 2048], [1, -2, 0.5]], dtype=np.float16)
    q = np.array([[2048, 2], [0.125, -3], [-2048, 4]], dtype=np.float16)
    got = linear.core_dot_fp32(a, q)
    assert got[0, 0] == 0
    np.testing.assert_array_equal(got[1], np.array([1 * 2048 + (-2) * 0.125 + 0.5 * -2048,
                                                     1 * 2 + (-2) * (-3) + 0.5 * 4], dtype=np.float32))


@pytest.mark.parametrize("shape", [(128, 256), (256, 128)])
def test_rectangular_layer_bounds_and_algebra(shape):
    # tests/test_numerics.py:128-155.
    inputs, outputs = shape
    rng = np.random.default_rng(220)
    packed = rng.integers(0, 65536, (inputs // 16, outputs // 16, 32), dtype=np.uint16)
    x = rng.normal(size=(2, 1, inputs)).astype(np.float32)
    left = rng.uniform(-2, 2, inputs).astype(np.float16)
    right = rng.uniform(-3, 3, outputs).astype(np.float16)
    left[::7], right[::5] = 0, 0
    bias = rng.normal(size=outputs).astype(np.float32)
    st = linear.matmul_fp32_stages(x, packed, left, right, bias=bias)
    a, q = st["core_input_fp16"], st["rotated_fp16"]
    exact = linear.core_exact_f64(a, q)
    assert np.all(np.abs(st["core_fp32"] - exact) <= linear.gamma_bound(a, q))
    h = parity_matrix(128) / np.sqrt(128)
    eh = (st["core_fp32"].astype(np.float64).reshape(-1, 128) @ h).reshape(2, 1, outputs)
    np.testing.assert_allclose(st["output_hadamard_fp32"], eh, rtol=2e-5, atol=1e-5)
    np.testing.assert_array_equal(st["scaled_output_fp32"], st["output_hadamard_fp32"] * right.astype(np.float32))
    np.testing.assert_array_equal(st["output_fp32"], st["scaled_output_fp32"] + bias)
    np.testing.assert_array_equal(st["output_fp32"][..., ::5], np.broadcast_to(bias[::5], (2, 1, len(bias[::5]))))


def test_fp64_dense_reconstruction_and_orientation():
    # tests/test_reference.py:135-150.
    rng = np.random.default_rng(41)
    packed = rng.integers(-32768, 32767, (8, 16, 32), dtype=np.int16)
    left = rng.normal(size=128)
    right = rng.normal(size=256)
    x = rng.normal(size=(2, 3, 128))
    bias = rng.normal(size=256)
    q = codec.dequantize_rotated(packed).astype(np.float64)
    hl = parity_matrix(128) / np.sqrt(128)
    hr = np.kron(np.eye(2), hl)
    dense = left[:, None] * (hl @ q @ hr) * right
    np.testing.assert_allclose(linear.reconstruct_weight(packed, left, right), dense, atol=2e-14)
    np.testing.assert_allclose(linear.matmul(x, packed, left, right, bias=bias), x @ dense + bias,
                               rtol=1e-12, atol=3e-13)


def test_staged_differs_from_fp64():
    # tests/test_numerics.py:157-163.
    packed = np.zeros((8, 8, 16), dtype=np.uint16)
    x = np.zeros(128, dtype=np.float32)
    x[0] = 1 + 2**-11
    staged = linear.matmul_fp32(x, packed, np.ones(128), np.ones(128))
    exact = linear.matmul(x, packed, np.ones(128), np.ones(128))
    assert np.max(np.abs(staged - exact)) > 1e-4


def test_alpha_beta_epilogue():
    lin = np.array([1.5, -2.0, 3.0], dtype=np.float32)
    old = np.array([np.nan, 4.0, 8.0], dtype=np.float32)
    np.testing.assert_array_equal(linear.apply_alpha_beta(lin, old, 1.0, 0.0)[1:], lin[1:])
    assert np.isfinite(linear.apply_alpha_beta(lin, old, 1.0, -0.0)).all()  # beta = -0 never reads old
    np.testing.assert_array_equal(linear.apply_alpha_beta(lin[1:], old[1:], -0.75, 0.25),
                                  np.float32(-0.75) * lin[1:] + np.float32(0.25) * old[1:])


def test_rejects_nonfinite_and_bad_shapes():
    for bad in (np.nan, np.inf, 1e100):
        x = np.ones(128)
        x[0] = bad
        with pytest.raises(ValueError):
            linear.input_stages_fp32(x, np.ones(128))
        with pytest.raises(ValueError):
            linear.output_stages_fp32(x, np.ones(128))
    with pytest.raises(ValueError):
        linear.input_stages_fp32(np.full(128, 65504), np.full(128, 2))
    with pytest.raises(ValueError):
        linear.core_dot_fp32(np.ones(2), np.ones((3, 4)))
