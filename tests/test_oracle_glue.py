"""Pins of the oracle's layer glue: RMSNorm (bnro_rms_norm, norm.rs:76-136),
absmax quantisation (bnro_absmax_quantize_row, absmax.rs:127-170) and the
squared-ReLU gate (bnro_sqrelu_gate, cpu/lib.rs:494-509).

Closed forms follow the reference's own tests (norm.rs:186-530,
absmax.rs:291-430); fp64 brute force bounds the RMSNorm rounding; the
quantiser is compared element-wise with an independent fp64 restatement
(round half away from zero)."""
import numpy as np
import pytest

import oracle

f32 = np.float32


def rms(x, w, eps=1e-5):
    x = np.asarray(x, f32)
    out = np.full(x.size, np.nan, f32)
    oracle.rms_norm(x, np.asarray(w, f32), eps, out)
    return out


def test_rms_norm_doc_example():  # norm.rs:62-74
    out = rms([1, 2, 3, 4], np.ones(4))
    assert out[0] == f32(1.0) / np.sqrt(f32(7.5) + f32(1e-5)).astype(f32)


def test_rms_norm_closed_forms():
    # zero input -> zero output (norm.rs:237); unit input -> ~1 (norm.rs:250)
    np.testing.assert_array_equal(rms(np.zeros(8), np.ones(8)), np.zeros(8))
    assert np.all(np.abs(rms(np.ones(64), np.ones(64)) - 1) < 1e-5)
    # scaled weight doubles output (norm.rs:214); sign preserved (norm.rs:291,307)
    x = np.arange(1, 17, dtype=f32)
    np.testing.assert_array_equal(rms(x, np.full(16, 2)), 2 * rms(x, np.ones(16)))
    assert np.all(rms(-x, np.ones(16)) < 0)
    o = rms([1, 1, 1], [1, -1, 1])
    assert o[0] > 0 and o[1] < 0 and o[2] > 0
    # single element: x / sqrt(x^2 + eps) (norm.rs:321)
    assert abs(rms([3.0], [1.0])[0] - 3 / np.sqrt(9 + 1e-5)) < 1e-6


@pytest.mark.parametrize("n", [1, 7, 8, 9, 2560, 6912, 10001])
def test_rms_norm_fp64_bound(n):
    rng = np.random.default_rng(n)
    x = (rng.standard_normal(n) * 3).astype(f32)
    w = rng.uniform(0.5, 1.5, n).astype(f32)
    got = rms(x, w).astype(np.float64)
    xd = x.astype(np.float64)
    exact = xd / np.sqrt(np.mean(xd * xd) + 1e-5) * w
    assert np.all(np.abs(got - exact) <= (n * 1e-7 + 4e-7) * np.abs(exact) + 1e-12)


def test_rms_norm_sum_order_avx2_vs_scalar():
    # the AVX2 path keeps 8 lane sums; the scalar fallback sums left to right
    x = np.array([f32(4096.0)] + [f32(0.0004)] * 15, f32)
    a = oracle.sum_squares(x)
    oracle.force_scalar(True)
    try:
        b = oracle.sum_squares(x)
    finally:
        oracle.force_scalar(False)
    lanes = [f32(x[i] * x[i] + x[i + 8] * x[i + 8]) for i in range(8)]  # fma of two terms
    lo, hi = lanes[:4], lanes[4:]
    s4 = [f32(lo[i] + hi[i]) for i in range(4)]
    assert a == f32(f32(s4[0] + s4[1]) + f32(s4[2] + s4[3]))
    seq = f32(0)
    for v in x:
        seq = f32(seq + f32(v * v))
    assert b == seq


def test_rms_norm_errors():
    with pytest.raises(oracle.InvalidShape, match=r"input.len\(\) == weight.len\(\) = 3, got input.len\(\) = 4"):
        oracle.rms_norm(np.zeros(4, f32), np.zeros(3, f32), 1e-5, np.zeros(4, f32))
    with pytest.raises(oracle.InvalidShape, match=r"input.len\(\) == output.len\(\) = 4"):
        oracle.rms_norm(np.zeros(4, f32), np.zeros(4, f32), 1e-5, np.zeros(5, f32))
    for eps, txt in [(0.0, "0"), (-1e-6, "-0.000001"), (float("nan"), "NaN")]:
        with pytest.raises(oracle.QuantizationError, match=f"eps must be finite and > 0, got {txt}$"):
            oracle.rms_norm(np.zeros(4, f32), np.zeros(4, f32), eps, np.zeros(4, f32))
    oracle.rms_norm(np.zeros(0, f32), np.zeros(0, f32), 1e-5, np.zeros(0, f32))  # empty: no-op


def quant_ref(x):
    x = np.asarray(x, f32)
    m = np.float32(max(np.max(np.abs(x)), f32(1e-5)))
    inv = f32(f32(127.0) / m)
    v = (x * inv).astype(np.float64)  # one f32 rounding of x * inv_scale
    r = np.where(v >= 0, np.floor(v + 0.5), np.ceil(v - 0.5))
    return np.clip(r, -128, 127).astype(np.int8), float(f32(m / f32(127.0)))


def test_absmax_closed_forms():  # absmax.rs:291-380
    q, s = oracle.absmax_quantize_row(np.array([0.5, -1.0, 2.0, -1.0], f32))
    assert q[2] == 127 and q[3] == -64 and s == float(f32(2.0) / f32(127.0))
    q, s = oracle.absmax_quantize_row(np.array([-3.0, 0.0, 1.5], f32))
    assert q.tolist() == [-127, 0, 64]
    q, s = oracle.absmax_quantize_row(np.zeros(5, f32))
    assert s > 0 and np.all(q == 0)
    assert oracle.absmax_quantize_row(np.array([5.0], f32))[0][0] == 127
    assert oracle.absmax_quantize_row(np.array([-4.0], f32))[0][0] == -127


@pytest.mark.parametrize("n", [1, 3, 2560, 6912])
def test_absmax_matches_independent_restatement(n):
    rng = np.random.default_rng(100 + n)
    x = (rng.standard_normal(n) * rng.uniform(0.01, 10)).astype(f32)
    x[rng.integers(0, n, size=max(1, n // 50))] = 0.5  # exercise halves
    q, s = oracle.absmax_quantize_row(x)
    qr, sr = quant_ref(x)
    np.testing.assert_array_equal(q, qr)
    assert s == sr


def test_absmax_errors():
    with pytest.raises(oracle.QuantizationError, match="cannot quantise an empty activation vector"):
        oracle.absmax_quantize_row(np.zeros(0, f32))
    with pytest.raises(oracle.QuantizationError, match="non-finite activation value at index 1: NaN"):
        oracle.absmax_quantize_row(np.array([0, np.nan, 1], f32))
    with pytest.raises(oracle.QuantizationError, match="non-finite activation value at index 0: -inf"):
        oracle.absmax_quantize_row(np.array([-np.inf], f32))


def test_sqrelu_gate():
    g = np.array([-2, -0.0, 0, 0.5, 3, np.nan], f32)
    u = np.array([5, 5, 5, 4, -2, 7], f32)
    out = np.full(6, np.nan, f32)
    oracle.sqrelu_gate(g, u, out)
    np.testing.assert_array_equal(out, [0, 0, 0, 1.0, -18.0, 0])
    with pytest.raises(oracle.InvalidShape, match=r"gate.len\(\) == up.len\(\) == out.len\(\) = 6"):
        oracle.sqrelu_gate(g, u[:5], out)
