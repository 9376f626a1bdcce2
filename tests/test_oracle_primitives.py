"""Pins of the oracle's dot / axpy / softmax (bitnet-cpu/src/simd.rs:292-307,
676-791; bitnet-core/src/backend/ops.rs:206-226).

The lane-order and FMA checks use inputs whose IEEE-754 results are worked
out by hand in the comments, so a wrong horizontal-sum order or an unfused
accumulation fails them."""
import numpy as np
import pytest

import oracle

f32 = np.float32


def test_dot_exact_small_integers():
    rng = np.random.default_rng(0)
    for n in [1, 7, 8, 9, 16, 128, 131]:
        a = rng.integers(-8, 8, n).astype(f32)
        b = rng.integers(-8, 8, n).astype(f32)
        assert oracle.dot(a, b) == float(np.dot(a.astype(np.int64), b.astype(np.int64)))


def test_dot_hsum_lane_order():
    # 8 lanes l = a*b = [2^24, -2^24, 0, 0, 1, 1, 0, 0].  The AVX2 horizontal sum
    # (simd.rs:292-307) is ((l0+l4)+(l1+l5)) + ((l2+l6)+(l3+l7)):
    #   l0+l4 = 2^24+1 -> ties-to-even 2^24;  l1+l5 = -2^24+1 (exact)
    #   2^24 + (1-2^24) = 1  -> result 1.0.
    # A left-to-right sum gives 2.0, the exact sum is 2.0.
    a = np.array([2.0**24, -2.0**24, 0, 0, 1, 1, 0, 0], f32)
    assert oracle.dot(a, np.ones(8, f32)) == 1.0
    oracle.force_scalar(True)
    try:
        assert oracle.dot(a, np.ones(8, f32)) == 2.0  # scalar fallback, simd.rs:724-731
    finally:
        oracle.force_scalar(False)


def test_dot_accumulates_with_fma():
    # Lane 0: chunk 0 gives -1, chunk 1 adds (1+2^-12)^2 = 1 + 2^-11 + 2^-24.
    # fmadd keeps the 2^-24 term: 2^-11 + 2^-24.  An unfused product rounds
    # 1+2^-11+2^-24 to 1+2^-11 (tie to even), leaving 2^-11.
    a = np.zeros(16, f32)
    b = np.zeros(16, f32)
    a[0], b[0] = -1.0, 1.0
    a[8] = b[8] = 1.0 + 2.0**-12
    assert oracle.dot(a, b) == 2.0**-11 + 2.0**-24


def test_dot_remainder_is_unfused_sequential():
    # n = 9: lanes give 0, remainder adds a[8]*b[8] unfused after the hsum.
    a = np.zeros(9, f32)
    b = np.zeros(9, f32)
    a[0], b[0] = -1.0, 1.0
    a[8] = b[8] = 1.0 + 2.0**-12
    assert oracle.dot(a, b) == 2.0**-11  # rounded product, then -1 + that


def test_axpy_fma_body_and_unfused_tail():
    x = np.full(9, 1.0 + 2.0**-12, f32)
    out = np.full(9, -1.0, f32)
    oracle.axpy(1.0 + 2.0**-12, x, out)
    assert np.all(out[:8] == f32(2.0**-11 + 2.0**-24))  # fmadd lanes
    assert out[8] == f32(2.0**-11)  # scalar remainder `out += alpha*x`


# --- ops.rs softmax tests (ops.rs:485-530) -----------------------------------

def test_softmax_sums_to_one():
    x = np.array([1, 2, 3, 4], f32)
    oracle.softmax(x)
    assert abs(x.sum() - 1.0) < 1e-6


def test_softmax_all_same_is_uniform():
    x = np.full(8, 0.5, f32)
    oracle.softmax(x)
    assert np.all(x == f32(0.125))  # exp(0)=1, sum 8, 1/8 exact


def test_softmax_large_value_dominates():
    x = np.array([0, 0, 100, 0], f32)
    oracle.softmax(x)
    assert x[2] > 0.999


def test_softmax_empty_noop():
    oracle.softmax(np.zeros(0, f32))


def test_softmax_matches_fp64():
    rng = np.random.default_rng(3)
    x = (rng.standard_normal(1000) * 5).astype(f32)
    ref = np.exp(x.astype(np.float64) - x.max())
    ref /= ref.sum()
    y = x.copy()
    oracle.softmax(y)
    np.testing.assert_allclose(y, ref, rtol=1e-5, atol=0)  # f32 sequential sum of 1000 terms


def test_softmax_subtracts_max():
    # Without the max shift exp(1000) overflows to inf and the result is NaN.
    x = np.array([1000.0, 999.0], f32)
    oracle.softmax(x)
    e = np.exp(-1.0)
    np.testing.assert_allclose(x, [1 / (1 + e), e / (1 + e)], rtol=1e-6)


def test_normal_generator_is_seeded_and_standard():
    a = oracle.normal(42, (100000,))
    b = oracle.normal(42, (100000,))
    np.testing.assert_array_equal(a, b)
    assert abs(a.mean()) < 0.02 and abs(a.std() - 1) < 0.02
    assert not np.array_equal(a, oracle.normal(43, (100000,)))
