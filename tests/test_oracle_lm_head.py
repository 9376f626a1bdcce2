"""Pins of the oracle's i8-weight LM head (bnro_lm_head_matmul_i8 /
bnro_dot_f32_i8w, restating CpuBackend::lm_head_matmul_i8_into,
bitnet-cpu/src/lib.rs:544-575, and simd::dot_f32_i8w_fast, simd.rs:1213-1269).

Closed forms with exactly representable sums, the order-specific rounding of
the AVX2 path (8 FMA lanes, hsum ((l0+h0)+(l1+h1))+((l2+h2)+(l3+h3)), unfused
tail) against hand-derived values, and an fp64 brute force bound."""
import numpy as np
import pytest

import oracle

f32 = np.float32


def lm(hidden, w, scales):
    v, h = w.shape
    out = np.full(v, np.nan, f32)
    oracle.lm_head_matmul_i8(np.ascontiguousarray(hidden, f32), w, np.ascontiguousarray(scales, f32),
                             out, v, h)
    return out


def test_closed_forms():
    h = np.arange(1, 20, dtype=f32)                   # 19: two 8-chunks + 3-element tail
    w = np.zeros((4, 19), np.int8)
    w[0, 0] = 1                                       # picks h[0]
    w[1, 18] = -1                                     # tail element
    w[2] = 1                                          # sum 1..19 = 190
    w[3, ::2] = 127                                   # 127 * (1+3+...+19) = 127*100
    out = lm(h, w, [1.0, 2.0, 0.5, 1.0])
    np.testing.assert_array_equal(out, [1.0, -38.0, 95.0, 12700.0])


def test_zero_and_empty():
    np.testing.assert_array_equal(lm(np.ones(16, f32), np.zeros((3, 16), np.int8), np.ones(3)), [0, 0, 0])
    np.testing.assert_array_equal(lm(np.zeros(0, f32), np.zeros((2, 0), np.int8), [3.0, 4.0]), [0, 0])


def test_avx2_lane_order():
    """Lane sums before the horizontal add: with h = [1e8, 1, 1, ... ] the
    AVX2 path keeps the small terms of other lanes apart from lane 0's 1e8
    until hsum; a sequential scalar sum would absorb them one at a time."""
    n = 16
    h = np.ones(n, f32)
    h[0] = f32(1e8)
    w = np.ones((1, n), np.int8)
    # lane 0: 1e8 + 1 (chunk 1) -> 1e8 (ulp 8); lanes 1..7: 2 each
    # hsum: ((1e8 + 2) + (2 + 2)) + ((2 + 2) + (2 + 2)) with f32 rounding
    a0 = f32(f32(1e8) + f32(1))
    l = [a0] + [f32(2)] * 7
    lo, hi = l[:4], l[4:]  # the high 128-bit half holds lanes 4..7
    s4 = [f32(lo[i] + hi[i]) for i in range(4)]
    expect = f32(f32(s4[0] + s4[1]) + f32(s4[2] + s4[3]))
    got = lm(h, w, [1.0])[0]
    assert got == expect
    oracle.force_scalar(True)
    try:
        scalar = lm(h, w, [1.0])[0]
    finally:
        oracle.force_scalar(False)
    seq = f32(0)
    for x in h:
        seq = f32(seq + x)
    assert scalar == seq


@pytest.mark.parametrize("v,h", [(7, 5), (33, 64), (100, 2560), (17, 2567)])
def test_brute_force_bound(v, h):
    rng = np.random.default_rng(v * 10000 + h)
    hid = rng.standard_normal(h).astype(f32)
    w = rng.integers(-128, 128, size=(v, h)).astype(np.int8)
    sc = rng.uniform(0.001, 0.05, size=v).astype(f32)
    got = lm(hid, w, sc).astype(np.float64)
    exact = (w.astype(np.float64) @ hid.astype(np.float64)) * sc.astype(np.float64)
    bound = 4 * h * np.finfo(f32).eps * (np.abs(w).astype(np.float64) @ np.abs(hid).astype(np.float64)) * sc + 1e-30
    assert np.all(np.abs(got - exact) <= bound)


def test_shape_errors():
    w = np.zeros((3, 4), np.int8)
    with pytest.raises(oracle.InvalidShape, match=r"hidden.len\(\) == 4, got hidden.len\(\) == 5"):
        oracle.lm_head_matmul_i8(np.zeros(5, f32), w, np.ones(3, f32), np.zeros(3, f32), 3, 4)
    with pytest.raises(oracle.InvalidShape, match="scales.len"):
        oracle.lm_head_matmul_i8(np.zeros(4, f32), w, np.ones(2, f32), np.zeros(3, f32), 3, 4)
    with pytest.raises(oracle.InvalidShape, match="output.len"):
        oracle.lm_head_matmul_i8(np.zeros(4, f32), w, np.ones(3, f32), np.zeros(4, f32), 3, 4)
    with pytest.raises(oracle.InvalidShape, match="weights_i8.len"):
        oracle.lm_head_matmul_i8(np.zeros(4, f32), w, np.ones(3, f32), np.zeros(3, f32), 2, 4)
