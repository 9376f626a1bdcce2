"""Pins of the oracle's W2A8 ternary GEMV (oracle/bnr_oracle.c,
bnro_ternary_gemv_preq / bnro_dot_packed_ternary_i8 / bnro_pack_ternary).

Closed forms are the reference's own tests (bitnet-cpu/src/gemv.rs:318-728,
restated for the pre-quantised entry point with act_absmax = 127 so that the
combined scale equals weight_scale); brute force is an independent numpy
computation from the unpacked int8 matrix.  Integer accumulation is exact, so
the comparison is bit-exact.
"""
import numpy as np
import pytest

import oracle

f32 = np.float32


def gemv(w_i8, ws, x_q, absmax):
    w_i8 = np.asarray(w_i8, np.int8)
    m, k = w_i8.shape
    out = np.full(m, np.nan, f32)
    oracle.ternary_gemv_preq(oracle.pack_rows(w_i8), ws, np.asarray(x_q, np.int8), absmax, out, m, k)
    return out


def brute(w_i8, ws, x_q, absmax):
    acc = np.asarray(w_i8, np.int64) @ np.asarray(x_q, np.int64)
    combined = f32(f32(f32(ws) * f32(absmax)) / f32(127.0))
    return acc.astype(f32) * combined


def test_pack_ternary_codes():
    # +1 -> 0b00, 0 -> 0b01, -1 -> 0b10, little-endian within the byte (ternary.rs:250-266)
    assert oracle.pack_ternary(np.array([1, 0, -1, -1], np.int8)).tolist() == [0 | 1 << 2 | 2 << 4 | 2 << 6]
    assert oracle.pack_ternary(np.array([1, 0, -1], np.int8)).tolist() == [36]  # unused code 0b00
    assert oracle.pack_ternary(np.array([0] * 5, np.int8)).tolist() == [0x55, 0x01]
    with pytest.raises(oracle.InvalidConfig):
        oracle.pack_ternary(np.array([2], np.int8))


def test_gemv_2x3():  # gemv.rs gemv_2x3
    np.testing.assert_array_equal(gemv([[1, 0, -1], [-1, 1, 0]], 0.5, [2, 3, 4], 127.0), [-1.0, 0.5])


def test_gemv_identity():  # gemv.rs gemv_identity_weight
    np.testing.assert_array_equal(gemv(np.eye(3, dtype=np.int8), 1.0, [5, 7, 9], 127.0), [5, 7, 9])


def test_gemv_negation():  # gemv.rs gemv_negation_weight
    np.testing.assert_array_equal(gemv([[-1] * 4], 2.0, [1, 2, 3, 4], 127.0), [-20.0])


def test_gemv_scale_applied():  # gemv.rs gemv_scale_applied_correctly
    np.testing.assert_array_equal(gemv([[1, 1, 1]], 0.25, [1, 1, 1], 127.0), [0.75])


def test_gemv_single_element_and_zeros():  # gemv_single_row_single_col, all_zero_weights
    np.testing.assert_array_equal(gemv([[-1]], 2.0, [3], 127.0), [-6.0])
    np.testing.assert_array_equal(gemv(np.zeros((3, 4), np.int8), 1.0, [1, 2, 3, 4], 127.0), [0, 0, 0])
    np.testing.assert_array_equal(gemv([[1, -1, 1], [0, 1, -1]], 1.0, [0, 0, 0], 127.0), [0, 0])


def test_gemv_quantised_nonzero_dot():  # gemv.rs gemv_quantised_nonzero_dot_product
    # w = [1,1,1,1] (w_scale 1), x_q = [127,0,0,0], max_abs = 1 -> 127 * 1 * 1 / 127 = 1
    np.testing.assert_array_equal(gemv([[1, 1, 1, 1]], 1.0, [127, 0, 0, 0], 1.0), [f32(127) * f32(f32(1.0 * 1.0) / f32(127))])


def test_gemv_linear_in_scale():  # gemv.rs gemv_output_linear_in_scale
    w = [[1, -1, 0], [1, 0, -1]]
    a = gemv(w, 1.0, [3, 5, 7], 127.0)
    b = gemv(w, 2.0, [3, 5, 7], 127.0)
    np.testing.assert_array_equal(b, 2 * a)


@pytest.mark.parametrize("m,k", [(1, 1), (2, 3), (5, 63), (7, 64), (3, 65), (4, 127), (9, 200),
                                 (33, 2560), (16, 6912)])
def test_gemv_brute_force(m, k):
    rng = np.random.default_rng(1000 * m + k)
    w = rng.integers(-1, 2, size=(m, k)).astype(np.int8)
    x = rng.integers(-128, 128, size=k).astype(np.int8)
    ws, aa = f32(rng.uniform(0.1, 3)), f32(rng.uniform(0.1, 50))
    np.testing.assert_array_equal(gemv(w, ws, x, aa), brute(w, ws, x, aa))


def test_gemv_extreme_accumulator():
    # |acc| = 128 * 6912 = 884736 < 2^24: exact in f32
    k = 6912
    w = -np.ones((2, k), np.int8)
    w[1] = 1
    out = gemv(w, 1.0, np.full(k, -128, np.int8), 127.0)
    np.testing.assert_array_equal(out, [884736.0, -884736.0])


def test_dot_packed_decodes_code3_as_zero_and_ignores_padding():
    # DECODE_LUT maps 0b11 to 0 (simd.rs:390-404); bits past n are never read.
    rng = np.random.default_rng(7)
    for n in [1, 3, 16, 63, 64, 65, 130]:
        packed = rng.integers(0, 256, size=(n + 3) // 4).astype(np.uint8)
        act = rng.integers(-128, 128, size=n).astype(np.int8)
        lut = np.array([1, 0, -1, 0], np.int64)
        codes = (packed[np.arange(n) // 4] >> (2 * (np.arange(n) % 4))) & 3
        assert oracle.dot_packed_ternary_i8(packed, act, n) == int(lut[codes] @ act.astype(np.int64))


def test_gemv_errors_match_reference():
    p = oracle.pack_rows(np.ones((2, 3), np.int8))
    out = np.zeros(2, f32)
    x = np.zeros(3, np.int8)
    with pytest.raises(oracle.InvalidShape, match=r"weight_packed.len\(\) == 2 \* ceil\(3/4\) = 2, got weight_packed.len\(\) == 3"):
        oracle.ternary_gemv_preq(np.zeros(3, np.uint8), 1.0, x, 1.0, out, 2, 3)
    with pytest.raises(oracle.InvalidShape, match=r"activation.len\(\) == 3, got activation.len\(\) == 4"):
        oracle.ternary_gemv_preq(p, 1.0, np.zeros(4, np.int8), 1.0, out, 2, 3)
    with pytest.raises(oracle.InvalidShape, match=r"output.len\(\) == 2, got output.len\(\) == 3"):
        oracle.ternary_gemv_preq(p, 1.0, x, 1.0, np.zeros(3, f32), 2, 3)
    with pytest.raises(oracle.QuantizationError, match="weight_scale must be finite > 0, got 0"):
        oracle.ternary_gemv_preq(p, 0.0, x, 1.0, out, 2, 3)
    with pytest.raises(oracle.QuantizationError, match="weight_scale must be finite > 0, got -1.5"):
        oracle.ternary_gemv_preq(p, -1.5, x, 1.0, out, 2, 3)
    with pytest.raises(oracle.QuantizationError, match="act_scale must be finite > 0, got NaN"):
        oracle.ternary_gemv_preq(p, 1.0, x, float("nan"), out, 2, 3)
    with pytest.raises(oracle.QuantizationError, match="act_scale must be finite > 0, got inf"):
        oracle.ternary_gemv_preq(p, 1.0, x, float("inf"), out, 2, 3)
    # shape errors come before scale errors (gemv.rs:260-295)
    with pytest.raises(oracle.InvalidShape):
        oracle.ternary_gemv_preq(p, 0.0, np.zeros(4, np.int8), 1.0, out, 2, 3)


def test_rust_float_display():
    # Rust's Display of f32 is the shortest round-trip decimal, positional
    p = oracle.pack_rows(np.ones((1, 1), np.int8))
    for v, txt in [(-1e-7, "-0.0000001"), (-2.5, "-2.5"), (-1e20, "-100000000000000000000"),
                   (-0.1, "-0.1"), (-3.0, "-3"), (float("-inf"), "-inf"), (-1.17549435e-38, None)]:
        with pytest.raises(oracle.QuantizationError) as ei:
            oracle.ternary_gemv_preq(p, 1.0, np.zeros(1, np.int8), v, np.zeros(1, f32), 1, 1)
        got = str(ei.value).rsplit("got ", 1)[1]
        if txt is not None:
            assert got == txt
        assert "e" not in got.lower() or got in ("-inf", "inf")
        assert f32(float(got)) == f32(v)  # reads back to the same f32
