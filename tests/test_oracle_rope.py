"""Pins of the oracle's RoPE (restatement of bitnet-cpu/src/rope.rs:100-430 and
CpuBackend::rope_embed, bitnet-cpu/src/lib.rs:289-314) against the
reference's closed-form tests (rope.rs:444-805, ops.rs:406-478,
cpu/lib.rs:714-745), an independent complex-number formulation and the
lazy-table policy."""
import numpy as np
import pytest

import oracle

f32 = np.float32


# --- RopeCache (rope.rs:444-512) ----------------------------------------------

def test_table_shape():
    c, s = oracle.rope_table(32, 16, 10000.0)
    assert c.shape == (32, 8) and s.shape == (32, 8)


def test_table_position_zero_is_identity():
    c, s = oracle.rope_table(4, 8, 10000.0)
    assert np.all(c[0] == 1.0) and np.all(s[0] == 0.0)


def test_table_unit_norm():
    c, s = oracle.rope_table(16, 32, 500000.0)
    np.testing.assert_allclose(c * c + s * s, 1.0, atol=1e-5)


@pytest.mark.parametrize("hd,theta", [(7, 1e4), (0, 1e4), (8, 0.0), (8, -1.0), (8, np.inf)])
def test_table_invalid_config(hd, theta):
    with pytest.raises(oracle.InvalidConfig):
        oracle.rope_table(4, hd, theta)


def test_table_empty_max_seq():
    c, s = oracle.rope_table(0, 8, 10000.0)
    assert c.size == 0 and s.size == 0


def test_table_matches_independent_angle_formula():
    # freq_i = theta^(-2i/d) rounded to f32, angle = f32(pos) * freq (one f32
    # rounding), then cos/sin of that f32 angle.  Computed here in float64
    # from the f32 intermediates; glibc powf/cosf/sinf are within 1 ulp, so
    # every entry must agree within 2 ulp of the float64 value.
    d, theta, max_seq = 128, f32(500000.0), 4096
    c, s = oracle.rope_table(max_seq, d, float(theta))
    i = np.arange(d // 2)
    exponent = (f32(-2.0) * i.astype(f32)) / f32(d)
    freq = (np.float64(theta) ** exponent.astype(np.float64)).astype(f32)
    angle = np.arange(max_seq, dtype=f32)[:, None] * freq[None, :]
    ref_c = np.cos(angle.astype(np.float64))
    ref_s = np.sin(angle.astype(np.float64))
    # 2 ulp of the f32 result plus one ulp of freq propagated through the angle
    ulp = np.spacing(np.abs(ref_c).astype(f32)).astype(np.float64)
    slack = np.abs(angle.astype(np.float64)) * 2.0**-23
    assert np.all(np.abs(c - ref_c) <= 2 * ulp + slack)
    ulp = np.spacing(np.abs(ref_s).astype(f32)).astype(np.float64)
    assert np.all(np.abs(s - ref_s) <= 2 * ulp + slack)


# --- apply_rope (rope.rs:518-677) ----------------------------------------------

def test_position_zero_is_identity():
    q = (np.arange(16) * 0.1).astype(f32)
    k = (np.arange(8) * 0.2).astype(f32)
    q0, k0 = q.copy(), k.copy()
    oracle.apply_rope(q, k, 0, 8, 2, 1, 10000.0)
    np.testing.assert_array_equal(q, q0)
    np.testing.assert_array_equal(k, k0)


@pytest.mark.parametrize("pos", [1, 5, 17, 100, 1000])
def test_preserves_head_norm(pos):
    q = ((np.arange(64) * 0.37 + 0.11) * 2 - 1).astype(f32)
    k = ((np.arange(32) * 0.53 + 0.07) * 2 - 1).astype(f32)
    nq = np.linalg.norm(q.reshape(4, 16), axis=1)
    nk = np.linalg.norm(k.reshape(2, 16), axis=1)
    oracle.apply_rope(q, k, pos, 16, 4, 2, 500000.0)
    np.testing.assert_allclose(np.linalg.norm(q.reshape(4, 16), axis=1), nq, atol=1e-4)
    np.testing.assert_allclose(np.linalg.norm(k.reshape(2, 16), axis=1), nk, atol=1e-4)


@pytest.mark.parametrize("qn,kn,hd,exc", [
    (15, 8, 8, oracle.InvalidShape), (16, 7, 8, oracle.InvalidShape),
    (7, 7, 7, oracle.InvalidShape),
])
def test_apply_rope_shape_errors(qn, kn, hd, exc):
    with pytest.raises(exc):
        oracle.apply_rope(np.zeros(qn, f32), np.zeros(kn, f32), 0, hd, 2 if qn > 8 else 1, 1,
                          10000.0)


def test_apply_rope_zero_theta():
    with pytest.raises(oracle.InvalidConfig):
        oracle.apply_rope(np.zeros(8, f32), np.zeros(8, f32), 0, 8, 1, 1, 0.0)


def test_90_degree_rotation_check():  # rope.rs:648-677
    q = np.array([1.0, 0.0], f32)
    k = np.array([1.0, 0.0], f32)
    oracle.apply_rope(q, k, 1, 2, 1, 1, 10000.0)
    np.testing.assert_allclose(q, [np.cos(1.0), np.sin(1.0)], atol=1e-6)


def test_half_split_pairing():
    # Pairing is (i, i+d/2), not (2i, 2i+1) (rope.rs:414-430,
    # bitnet-convert/src/lib.rs:176-183).  d=4, pos=1: freq = [1, theta^-0.5].
    theta = 10000.0
    q = np.array([1.0, 0.0, 0.0, 0.0], f32)
    k = np.zeros(4, f32)
    oracle.apply_rope(q, k, 1, 4, 1, 1, theta)
    # x0 pairs with x2: x0' = cos 1, x2' = sin 1; x1, x3 untouched (zero).
    np.testing.assert_allclose(q, [np.cos(1.0), 0.0, np.sin(1.0), 0.0], atol=1e-6)


def test_matches_complex_rotation():
    # (x_lo + i x_hi) * exp(i angle) in float64 == half-split rotation.
    d, theta = 128, 500000.0
    q = oracle.normal(5, (20 * d,))
    k = oracle.normal(6, (5 * d,))
    for pos in [0, 1, 511, 4095]:
        qq, kk = q.copy(), k.copy()
        oracle.apply_rope(qq, kk, pos, d, 20, 5, theta)
        i = np.arange(d // 2)
        ang = pos * np.float64(theta) ** (-2.0 * i / d)
        for x, y in [(q, qq), (k, kk)]:
            z = (x.reshape(-1, d)[:, :64] + 1j * x.reshape(-1, d)[:, 64:]) * np.exp(1j * ang)
            ref = np.concatenate([z.real, z.imag], axis=1).reshape(-1)
            # the f32 angle carries ~pos*2^-24 rad of rounding (plus one ulp of freq)
            atol = np.abs(x).max() * 2 * (pos + 1) * 2.0**-23 + 1e-5
            np.testing.assert_allclose(y, ref, atol=atol, rtol=0)


def test_different_positions_give_different_rotations():
    q0 = np.array([1.0, 0.5, -0.3, 0.8, 0.1, -0.6, 0.4, -0.2], f32)
    a, b = q0.copy(), q0.copy()
    oracle.apply_rope(a, np.zeros(8, f32), 1, 8, 1, 1, 10000.0)
    oracle.apply_rope(b, np.zeros(8, f32), 2, 8, 1, 1, 10000.0)
    assert np.abs(a - b).sum() > 1e-4


# --- apply_rope_cached (rope.rs:705-766) ----------------------------------------

def test_cached_matches_uncached():
    c, s = oracle.rope_table(64, 16, 500000.0)
    for pos in [0, 1, 10, 31, 63]:
        q0 = (np.arange(64) * 0.1 - 3.2).astype(f32)
        k0 = (np.arange(32) * 0.2 - 3.2).astype(f32)
        qa, ka, qb, kb = q0.copy(), k0.copy(), q0.copy(), k0.copy()
        oracle.apply_rope(qa, ka, pos, 16, 4, 2, 500000.0)
        oracle.apply_rope_cached(qb, kb, pos, 4, 2, c, s, 16)
        np.testing.assert_array_equal(qa, qb)
        np.testing.assert_array_equal(ka, kb)


def test_cached_out_of_bounds():
    c, s = oracle.rope_table(4, 8, 10000.0)
    with pytest.raises(oracle.InvalidShape):
        oracle.apply_rope_cached(np.zeros(8, f32), np.zeros(8, f32), 4, 1, 1, c, s, 8)


def test_relative_position_invariance():  # rope.rs:773-805
    qi = np.array([0.5, -0.3, 0.7, 0.1, -0.2, 0.4, 0.6, -0.5], f32)
    ki = np.array([0.2, 0.8, -0.4, 0.3, 0.5, -0.1, 0.7, -0.6], f32)

    def rot(x, pos):
        y = x.copy()
        oracle.apply_rope(y, np.zeros(8, f32), pos, 8, 1, 1, 10000.0)
        return y

    assert abs(rot(qi, 3) @ rot(ki, 1) - rot(qi, 13) @ rot(ki, 11)) < 1e-3


# --- CpuBackend::rope_embed lazy-table policy (cpu/lib.rs:289-314) -------------

def test_backend_rope_embed_identity_and_error():  # cpu/lib.rs:714-745
    be = oracle.CpuBackend()
    q = (np.arange(8) * 0.1).astype(f32)
    q0 = q.copy()
    be.rope_embed(q, (np.arange(8) * 0.2).astype(f32), 0, 8, 1, 1, 10000.0)
    np.testing.assert_array_equal(q, q0)
    with pytest.raises(oracle.InvalidShape):
        be.rope_embed(np.zeros(7, f32), np.zeros(8, f32), 0, 8, 1, 1, 10000.0)


def test_backend_table_policy():
    be = oracle.CpuBackend()
    assert be.rope_state() is None
    q, k = np.zeros(128, f32), np.zeros(128, f32)
    be.rope_embed(q, k, 10, 128, 1, 1, 500000.0)
    assert be.rope_state() == (4096, 128, 500000.0)
    be.rope_embed(q, k, 5000, 128, 1, 1, 500000.0)  # pos >= max_seq -> pos+1
    assert be.rope_state() == (5001, 128, 500000.0)
    be.rope_embed(q[:64], k[:64], 3, 64, 1, 1, 500000.0)  # head_dim change -> 4096
    assert be.rope_state() == (4096, 64, 500000.0)
    be.rope_embed(q[:64], k[:64], 3, 64, 1, 1, 1.0)  # theta change -> rebuild
    assert be.rope_state() == (4096, 64, 1.0)
    be.rope_embed(q[:64], k[:64], 3, 64, 1, 1, 1.0005)  # |dtheta| <= 1e-3: reuse
    assert be.rope_state() == (4096, 64, 1.0)
    be.rope_embed(q[:64], k[:64], 3, 64, 1, 1, 1.002)  # |dtheta| > 1e-3: rebuild
    assert be.rope_state()[2] == pytest.approx(1.002)


def test_backend_rope_config_errors_keep_table():
    be = oracle.CpuBackend()
    q, k = np.zeros(8, f32), np.zeros(8, f32)
    be.rope_embed(q, k, 0, 8, 1, 1, 10000.0)
    with pytest.raises(oracle.InvalidConfig):  # odd head_dim via RopeCache::new
        be.rope_embed(np.zeros(7, f32), np.zeros(7, f32), 0, 7, 1, 1, 10000.0)
    with pytest.raises(oracle.InvalidConfig):
        be.rope_embed(q, k, 0, 8, 1, 1, -5.0)
    assert be.rope_state() == (4096, 8, 10000.0)
