"""Pins of the oracle's attention (restatement of bitnet-cpu/src/attention.rs:
97-209) against the reference's own closed-form tests (attention.rs:248-719,
bitnet-cpu/src/lib.rs:748-779), fp64 brute force and torch's
scaled_dot_product_attention (an independent library routine)."""
import numpy as np
import pytest

import oracle
from common import attention_f64, assert_close, decode_workload

f32 = np.float32


def run(q, k, v, n_heads, n_kv, head_dim, cur_pos):
    out = np.zeros(n_heads * head_dim, f32)
    oracle.masked_attention(np.asarray(q, f32), np.asarray(k, f32), np.asarray(v, f32), out,
                            n_heads, n_kv, head_dim, cur_pos)
    return out


def positional_cache(seq_len, n_kv, head_dim, scale):
    c = np.zeros((n_kv, seq_len, head_dim), f32)
    for t in range(seq_len):
        c[:, t, :] = t * scale
    return c.reshape(-1)


# --- ports of attention.rs tests ---------------------------------------------

def test_single_head_single_position_is_identity():  # attention.rs:248-268
    out = run([1, 0, 0, 0], [1, 0, 0, 0], [0.1, 0.2, 0.3, 0.4], 1, 1, 4, 0)
    np.testing.assert_allclose(out, [0.1, 0.2, 0.3, 0.4], atol=1e-5)


def test_uniform_scores_produce_averaged_values():  # attention.rs:271-311
    k = np.arange(1, 7, dtype=f32)
    v = np.array([1, 0, 2, 0, 3, 0], f32)
    out = run([0, 0], k, v, 1, 1, 2, 2)
    assert abs(out[0] - 2.0) < 1e-5 and abs(out[1]) < 1e-5


def test_high_score_for_last_position_attends_to_last_value():  # attention.rs:314-343
    k = np.zeros(6, f32)
    k[4] = 1.0
    v = np.zeros(6, f32)
    v[0], v[2], v[4] = 1.0, 2.0, 99.0
    out = run([1000.0, 0.0], k, v, 1, 1, 2, 2)
    assert abs(out[0] - 99.0) < 1.0


def test_gqa_groups_correct_kv_head_assignment():  # attention.rs:346-424
    v = np.array([1, 0, 0, 1], f32)
    out = run(np.zeros(8), np.zeros(4), v, 4, 2, 2, 0)
    np.testing.assert_allclose(out, [1, 0, 1, 0, 0, 1, 0, 1], atol=1e-5)


def test_attention_output_is_convex_combination_of_values():  # attention.rs:427-469
    hd, L = 4, 5
    q = np.array([0.5, -0.3, 0.7, 0.1], f32)
    t = np.arange(L)[:, None]
    d = np.arange(hd)[None, :]
    k = (t * 0.1 + d * 0.2 - 0.5).astype(f32).reshape(-1)
    v = ((t + 1) * (d + 1) * 0.1).astype(f32)
    out = run(q, k, v.reshape(-1), 1, 1, hd, L - 1)
    assert np.all(out >= v.min(0) - 1e-5) and np.all(out <= v.max(0) + 1e-5)


def test_output_all_finite():  # attention.rs:472-506
    q = ((np.arange(32) - 16.0) * 0.1).astype(f32)
    k = ((np.arange(128) - 32.0) * 0.05).astype(f32)
    v = (np.arange(128) * 0.01).astype(f32)
    assert np.all(np.isfinite(run(q, k, v, 4, 2, 8, 7)))


@pytest.mark.parametrize("args,exc", [
    ((np.zeros(7), np.zeros(8), np.zeros(8), np.zeros(8), 2, 2, 4, 0), oracle.InvalidShape),
    ((np.zeros(8), np.zeros(8), np.zeros(8), np.zeros(6), 2, 2, 4, 0), oracle.InvalidShape),
    ((np.zeros(8), np.zeros(3), np.zeros(8), np.zeros(8), 2, 2, 4, 0), oracle.InvalidShape),
    ((np.zeros(8), np.zeros(8), np.zeros(3), np.zeros(8), 2, 2, 4, 0), oracle.InvalidShape),
    ((np.zeros(12), np.zeros(8), np.zeros(8), np.zeros(12), 3, 2, 4, 0), oracle.InvalidConfig),
    ((np.zeros(0), np.zeros(0), np.zeros(0), np.zeros(0), 1, 1, 0, 0), oracle.InvalidShape),
    ((np.zeros(4), np.zeros(0), np.zeros(0), np.zeros(4), 1, 0, 4, 0), oracle.InvalidConfig),
])
def test_error_kinds(args, exc):  # attention.rs:512-581
    q, k, v, out = (np.asarray(a, f32) for a in args[:4])
    with pytest.raises(exc):
        oracle.masked_attention(q, k, v, out, *args[4:])


def test_stride_too_short_is_invalid_shape():  # attention.rs:146-151
    with pytest.raises(oracle.InvalidShape):
        run(np.zeros(4), np.zeros(8), np.zeros(8), 1, 1, 4, 2)  # 2 rows held, 3 needed


def test_output_scales_linearly_with_values():  # attention.rs:589-614
    q = (np.arange(4) * 0.1).astype(f32)
    k = positional_cache(4, 1, 4, 0.1)
    v1 = positional_cache(4, 1, 4, 0.5)
    np.testing.assert_allclose(3 * run(q, k, v1, 1, 1, 4, 3), run(q, k, 3 * v1, 1, 1, 4, 3),
                               atol=1e-5)


def test_softmax_shift_invariance_in_attention():  # attention.rs:621-683
    q = np.array([0.5, -0.3, 0.1, 0.8], f32)
    k = ((np.arange(12) - 6.0) * 0.2).astype(f32)
    v = positional_cache(3, 1, 4, 0.3)
    np.testing.assert_allclose(run(q, k, v, 1, 1, 4, 2), run(q, k + 1, v, 1, 1, 4, 2),
                               atol=1e-4)


def test_bitnet_2b_dimensions_smoke():  # attention.rs:690-719
    out = run(np.zeros(20 * 128), np.zeros(4 * 5 * 128), np.full(4 * 5 * 128, 0.1), 20, 5,
              128, 3)
    np.testing.assert_allclose(out, 0.1, atol=1e-5)


def test_fixed_capacity_cache_ignores_reserved_rows():  # mod.rs:278-287, lib.rs:262-280
    # Rows past cur_pos hold garbage; only rows 0..=cur_pos may be read.
    w = decode_workload(7, 9, cap=16, n_heads=4, n_kv=2, head_dim=8)
    kc, vc = w["k_cache"].copy(), w["v_cache"].copy()
    out1 = run(w["q"], kc.reshape(-1), vc.reshape(-1), 4, 2, 8, 8)
    kc[:, 9:] = 1e6
    vc[:, 9:] = -1e6
    out2 = run(w["q"], kc.reshape(-1), vc.reshape(-1), 4, 2, 8, 8)
    np.testing.assert_array_equal(out1, out2)


# --- independent pins --------------------------------------------------------

@pytest.mark.parametrize("n_heads,n_kv,hd,pos,cap", [
    (1, 1, 4, 0, 1), (4, 2, 8, 7, 8), (20, 5, 128, 511, 4096), (8, 8, 16, 40, 64),
    (20, 5, 128, 4095, 4096), (6, 3, 10, 33, 50),
])
def test_matches_fp64_brute_force(n_heads, n_kv, hd, pos, cap):
    w = decode_workload(9, pos, cap=cap, q_scale=4.0, n_heads=n_heads, n_kv=n_kv, head_dim=hd)
    kc, vc = w["k_cache"].reshape(-1), w["v_cache"].reshape(-1)
    kc[:] = np.where(kc == 0, 0.25, kc)  # fill the new row too
    out = run(w["q"], kc, vc, n_heads, n_kv, hd, pos)
    ref = attention_f64(w["q"], kc, vc, n_heads, n_kv, hd, pos)
    assert_close(out, ref, "oracle vs fp64", atol=1e-5, rtol=1e-4)


def test_matches_torch_sdpa_fp64():
    torch = pytest.importorskip("torch")
    n_heads, n_kv, hd, pos = 20, 5, 128, 300
    w = decode_workload(10, pos + 1, cap=512, n_heads=n_heads, n_kv=n_kv, head_dim=hd)
    kc, vc = w["k_cache"], w["v_cache"]
    out = run(w["q"], kc.reshape(-1), vc.reshape(-1), n_heads, n_kv, hd, pos)
    q = torch.from_numpy(w["q"].reshape(1, n_heads, 1, hd)).double()
    K = torch.from_numpy(kc[:, :pos + 1]).double().repeat_interleave(4, 0)[None]
    V = torch.from_numpy(vc[:, :pos + 1]).double().repeat_interleave(4, 0)[None]
    ref = torch.nn.functional.scaled_dot_product_attention(q, K.contiguous(), V.contiguous())
    assert_close(out, ref.reshape(-1).numpy(), "oracle vs sdpa", atol=1e-5, rtol=1e-4)


def test_scalar_and_avx2_paths_agree():
    w = decode_workload(11, 200, cap=256, n_heads=8, n_kv=2, head_dim=128)
    args = (w["q"], w["k_cache"].reshape(-1), w["v_cache"].reshape(-1), 8, 2, 128, 199)
    a = run(*args)
    oracle.force_scalar(True)
    try:
        b = run(*args)
    finally:
        oracle.force_scalar(False)
    assert_close(a, b, "avx2 vs scalar", atol=1e-5, rtol=1e-5)


def test_thread_count_does_not_change_result():
    w = decode_workload(12, 100, cap=128)
    args = (w["q"], w["k_cache"].reshape(-1), w["v_cache"].reshape(-1), 20, 5, 128, 99)
    a = run(*args)
    n0 = oracle.get_threads()
    oracle.set_threads(1)
    try:
        b = run(*args)
    finally:
        oracle.set_threads(n0)
    np.testing.assert_array_equal(a, b)
