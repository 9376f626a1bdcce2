"""GPU parity of the HIP path against the oracle (the C restatement of the
reference's CPU path), through the C ABI.

Bit-exact: rotated q/k and appended cache rows.  Attention outputs: per
element |gpu - ref| <= 2e-3 + 1e-3|ref| (fp32 I/O); long contexts also
|gpu - ref| <= 1e-5 + 1e-4 max|ref| over the output, and row-count cases
(q = 0, one-hot value rows: outputs are row counts) within 1e-6 relative, so
that a single row attended twice or not at all fails.
"""
import sys

import numpy as np
import pytest

import oracle
from common import (D, HKV, HQ, THETA, assert_close, assert_close_scaled, batched_lengths,
                    error_from_parts,
                    decode_workload, oracle_decode, oracle_prefill, prefill_workload, seed)

pytestmark = pytest.mark.gpu
f32 = np.float32


def case(msg):
    print(f"[gpu case] {msg}", flush=True)
    sys.stdout.flush()


def dev(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda")


def host(t):
    import torch

    torch.cuda.synchronize()
    return t.cpu().numpy()


# --- trait-shaped host entry points ------------------------------------------------

def test_host_closed_forms(backend):
    case("host closed forms (attention.rs:248-719)")
    out = np.zeros(4, f32)
    backend.masked_attention(np.array([1, 0, 0, 0], f32), np.array([1, 0, 0, 0], f32),
                             np.array([.1, .2, .3, .4], f32), out, 1, 1, 4, 0)
    np.testing.assert_allclose(out, [.1, .2, .3, .4], atol=1e-5)
    out = np.zeros(2, f32)
    backend.masked_attention(np.zeros(2, f32), np.arange(1, 7, dtype=f32),
                             np.array([1, 0, 2, 0, 3, 0], f32), out, 1, 1, 2, 2)
    np.testing.assert_allclose(out, [2, 0], atol=1e-5)
    out = np.zeros(8, f32)
    backend.masked_attention(np.zeros(8, f32), np.zeros(4, f32), np.array([1, 0, 0, 1], f32),
                             out, 4, 2, 2, 0)
    np.testing.assert_allclose(out, [1, 0, 1, 0, 0, 1, 0, 1], atol=1e-5)
    out = np.zeros(20 * 128, f32)
    backend.masked_attention(np.zeros(20 * 128, f32), np.zeros(4 * 640, f32),
                             np.full(4 * 640, 0.1, f32), out, 20, 5, 128, 3)
    np.testing.assert_allclose(out, 0.1, atol=1e-5)


@pytest.mark.parametrize("args", [
    (7, 8, 8, 8, 2, 2, 4, 0), (8, 8, 8, 6, 2, 2, 4, 0), (8, 3, 8, 8, 2, 2, 4, 0),
    (8, 8, 3, 8, 2, 2, 4, 0), (12, 8, 8, 12, 3, 2, 4, 0), (0, 0, 0, 0, 1, 1, 0, 0),
    (4, 0, 0, 4, 1, 0, 4, 0), (4, 8, 8, 4, 1, 1, 4, 2),
])
def test_host_error_kinds_match_oracle(backend, args):
    case(f"host error kinds {args}")
    import bitnetrs_amd

    arrs = [np.zeros(n, f32) for n in args[:4]]
    with pytest.raises(oracle.OracleError) as e_ref:
        oracle.masked_attention(*arrs, *args[4:])
    with pytest.raises(bitnetrs_amd.BitNetError) as e_gpu:
        backend.masked_attention(*arrs, *args[4:])
    assert e_gpu.value.kind == e_ref.value.kind
    assert str(e_gpu.value) == str(e_ref.value)
    # the variant rebuilt from bnr_last_error_parts prints the oracle's text
    assert error_from_parts() == (e_ref.value.kind, str(e_ref.value))


def test_host_rope_embed_bit_exact(backend):
    """Positions past the table's end grow it (the library doubles it, the
    reference rebuilds at position + 1): the values stay bit-identical."""
    case("host rope_embed bit-exact, d=128 theta=5e5, positions 0..16500")
    ref = oracle.CpuBackend()
    for pos in [0, 1, 2, 511, 4095, 4096, 4097, 4100, 8191, 8192, 8300, 16500, 3]:
        q = oracle.normal(seed(1, 0) + pos, (HQ * D,))
        k = oracle.normal(seed(1, 1) + pos, (HKV * D,))
        q2, k2 = q.copy(), k.copy()
        ref.rope_embed(q, k, pos, D, HQ, HKV, THETA)
        backend.rope_embed(q2, k2, pos, D, HQ, HKV, THETA)
        np.testing.assert_array_equal(q2, q)
        np.testing.assert_array_equal(k2, k)


def test_host_rope_embed_errors(backend):
    case("host rope_embed errors")
    import bitnetrs_amd

    ref = oracle.CpuBackend()
    for n_q, n_k, hd, theta, cls in [(7, 7, 7, 1e4, bitnetrs_amd.InvalidConfig),
                                     (8, 8, 8, 0.0, bitnetrs_amd.InvalidConfig),
                                     (0, 0, 0, 1e4, bitnetrs_amd.InvalidConfig),
                                     (7, 8, 8, 1e4, bitnetrs_amd.InvalidShape),
                                     (8, 7, 8, 1e4, bitnetrs_amd.InvalidShape)]:
        with pytest.raises(cls) as e_gpu:
            backend.rope_embed(np.zeros(n_q, f32), np.zeros(n_k, f32), 0, hd, 1, 1, theta)
        got = error_from_parts()
        with pytest.raises(oracle.OracleError) as e_ref:
            ref.rope_embed(np.zeros(n_q, f32), np.zeros(n_k, f32), 0, hd, 1, 1, theta)
        assert got == (e_ref.value.kind, str(e_ref.value)) == (e_gpu.value.kind, str(e_gpu.value))


def test_host_decode_sequence_c1(backend):
    case("host path C1: rope_embed -> store -> masked_attention at pos 511")
    backend.mirror_invalidate()  # a recycled host address must not look in sync
    w = decode_workload(1, 511)
    q_ref, k_ref, _, _, out_ref = oracle_decode(w)
    q, k = w["q"].copy(), w["k"].copy()
    backend.rope_embed(q, k, 511, D, HQ, HKV, THETA)
    np.testing.assert_array_equal(q, q_ref)
    np.testing.assert_array_equal(k, k_ref)
    kc, vc = w["k_cache"].copy(), w["v_cache"].copy()
    kc[:, 511] = k.reshape(HKV, D)
    vc[:, 511] = w["v"].reshape(HKV, D)
    out = np.zeros(HQ * D, f32)
    backend.masked_attention(q, kc.reshape(-1), vc.reshape(-1), out, HQ, HKV, D, 511)
    print(assert_close(out, out_ref, "C1 host"))


@pytest.mark.parametrize("n_heads,n_kv,hd", [(20, 5, 128), (8, 8, 128), (8, 4, 128),
                                            (4, 2, 16), (6, 3, 64), (8, 1, 128)])
def test_host_mirror_incremental_decode(backend, n_heads, n_kv, hd):
    case(f"host mirror: 40 decode steps + rewind, heads {n_heads}/{n_kv} d {hd}")
    cap = 64
    ref = oracle.CpuBackend()
    kc = np.zeros((n_kv, cap, hd), f32)
    vc = np.zeros_like(kc)
    for step in range(40):
        q = oracle.normal(seed(30, 0) + step, (n_heads * hd,))
        k = oracle.normal(seed(30, 1) + step, (n_kv * hd,))
        v = oracle.normal(seed(30, 2) + step, (n_kv * hd,))
        ref.rope_embed(q, k, step, hd, n_heads, n_kv, 10000.0)
        kc[:, step] = k.reshape(n_kv, hd)
        vc[:, step] = v.reshape(n_kv, hd)
        out_ref = np.zeros(n_heads * hd, f32)
        oracle.masked_attention(q, kc.reshape(-1), vc.reshape(-1), out_ref, n_heads, n_kv, hd,
                                step)
        out = np.zeros_like(out_ref)
        backend.masked_attention(q, kc.reshape(-1), vc.reshape(-1), out, n_heads, n_kv, hd, step)
        assert_close(out, out_ref, f"step {step}")
    # rewind (new conversation into the same buffers): full resync
    kc[:] = oracle.normal(seed(30, 5), kc.shape)
    out_ref = np.zeros(n_heads * hd, f32)
    oracle.masked_attention(q, kc.reshape(-1), vc.reshape(-1), out_ref, n_heads, n_kv, hd, 5)
    out = np.zeros_like(out_ref)
    backend.masked_attention(q, kc.reshape(-1), vc.reshape(-1), out, n_heads, n_kv, hd, 5)
    assert_close(out, out_ref, "rewind")


@pytest.mark.parametrize("row", ["first", "middle", "last"])
@pytest.mark.parametrize("n_heads,n_kv,hd", [(HQ, HKV, D), (4, 2, 2), (6, 3, 16)])
def test_host_mirror_sampled_rewrite_resyncs(backend, row, n_heads, n_kv, hd):
    """A cached row rewritten in place without bnr_mirror_invalidate: when it
    is one of the rows the mirror samples at each sync (0, (n-1)/2, n-1 of
    the n synced rows; min(4, head_dim) floats at each end of a row), the
    next call re-uploads every row and matches the oracle on the rewritten
    cache."""
    case(f"host mirror: in-place rewrite of the {row} synced row, heads {n_heads}/{n_kv} d {hd}")
    backend.mirror_invalidate()
    cap = 128
    w = decode_workload(32, 100, cap=cap, n_heads=n_heads, n_kv=n_kv, head_dim=hd)
    kc, vc = w["k_cache"].reshape(-1), w["v_cache"].reshape(-1)
    q = w["q"]
    out = np.zeros(n_heads * hd, f32)
    backend.masked_attention(q, kc, vc, out, n_heads, n_kv, hd, 99)  # synced to rows 0..99
    r = {"first": 0, "middle": 49, "last": 99}[row]
    kc[r * hd:(r + 1) * hd] += 3.0  # kv head 0's row r: its first and last floats change
    h2 = n_kv - 1
    vc[(h2 * cap + r) * hd:(h2 * cap + r + 1) * hd] -= 2.0  # the last kv head's row r
    ref = np.zeros_like(out)
    oracle.masked_attention(q, kc, vc, ref, n_heads, n_kv, hd, 100)
    backend.masked_attention(q, kc, vc, out, n_heads, n_kv, hd, 100)
    assert_close(out, ref, f"{row} row rewritten")


def test_host_mirror_invalidate_and_full_mode(backend):
    case("host mirror invalidate / full mode")
    import bitnetrs_amd

    backend.mirror_invalidate()
    w = decode_workload(31, 100, cap=128)
    kc, vc = w["k_cache"].reshape(-1), w["v_cache"].reshape(-1)
    q = w["q"]
    out = np.zeros(HQ * D, f32)
    backend.masked_attention(q, kc, vc, out, HQ, HKV, D, 99)
    kc[5 * D:6 * D] += 3.0  # rewrite an old row of kv head 0
    ref = np.zeros_like(out)
    oracle.masked_attention(q, kc, vc, ref, HQ, HKV, D, 100)
    backend.mirror_invalidate()
    backend.masked_attention(q, kc, vc, out, HQ, HKV, D, 100)
    assert_close(out, ref, "after invalidate")
    backend.set_mirror_mode(bitnetrs_amd.BNR_MIRROR_FULL)
    try:
        vc[7 * D:8 * D] -= 2.0
        oracle.masked_attention(q, kc, vc, ref, HQ, HKV, D, 101)
        backend.masked_attention(q, kc, vc, out, HQ, HKV, D, 101)
        assert_close(out, ref, "full mode")
    finally:
        backend.set_mirror_mode(bitnetrs_amd.BNR_MIRROR_INCREMENTAL)


# --- device entry points -----------------------------------------------------------

@pytest.mark.parametrize("cfg,pos,q_scale", [(1, 511, 1.0), (2, 4095, 4.0), (5, 0, 1.0),
                                             (6, 1, 1.0), (7, 16, 1.0), (8, 1000, 2.0),
                                             (9, 2047, 1.0)])
def test_dev_decode_step_fused(backend, cfg, pos, q_scale):
    case(f"fused decode step cfg {cfg} pos {pos} q*{q_scale}")
    import torch

    w = decode_workload(cfg, pos, cap=4096, q_scale=q_scale)
    q_ref, k_ref, kc_ref, vc_ref, out_ref = oracle_decode(w)
    q, k, v = dev(w["q"]), dev(w["k"]), dev(w["v"])
    kc, vc = dev(w["k_cache"]), dev(w["v_cache"])
    out = torch.zeros(HQ * D, device="cuda")
    q_rot = torch.zeros_like(q)
    k_rot = torch.zeros_like(k)
    backend.dev_decode_step(q, k, v, pos, HQ, HKV, D, THETA, kc, vc, 4096, out, q_rot, k_rot)
    np.testing.assert_array_equal(host(q_rot), q_ref)
    np.testing.assert_array_equal(host(k_rot), k_ref)
    np.testing.assert_array_equal(host(kc)[:, pos], kc_ref[:, pos])
    np.testing.assert_array_equal(host(vc)[:, pos], vc_ref[:, pos])
    np.testing.assert_array_equal(host(q), w["q"])  # inputs untouched
    print(assert_close(host(out), out_ref, f"decode cfg {cfg}"))


@pytest.mark.parametrize("pos", [0, 63, 64, 511, 4095])
def test_dev_decode_attention_prerotated(backend, pos):
    case(f"decode attention (pre-rotated q) pos {pos}")
    import torch

    w = decode_workload(40, pos, cap=4096)
    q_ref, _, kc_ref, vc_ref, out_ref = oracle_decode(w)
    out = torch.zeros(HQ * D, device="cuda")
    backend.dev_decode_attention(dev(q_ref), dev(kc_ref), dev(vc_ref), 4096, out, HQ, HKV, D, pos)
    assert_close(host(out), out_ref, f"decode attention pos {pos}")


@pytest.mark.parametrize("n_heads,n_kv,hd", [(4, 4, 128), (8, 4, 128), (16, 2, 64), (6, 2, 16)])
def test_dev_decode_step_other_shapes(backend, n_heads, n_kv, hd):
    case(f"decode step heads {n_heads}/{n_kv} d {hd}")
    import torch

    pos = 300
    w = decode_workload(41, pos, cap=512, n_heads=n_heads, n_kv=n_kv, head_dim=hd)
    q_ref, k_ref, kc_ref, _, out_ref = oracle_decode(w, n_heads, n_kv, hd)
    kc, vc = dev(w["k_cache"]), dev(w["v_cache"])
    out = torch.zeros(n_heads * hd, device="cuda")
    k_rot = torch.zeros(n_kv * hd, device="cuda")
    backend.dev_decode_step(dev(w["q"]), dev(w["k"]), dev(w["v"]), pos, n_heads, n_kv, hd, THETA,
                            kc, vc, 512, out, None, k_rot)
    np.testing.assert_array_equal(host(k_rot), k_ref)
    np.testing.assert_array_equal(host(kc)[:, pos], kc_ref[:, pos])
    assert_close(host(out), out_ref, "other shape")


def test_dev_batched_decode_c4(backend):
    case("batched decode C4: 32 seqs, lengths U[128,4096)")
    import torch

    lens = batched_lengths()
    B, cap = len(lens), 4096
    q = oracle.normal(seed(4, 0), (B, HQ * D))
    k = oracle.normal(seed(4, 1), (B, HKV * D))
    v = oracle.normal(seed(4, 2), (B, HKV * D))
    kc = oracle.normal(seed(4, 3), (B, HKV, cap, D))
    vc = oracle.normal(seed(4, 4), (B, HKV, cap, D))
    d_kc, d_vc = dev(kc), dev(vc)
    out = torch.zeros(B, HQ * D, device="cuda")
    backend.dev_decode_step_batched(dev(q), dev(k), dev(v), lens, HQ, HKV, D, THETA, d_kc, d_vc,
                                    cap, out)
    got = host(out)
    gk = host(d_kc)
    for b in range(B):
        w = {"q": q[b], "k": k[b], "v": v[b], "k_cache": kc[b], "v_cache": vc[b],
             "pos": int(lens[b]), "cap": cap}
        _, k_ref, _, _, out_ref = oracle_decode(w)
        np.testing.assert_array_equal(gk[b][:, lens[b]], k_ref.reshape(HKV, D))
        assert_close(got[b], out_ref, f"seq {b} len {lens[b]}")


def test_dev_batched_decode_edge_lengths(backend):
    case("batched decode edge lengths 0,1,15,16,17,...; batch 70 > one launch")
    import torch

    lens = np.resize(np.array([0, 1, 15, 16, 17, 31, 32, 33, 255, 256, 257, 1023], np.int32), 70)
    B, cap = len(lens), 1024
    q = oracle.normal(seed(42, 0), (B, HQ * D))
    k = oracle.normal(seed(42, 1), (B, HKV * D))
    v = oracle.normal(seed(42, 2), (B, HKV * D))
    kc = oracle.normal(seed(42, 3), (B, HKV, cap, D))
    vc = oracle.normal(seed(42, 4), (B, HKV, cap, D))
    out = torch.zeros(B, HQ * D, device="cuda")
    backend.dev_decode_step_batched(dev(q), dev(k), dev(v), lens, HQ, HKV, D, THETA, dev(kc),
                                    dev(vc), cap, out)
    got = host(out)
    for b in range(B):
        w = {"q": q[b], "k": k[b], "v": v[b], "k_cache": kc[b], "v_cache": vc[b],
             "pos": int(lens[b]), "cap": cap}
        assert_close(got[b], oracle_decode(w)[4], f"seq {b} len {lens[b]}")


@pytest.mark.parametrize("pos", [40000, 70000])
def test_dev_decode_step_long_context(backend, pos):
    """Contexts past 256 splits of 128 rows: each split runs several passes
    over its rows and the last split merges its 150+ partners in rounds of
    64 (one load round trip each)."""
    case(f"fused decode step long context pos {pos}")
    import torch

    cap = pos + 64
    w = decode_workload(11, pos, cap=cap, q_scale=2.0)
    q_ref, k_ref, kc_ref, vc_ref, out_ref = oracle_decode(w)
    kc, vc = dev(w["k_cache"]), dev(w["v_cache"])
    out = torch.zeros(HQ * D, device="cuda")
    backend.dev_decode_step(dev(w["q"]), dev(w["k"]), dev(w["v"]), pos, HQ, HKV, D, THETA, kc, vc,
                            cap, out)
    np.testing.assert_array_equal(host(kc)[:, pos], kc_ref[:, pos])
    np.testing.assert_array_equal(host(vc)[:, pos], vc_ref[:, pos])
    assert_close_scaled(host(out), out_ref, f"decode pos {pos}")


def one_hot_rows(n_rows, cap):
    """Value rows one-hot at dim (t mod head_dim), every kv head alike."""
    v = np.zeros((HKV, cap, D), np.float32)
    t = np.arange(n_rows)
    v[:, t, t % D] = 1.0
    return v


def row_counts(L):
    """#{t < L : t mod head_dim = d} for every q head's dims."""
    return np.tile(np.bincount(np.arange(L) % D, minlength=D).astype(np.float64), HQ)


def check_row_counts(got, L, what):
    """out * L recovers the row counts; a row attended twice or not at all
    moves one of them by 1."""
    err = np.abs(np.asarray(got, np.float64) * L - row_counts(L))
    assert float(err.max()) <= 1e-3, f"{what}: row counts off by up to {float(err.max()):.3e}"


@pytest.mark.parametrize("waves", [8, 4])
@pytest.mark.parametrize("pos", [40000, 70000])
def test_long_context_every_row_counts(monkeypatch, waves, pos):
    """q = 0 weighs every row alike (scores 0, weights exp2(0) = 1) and value
    row t is one-hot at dim t mod 128, so out[g, d] is a count of rows over
    pos + 1, which fp32 computes to within a rounding or two.  A row attended
    twice or not at all -- a split boundary off by one, the appended row
    lost -- moves one output by 1/312 of itself or more."""
    case(f"row counts pos {pos} waves {waves}")
    import torch

    import bitnetrs_amd

    monkeypatch.setenv("BNR_DECODE_REF_WAVES", str(waves))
    be = bitnetrs_amd.HipBackend(0)
    try:
        cap = pos + 64
        kc = torch.zeros(HKV, cap, D, device="cuda")
        vc = dev(one_hot_rows(pos, cap))  # rows 0..pos-1; row pos is appended
        v_new = np.zeros((HKV, D), np.float32)
        v_new[:, pos % D] = 1.0
        q = torch.zeros(HQ * D, device="cuda")
        k = dev(oracle.normal(seed(12, 1), (HKV * D,)))
        out = torch.zeros(HQ * D, device="cuda")
        be.dev_decode_step(q, k, dev(v_new.reshape(-1)), pos, HQ, HKV, D, THETA, kc, vc, cap, out)
        check_row_counts(host(out), pos + 1, f"decode pos {pos}")
        assert np.array_equal(host(vc)[:, pos], v_new), "appended v row"
    finally:
        be.close()


def test_batched_every_row_counts(backend):
    """The row-count check through the batched launch (large launches: 4-wave
    workgroups, 64-row splits and more), lengths long and short."""
    case("batched row counts")
    import torch

    lens = np.array([40000, 100, 4097, 1, 12345, 64], np.int32)
    B, cap = len(lens), 40064
    v1 = one_hot_rows(cap, cap)
    vc = dev(np.broadcast_to(v1, (B, HKV, cap, D)))
    kc = torch.zeros(B, HKV, cap, D, device="cuda")
    v_new = np.zeros((B, HKV, D), np.float32)
    for b in range(B):
        v_new[b, :, lens[b] % D] = 1.0
    q = torch.zeros(B, HQ * D, device="cuda")
    k = dev(oracle.normal(seed(12, 2), (B, HKV * D)))
    out = torch.zeros(B, HQ * D, device="cuda")
    backend.dev_decode_step_batched(q, k, dev(v_new.reshape(B, -1)), lens, HQ, HKV, D, THETA, kc,
                                    vc, cap, out)
    got = host(out)
    for b in range(B):
        check_row_counts(got[b], int(lens[b]) + 1, f"seq {b} len {lens[b]}")


def test_dev_batched_decode_long_and_short(backend):
    """A large launch (64-row splits merged by the second kernel) with one
    sequence long enough for several passes per split and one short one."""
    case("batched decode lengths 40000 and 100")
    import torch

    lens = np.array([40000, 100], np.int32)
    B, cap = len(lens), 40064
    q = oracle.normal(seed(43, 0), (B, HQ * D))
    k = oracle.normal(seed(43, 1), (B, HKV * D))
    v = oracle.normal(seed(43, 2), (B, HKV * D))
    kc = oracle.normal(seed(43, 3), (B, HKV, cap, D))
    vc = oracle.normal(seed(43, 4), (B, HKV, cap, D))
    out = torch.zeros(B, HQ * D, device="cuda")
    backend.dev_decode_step_batched(dev(q), dev(k), dev(v), lens, HQ, HKV, D, THETA, dev(kc),
                                    dev(vc), cap, out)
    got = host(out)
    for b in range(B):
        w = {"q": q[b], "k": k[b], "v": v[b], "k_cache": kc[b], "v_cache": vc[b],
             "pos": int(lens[b]), "cap": cap}
        assert_close_scaled(got[b], oracle_decode(w)[4], f"seq {b} len {lens[b]}")


@pytest.mark.parametrize("n_tokens,start", [(2048, 0), (100, 0), (37, 200)])
def test_dev_prefill(backend, n_tokens, start):
    case(f"prefill n {n_tokens} start {start}")
    import torch

    cap = 2048 if start == 0 and n_tokens == 2048 else 512
    w = prefill_workload(3, n_tokens)
    cache = oracle.KVCache(1, HKV, D, cap)
    be = oracle.CpuBackend()
    d_kc = torch.zeros(HKV, cap, D, device="cuda")
    d_vc = torch.zeros_like(d_kc)
    if start:
        pre = prefill_workload(33, start)
        oracle_prefill(pre, cache=cache, backend=be)
        d_kc.copy_(torch.from_numpy(cache.k(0).reshape(HKV, cap, D)))
        d_vc.copy_(torch.from_numpy(cache.v(0).reshape(HKV, cap, D)))
    q_ref, k_ref, cache, out_ref = oracle_prefill(w, start_pos=start, cache=cache, backend=be)
    q, k = dev(w["q"]), dev(w["k"])
    out = torch.zeros(n_tokens, HQ * D, device="cuda")
    backend.dev_prefill(q, k, dev(w["v"]), n_tokens, start, HQ, HKV, D, THETA, d_kc, d_vc, cap, out)
    np.testing.assert_array_equal(host(q), q_ref)
    np.testing.assert_array_equal(host(k), k_ref)
    np.testing.assert_array_equal(host(d_kc).reshape(-1), cache.k(0))
    np.testing.assert_array_equal(host(d_vc).reshape(-1), cache.v(0))
    print(assert_close(host(out), out_ref, f"prefill {n_tokens}"))


def test_dev_argument_errors(backend):
    case("device entry point errors")
    import bitnetrs_amd
    import torch

    t = torch.zeros(HQ * D, device="cuda")
    kc = torch.zeros(HKV, 16, D, device="cuda")
    with pytest.raises(bitnetrs_amd.InvalidShape):  # position >= cap
        backend.dev_decode_step(t, t[:HKV * D], t[:HKV * D], 16, HQ, HKV, D, THETA, kc, kc, 16, t)
    with pytest.raises(bitnetrs_amd.InvalidConfig):
        backend.dev_decode_attention(t, kc, kc, 16, t, 20, 3, D, 0)
    with pytest.raises(bitnetrs_amd.InvalidConfig):
        backend.dev_rope_append(t, t, t, 1, 0, HQ, HKV, D, -1.0, kc, kc, 16)


@pytest.mark.parametrize("n_heads,n_kv,n_tokens,start", [(20, 5, 33, 0), (20, 5, 1, 0),
                                                        (20, 5, 64, 31), (16, 2, 70, 5),
                                                        (8, 4, 40, 0), (8, 8, 20, 3)])
def test_dev_prefill_shapes(backend, n_heads, n_kv, n_tokens, start):
    case(f"prefill heads {n_heads}/{n_kv} n {n_tokens} start {start}")
    import torch

    cap = start + n_tokens + 7
    cache = oracle.KVCache(1, n_kv, D, cap)
    be = oracle.CpuBackend()
    d_kc = torch.zeros(n_kv, cap, D, device="cuda")
    d_vc = torch.zeros_like(d_kc)
    if start:
        pre = prefill_workload(34, start, n_heads, n_kv)
        oracle_prefill(pre, cache=cache, backend=be, n_heads=n_heads, n_kv=n_kv)
        d_kc.copy_(torch.from_numpy(cache.k(0).reshape(n_kv, cap, D)))
        d_vc.copy_(torch.from_numpy(cache.v(0).reshape(n_kv, cap, D)))
    w = prefill_workload(35, n_tokens, n_heads, n_kv)
    q_ref, k_ref, cache, out_ref = oracle_prefill(w, start_pos=start, cache=cache, backend=be,
                                                  n_heads=n_heads, n_kv=n_kv)
    out = torch.zeros(n_tokens, n_heads * D, device="cuda")
    q_d, k_d = dev(w["q"]), dev(w["k"])
    backend.dev_prefill(q_d, k_d, dev(w["v"]), n_tokens, start, n_heads, n_kv, D,
                        THETA, d_kc, d_vc, cap, out)
    # q and k rotated in place, bit for bit
    np.testing.assert_array_equal(host(q_d), q_ref)
    np.testing.assert_array_equal(host(k_d), k_ref)
    np.testing.assert_array_equal(host(d_kc).reshape(-1), cache.k(0))
    assert_close(host(out), out_ref, f"prefill {n_heads}/{n_kv} n {n_tokens}")


@pytest.mark.parametrize("tiles,persistent", [(1, 0), (2, 0), (3, 0), (5, 0), (8, 0), (2, 1), (3, 1),
                                               (8, 1), (1 << 20, 1)])
def test_dev_prefill_key_chunks(monkeypatch, tiles, persistent):
    """Query tiles cut into key chunks of `tiles` key tiles (merged by the last
    chunk to finish), at start positions that are not tile-aligned so some
    chunks see no key at all for their first queries; two prefills in a row
    check that the merge tickets (and, persistent, the item queue) reset
    themselves.  persistent: resident workgroups take items from a queue."""
    case(f"prefill key chunks tiles {tiles} persistent {persistent}")
    import torch

    import bitnetrs_amd

    monkeypatch.setenv("BNR_PREFILL_CHUNK_TILES", str(tiles))
    monkeypatch.setenv("BNR_PREFILL_PERSISTENT", str(persistent))
    be_gpu = bitnetrs_amd.HipBackend(0)
    try:
        cap = 640
        cache = oracle.KVCache(1, HKV, D, cap)
        be = oracle.CpuBackend()
        d_kc = torch.zeros(HKV, cap, D, device="cuda")
        d_vc = torch.zeros_like(d_kc)
        pre = prefill_workload(36, 45)
        oracle_prefill(pre, cache=cache, backend=be)
        d_kc.copy_(torch.from_numpy(cache.k(0).reshape(HKV, cap, D)))
        d_vc.copy_(torch.from_numpy(cache.v(0).reshape(HKV, cap, D)))
        start = 45
        for n_tokens, s in ((300, 37), (129, 38)):
            w = prefill_workload(s, n_tokens)
            q_ref, k_ref, cache, out_ref = oracle_prefill(w, start_pos=start, cache=cache,
                                                          backend=be)
            out = torch.zeros(n_tokens, HQ * D, device="cuda")
            q_d, k_d = dev(w["q"]), dev(w["k"])
            be_gpu.dev_prefill(q_d, k_d, dev(w["v"]), n_tokens, start, HQ, HKV, D,
                               THETA, d_kc, d_vc, cap, out)
            # q and k rotated in place, bit for bit
            np.testing.assert_array_equal(host(q_d), q_ref)
            np.testing.assert_array_equal(host(k_d), k_ref)
            assert_close(host(out), out_ref, f"prefill chunks of {tiles} n {n_tokens} start {start}")
            start += n_tokens
    finally:
        be_gpu.close()


@pytest.mark.parametrize("q16", [0, 1])
@pytest.mark.parametrize("n_heads,n_kv,tiles,balanced", [(20, 5, 3, 0), (20, 5, 5, 1),
                                                         (20, 5, 1 << 20, 0), (16, 2, 4, 0),
                                                         (32, 4, 3, 0), (8, 8, 2, 1)])
def test_dev_prefill_query_height(monkeypatch, q16, n_heads, n_kv, tiles, balanced):
    """32-query tiles (prefill_kernel) and 16-query halves (prefill16_kernel)
    forced on the same launches: chunked and whole query tiles, plain and
    balanced chunks, 2 to 8 q heads per kv head, token counts that leave the
    last tile's second half empty (n % 32 <= 16) or partly filled, and start
    positions off the tile grid; two prefills in a row so that the halves'
    tickets reset themselves.  Rotated q/k and cache rows bit for bit."""
    case(f"prefill q16 {q16} heads {n_heads}/{n_kv} tiles {tiles} balanced {balanced}")
    import torch

    import bitnetrs_amd

    monkeypatch.setenv("BNR_PREFILL_Q16", str(q16))
    monkeypatch.setenv("BNR_PREFILL_CHUNK_TILES", str(tiles))
    monkeypatch.setenv("BNR_PREFILL_BALANCED", str(balanced))
    be_gpu = bitnetrs_amd.HipBackend(0)
    try:
        cap = 700
        cache = oracle.KVCache(1, n_kv, D, cap)
        be = oracle.CpuBackend()
        d_kc = torch.zeros(n_kv, cap, D, device="cuda")
        d_vc = torch.zeros_like(d_kc)
        pre = prefill_workload(53, 29, n_heads, n_kv)
        oracle_prefill(pre, cache=cache, backend=be, n_heads=n_heads, n_kv=n_kv)
        d_kc.copy_(torch.from_numpy(cache.k(0).reshape(n_kv, cap, D)))
        d_vc.copy_(torch.from_numpy(cache.v(0).reshape(n_kv, cap, D)))
        start = 29
        for n_tokens, sd in ((272, 54), (210, 55), (17, 56)):
            w = prefill_workload(sd, n_tokens, n_heads, n_kv)
            q_ref, k_ref, cache, out_ref = oracle_prefill(w, start_pos=start, cache=cache,
                                                          backend=be, n_heads=n_heads, n_kv=n_kv)
            out = torch.zeros(n_tokens, n_heads * D, device="cuda")
            q_d, k_d = dev(w["q"]), dev(w["k"])
            be_gpu.dev_prefill(q_d, k_d, dev(w["v"]), n_tokens, start, n_heads, n_kv, D, THETA,
                               d_kc, d_vc, cap, out)
            np.testing.assert_array_equal(host(q_d), q_ref)
            np.testing.assert_array_equal(host(k_d), k_ref)
            np.testing.assert_array_equal(host(d_kc).reshape(-1), cache.k(0))
            assert_close(host(out), out_ref,
                         f"prefill q16 {q16} {n_heads}/{n_kv} tiles {tiles} n {n_tokens} "
                         f"start {start}")
            start += n_tokens
    finally:
        be_gpu.close()


@pytest.mark.parametrize("n_heads,n_kv,start,lens", [(20, 5, 29, (272, 210, 17)),
                                                     (20, 5, 0, (1024,)),
                                                     (20, 5, 512, (512, 100)),
                                                     (20, 5, 1500, (40, 1)),
                                                     (16, 2, 45, (230, 33)),
                                                     (8, 4, 3, (200, 64))])
def test_dev_prefill_paired(monkeypatch, n_heads, n_kv, start, lens):
    """Paired launches of the 16-query kernel forced (one dispatch round,
    at most two key-range pieces of 16-query units per bin): whole units
    paired, long units cut into chains of pieces whose last finisher merges
    the others, the 30-layer stack's 1024-token shape, launches after a
    prefix whose units are all cut, a single token, 2 to 8 q heads per kv
    head, and launches in a row so that the tickets reset themselves.
    Rotated q/k and cache rows bit for bit, outputs within tolerance."""
    case(f"prefill paired heads {n_heads}/{n_kv} start {start} lens {lens}")
    import torch

    import bitnetrs_amd

    monkeypatch.setenv("BNR_PREFILL_PAIR", "1")
    be_gpu = bitnetrs_amd.HipBackend(0)
    try:
        cap = start + sum(lens) + 40
        cache = oracle.KVCache(1, n_kv, D, cap)
        be = oracle.CpuBackend()
        d_kc = torch.zeros(n_kv, cap, D, device="cuda")
        d_vc = torch.zeros_like(d_kc)
        if start:
            pre = prefill_workload(61, start, n_heads, n_kv)
            oracle_prefill(pre, cache=cache, backend=be, n_heads=n_heads, n_kv=n_kv)
            d_kc.copy_(torch.from_numpy(cache.k(0).reshape(n_kv, cap, D)))
            d_vc.copy_(torch.from_numpy(cache.v(0).reshape(n_kv, cap, D)))
        for i, n_tokens in enumerate(lens):
            w = prefill_workload(62 + i, n_tokens, n_heads, n_kv)
            q_ref, k_ref, cache, out_ref = oracle_prefill(w, start_pos=start, cache=cache,
                                                          backend=be, n_heads=n_heads, n_kv=n_kv)
            out = torch.zeros(n_tokens, n_heads * D, device="cuda")
            q_d, k_d = dev(w["q"]), dev(w["k"])
            be_gpu.dev_prefill(q_d, k_d, dev(w["v"]), n_tokens, start, n_heads, n_kv, D, THETA,
                               d_kc, d_vc, cap, out)
            np.testing.assert_array_equal(host(q_d), q_ref)
            np.testing.assert_array_equal(host(k_d), k_ref)
            np.testing.assert_array_equal(host(d_kc).reshape(-1), cache.k(0))
            assert_close(host(out), out_ref,
                         f"prefill paired {n_heads}/{n_kv} n {n_tokens} start {start}")
            start += n_tokens
    finally:
        be_gpu.close()


@pytest.mark.parametrize("n_heads,n_kv,tiles,persistent", [(16, 2, 2, 0), (16, 2, 3, 1),
                                                           (8, 4, 3, 0), (8, 4, 2, 1)])
def test_dev_prefill_key_chunks_groups(monkeypatch, n_heads, n_kv, tiles, persistent):
    """Key-chunk merges with 8 and 2 query heads per kv head (8 and 2 waves
    per workgroup; the persistent kernel keeps one workgroup of 8 waves per
    CU): 230 queries after 45 cached rows, two launches in a row."""
    case(f"prefill key chunks heads {n_heads}/{n_kv} tiles {tiles} persistent {persistent}")
    import torch

    import bitnetrs_amd

    monkeypatch.setenv("BNR_PREFILL_CHUNK_TILES", str(tiles))
    monkeypatch.setenv("BNR_PREFILL_PERSISTENT", str(persistent))
    be_gpu = bitnetrs_amd.HipBackend(0)
    try:
        cap = 520
        cache = oracle.KVCache(1, n_kv, D, cap)
        be = oracle.CpuBackend()
        d_kc = torch.zeros(n_kv, cap, D, device="cuda")
        d_vc = torch.zeros_like(d_kc)
        pre = prefill_workload(40, 45, n_heads, n_kv)
        oracle_prefill(pre, cache=cache, backend=be, n_heads=n_heads, n_kv=n_kv)
        d_kc.copy_(torch.from_numpy(cache.k(0).reshape(n_kv, cap, D)))
        d_vc.copy_(torch.from_numpy(cache.v(0).reshape(n_kv, cap, D)))
        start = 45
        for n_tokens, s in ((230, 41), (200, 42)):
            w = prefill_workload(s, n_tokens, n_heads, n_kv)
            q_ref, k_ref, cache, out_ref = oracle_prefill(w, start_pos=start, cache=cache,
                                                          backend=be, n_heads=n_heads, n_kv=n_kv)
            out = torch.zeros(n_tokens, n_heads * D, device="cuda")
            q_d, k_d = dev(w["q"]), dev(w["k"])
            be_gpu.dev_prefill(q_d, k_d, dev(w["v"]), n_tokens, start, n_heads,
                               n_kv, D, THETA, d_kc, d_vc, cap, out)
            # q and k rotated in place, bit for bit
            np.testing.assert_array_equal(host(q_d), q_ref)
            np.testing.assert_array_equal(host(k_d), k_ref)
            np.testing.assert_array_equal(host(d_kc).reshape(-1), cache.k(0))
            assert_close(host(out), out_ref,
                         f"prefill {n_heads}/{n_kv} chunks of {tiles} n {n_tokens} start {start}")
            start += n_tokens
    finally:
        be_gpu.close()


@pytest.mark.parametrize("n_heads,n_kv,tiles,persistent", [(20, 5, 2, 0), (20, 5, 3, 0), (20, 5, 5, 0),
                                                           (20, 5, 7, 0), (20, 5, 3, 1), (20, 5, 6, 1),
                                                           (16, 2, 3, 0), (16, 2, 5, 1), (8, 4, 4, 0),
                                                           (8, 4, 3, 1)])
def test_dev_prefill_balanced_chunks(monkeypatch, n_heads, n_kv, tiles, persistent):
    """Balanced key chunks (a query tile's chunks differ by at most one key
    tile, dispatched longest first): queries after cached rows that are not
    tile-aligned, 2, 4 and 8 query heads per kv head, grid and persistent
    launches, and two launches in a row (the merge tickets reset
    themselves)."""
    case(f"prefill balanced chunks heads {n_heads}/{n_kv} tiles {tiles} persistent {persistent}")
    import torch

    import bitnetrs_amd

    monkeypatch.setenv("BNR_PREFILL_CHUNK_TILES", str(tiles))
    monkeypatch.setenv("BNR_PREFILL_BALANCED", "1")
    monkeypatch.setenv("BNR_PREFILL_PERSISTENT", str(persistent))
    be_gpu = bitnetrs_amd.HipBackend(0)
    try:
        cap = 640
        cache = oracle.KVCache(1, n_kv, D, cap)
        be = oracle.CpuBackend()
        d_kc = torch.zeros(n_kv, cap, D, device="cuda")
        d_vc = torch.zeros_like(d_kc)
        pre = prefill_workload(46, 45, n_heads, n_kv)
        oracle_prefill(pre, cache=cache, backend=be, n_heads=n_heads, n_kv=n_kv)
        d_kc.copy_(torch.from_numpy(cache.k(0).reshape(n_kv, cap, D)))
        d_vc.copy_(torch.from_numpy(cache.v(0).reshape(n_kv, cap, D)))
        start = 45
        for n_tokens, s in ((300, 47), (129, 48)):
            w = prefill_workload(s, n_tokens, n_heads, n_kv)
            q_ref, k_ref, cache, out_ref = oracle_prefill(w, start_pos=start, cache=cache,
                                                          backend=be, n_heads=n_heads, n_kv=n_kv)
            out = torch.zeros(n_tokens, n_heads * D, device="cuda")
            q_d, k_d = dev(w["q"]), dev(w["k"])
            be_gpu.dev_prefill(q_d, k_d, dev(w["v"]), n_tokens, start, n_heads,
                               n_kv, D, THETA, d_kc, d_vc, cap, out)
            # q and k rotated in place, bit for bit
            np.testing.assert_array_equal(host(q_d), q_ref)
            np.testing.assert_array_equal(host(k_d), k_ref)
            np.testing.assert_array_equal(host(d_kc).reshape(-1), cache.k(0))
            assert_close(host(out), out_ref,
                         f"prefill balanced {n_heads}/{n_kv} chunks of {tiles} n {n_tokens} "
                         f"start {start}")
            start += n_tokens
    finally:
        be_gpu.close()


@pytest.mark.parametrize("n_heads,n_kv,wgs", [(20, 5, 0), (20, 5, 1), (20, 5, 3), (20, 5, 37),
                                              (16, 2, 0), (16, 2, 5), (8, 4, 0), (8, 4, 11)])
def test_dev_prefill_streamk(monkeypatch, n_heads, n_kv, wgs):
    """Stream-K prefill (the default tiled launch) with every resident slot
    (wgs 0) and with few workgroups, so that runs hold many segments and a
    query tile's key tiles are split over several runs at arbitrary points:
    queries after cached rows that are not tile-aligned (some segments see no
    key for their first queries), 2, 4 and 8 query heads per kv head, and two
    launches in a row (the merge tickets reset themselves)."""
    case(f"prefill stream-K heads {n_heads}/{n_kv} workgroups {wgs}")
    import torch

    import bitnetrs_amd

    monkeypatch.setenv("BNR_PREFILL_MODE", "2")
    monkeypatch.setenv("BNR_PREFILL_SK_WGS", str(wgs))
    be_gpu = bitnetrs_amd.HipBackend(0)
    try:
        cap = 700
        cache = oracle.KVCache(1, n_kv, D, cap)
        be = oracle.CpuBackend()
        d_kc = torch.zeros(n_kv, cap, D, device="cuda")
        d_vc = torch.zeros_like(d_kc)
        pre = prefill_workload(44, 45, n_heads, n_kv)
        oracle_prefill(pre, cache=cache, backend=be, n_heads=n_heads, n_kv=n_kv)
        d_kc.copy_(torch.from_numpy(cache.k(0).reshape(n_kv, cap, D)))
        d_vc.copy_(torch.from_numpy(cache.v(0).reshape(n_kv, cap, D)))
        start = 45
        for n_tokens, s in ((333, 45), (1, 46), (300, 47)):
            w = prefill_workload(s, n_tokens, n_heads, n_kv)
            q_ref, k_ref, cache, out_ref = oracle_prefill(w, start_pos=start, cache=cache,
                                                          backend=be, n_heads=n_heads, n_kv=n_kv)
            out = torch.zeros(n_tokens, n_heads * D, device="cuda")
            q_d, k_d = dev(w["q"]), dev(w["k"])
            be_gpu.dev_prefill(q_d, k_d, dev(w["v"]), n_tokens, start, n_heads,
                               n_kv, D, THETA, d_kc, d_vc, cap, out)
            # q and k rotated in place, bit for bit
            np.testing.assert_array_equal(host(q_d), q_ref)
            np.testing.assert_array_equal(host(k_d), k_ref)
            np.testing.assert_array_equal(host(d_kc).reshape(-1), cache.k(0))
            assert_close_scaled(host(out), out_ref,
                                f"stream-K {n_heads}/{n_kv} wgs {wgs} n {n_tokens} start {start}")
            start += n_tokens
    finally:
        be_gpu.close()
