"""GPU parity of the reference merge of the split-K decode (merge mode 2):
splits weigh their rows against the score of the newest row and add their
sums with device-scope atomics.  Covers the plain case over the planner's
range, consecutive launches on one context (the accumulators must come back
to zero), both workgroup shapes (8 and 4 waves), and the exact path: splits
whose scores run more than 2^64 above the reference keep their own maximum
and are folded in by the merging workgroup.  Planted rows make single
splits, several splits, the newest row's own split and every split take it.
References: the oracle's rope_embed -> store_kv -> masked_attention
(bitnet-cpu/src/rope.rs:414-430, bitnet-model/src/lib.rs:184-236,
bitnet-cpu/src/attention.rs:97-209)."""
import sys

import numpy as np
import pytest

import oracle
from common import (D, HKV, HQ, THETA, assert_close_scaled, decode_workload, oracle_decode)

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


@pytest.fixture(params=[8, 4], ids=["8waves", "4waves"])
def ref_backend(monkeypatch, request):
    # Small launches run 8-wave workgroups by default; the 4-wave kernel (the
    # large launches' one) is forced on the same cases.
    import bitnetrs_amd

    monkeypatch.setenv("BNR_DECODE_MERGE", "2")
    monkeypatch.setenv("BNR_DECODE_REF_WAVES", str(request.param))
    be = bitnetrs_amd.HipBackend(0)
    yield be
    be.close()


def decode_step(be, w, n_heads=HQ, n_kv=HKV, hd=D):
    import torch

    kc, vc = dev(w["k_cache"]), dev(w["v_cache"])
    out = torch.zeros(n_heads * hd, device="cuda")
    be.dev_decode_step(dev(w["q"]), dev(w["k"]), dev(w["v"]), w["pos"], n_heads, n_kv, hd, THETA,
                       kc, vc, w["cap"], out)
    return host(out), host(kc), host(vc)


def check(be, w, what, n_heads=HQ, n_kv=HKV, hd=D):
    case(what)
    out, kc, vc = decode_step(be, w, n_heads, n_kv, hd)
    _, _, kc_ref, vc_ref, ref = oracle_decode(w, n_heads, n_kv, hd)
    assert np.array_equal(kc[:, w["pos"]], kc_ref[:, w["pos"]]), f"{what}: appended k row"
    assert np.array_equal(vc[:, w["pos"]], vc_ref[:, w["pos"]]), f"{what}: appended v row"
    return assert_close_scaled(out, ref, what)


@pytest.mark.parametrize("pos", [0, 1, 15, 16, 95, 96, 97, 511, 1000, 2047, 4095, 8191, 20000])
def test_ref_merge_lengths(ref_backend, pos):
    w = decode_workload(60, pos, cap=max(4096, pos + 1), q_scale=4.0 if pos == 4095 else 1.0)
    check(ref_backend, w, f"ref merge pos {pos}")


@pytest.mark.parametrize("n_heads,n_kv", [(8, 8), (8, 4), (16, 4), (4, 1)])
def test_ref_merge_group_sizes(ref_backend, n_heads, n_kv):
    w = decode_workload(61, 3000, cap=4096, n_heads=n_heads, n_kv=n_kv)
    check(ref_backend, w, f"ref merge {n_heads}/{n_kv} heads", n_heads, n_kv)


def test_ref_merge_consecutive(ref_backend):
    # Different split counts on one context: every launch must find the
    # accumulators, masks and tickets it left at zero.
    for i, pos in enumerate([4095, 700, 4095, 33, 2500, 4095]):
        w = decode_workload(62 + i, pos, cap=4096, q_scale=2.0)
        check(ref_backend, w, f"consecutive launch {i} pos {pos}")


def rotated_q(w, n_heads=HQ, n_kv=HKV, hd=D):
    q = w["q"].copy()
    k = w["k"].copy()
    oracle.CpuBackend().rope_embed(q, k, w["pos"], hd, n_heads, n_kv, THETA)
    return q.reshape(n_heads, hd)


def plant(w, rows, head, scale):
    """Cache rows `rows` of kv head `head` become scale * (rotated q of the
    group's first q head): their scores exceed the rest by ~scale*|q|^2/sqrt(d)."""
    qr = rotated_q(w)
    g = HQ // HKV
    for t in rows:
        w["k_cache"][head, t] = (scale * qr[head * g]).astype(f32)
    return w


@pytest.mark.parametrize("rows,head", [([100], 0), ([1234], 2), ([5, 900, 2100, 3900], 4),
                                       ([4000], 1), ([0, 4094], 3)])
def test_ref_merge_exact_path_planted(ref_backend, rows, head):
    # scale 8: ~8*128/11.3 = 90 natural units = 130 log2 units above the rest
    w = plant(decode_workload(63, 4095, cap=4096), rows, head, 8.0)
    check(ref_backend, w, f"planted rows {rows} in kv head {head}")


def test_ref_merge_exact_path_every_split(ref_backend):
    # The newest key points away from q: its score (the reference) sits far
    # below every other row, so every split of every head takes the exact path.
    w = decode_workload(64, 3000, cap=4096)
    qr = rotated_q(w)
    g = HQ // HKV
    k = w["k"].reshape(HKV, D)
    # raw k whose rotation is -8 * q_rot: rotate back by the inverse angle
    for h in range(HKV):
        target = (-8.0 * qr[h * g]).astype(f32)
        k[h] = oracle_unrotate(target, w["pos"])
    w["k"] = k.reshape(-1).astype(f32)
    check(ref_backend, w, "every split on the exact path")


def oracle_unrotate(x, pos):
    """Raw key whose half-split rotation at `pos` is (close to) x: rotation
    by the negative angle, in float64."""
    half = D // 2
    i = np.arange(half, dtype=np.float64)
    ang = pos * THETA ** (-2.0 * i / D)
    c, s = np.cos(ang), np.sin(ang)
    lo, hi = x[:half].astype(np.float64), x[half:].astype(np.float64)
    return np.concatenate([lo * c + hi * s, hi * c - lo * s]).astype(f32)


def test_ref_merge_exact_then_plain(ref_backend):
    # A launch with flagged splits, then plain launches: the masks are cleared.
    w = plant(decode_workload(65, 4095, cap=4096), [50, 3000], 0, 8.0)
    check(ref_backend, w, "flagged launch")
    for i, pos in enumerate([4095, 1500]):
        check(ref_backend, decode_workload(66 + i, pos, cap=4096), f"plain launch after flags {i}")


def test_ref_merge_batched(ref_backend):
    import torch

    lens = np.array([130, 4095, 1, 2000, 3999, 64, 700, 2048], np.int32)
    n = lens.size
    ws = [decode_workload(70 + i, int(L), cap=4096) for i, L in enumerate(lens)]
    plant(ws[3], [10], 2, 8.0)
    q = dev(np.stack([w["q"] for w in ws]))
    k = dev(np.stack([w["k"] for w in ws]))
    v = dev(np.stack([w["v"] for w in ws]))
    kc = dev(np.stack([w["k_cache"] for w in ws]))
    vc = dev(np.stack([w["v_cache"] for w in ws]))
    out = torch.zeros(n, HQ * D, device="cuda")
    case("ref merge batched 8 sequences")
    ref_backend.dev_decode_step_batched(q, k, v, lens, HQ, HKV, D, THETA, kc, vc, 4096, out)
    got = host(out)
    for i, w in enumerate(ws):
        _, _, _, _, ref = oracle_decode(w)
        assert_close_scaled(got[i], ref, f"batched sequence {i} pos {lens[i]}")


@pytest.mark.parametrize("mode", [None, 1])
@pytest.mark.parametrize("n_heads,n_kv,pos", [(8, 8, 16), (8, 8, 32), (20, 5, 16), (4, 4, 48),
                                              (8, 2, 64)])
def test_split_starting_at_position_poisoned(monkeypatch, mode, n_heads, n_kv, pos):
    # Rows past a split's end are loaded clamped onto its first row, with
    # weight 0.  When a split starts at `position`, that row is the one this
    # launch appends: it must come from the new k/v, not from the cache,
    # whose row here holds NaN and inf (0 * inf would be NaN).
    import torch

    import bitnetrs_amd

    if mode is not None:
        monkeypatch.setenv("BNR_DECODE_MERGE", str(mode))
        monkeypatch.setenv("BNR_DECODE_RPG", "1")
    be = bitnetrs_amd.HipBackend(0)
    try:
        w = decode_workload(80 + pos, pos, cap=128, n_heads=n_heads, n_kv=n_kv)
        poisoned = w["k_cache"].copy(), w["v_cache"].copy()
        for c in poisoned:
            c[:, pos::2] = np.nan
            c[:, pos + 1::2] = np.inf
        case(f"split at position {pos}, heads {n_heads}/{n_kv}, merge {mode}")
        kc, vc = dev(poisoned[0]), dev(poisoned[1])
        out = torch.zeros(n_heads * D, device="cuda")
        be.dev_decode_step(dev(w["q"]), dev(w["k"]), dev(w["v"]), pos, n_heads, n_kv, D, THETA,
                           kc, vc, 128, out)
        _, _, kc_ref, vc_ref, ref = oracle_decode(w, n_heads, n_kv)
        assert np.array_equal(host(kc)[:, pos], kc_ref[:, pos])
        assert np.array_equal(host(vc)[:, pos], vc_ref[:, pos])
        assert_close_scaled(host(out), ref, f"split at position {pos}")
    finally:
        be.close()
