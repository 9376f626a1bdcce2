"""GPU parity of the deterministic ways a split-K decode launch merges its
splits: a second kernel (0), the last workgroup to take a ticket (1), and the
reference merge's deterministic form (3: splits store (m, l, O), the last
workgroup combines them in a fixed order).  Each mode is
forced on a fresh context and run over consecutive launches with different
split counts on the same workspace, so every launch also checks that the
previous one left the merge state clean (tickets back at zero).
References: the oracle's rope_embed -> store_kv -> masked_attention
(bitnet-cpu/src/rope.rs:414-430, bitnet-model/src/lib.rs:184-236,
bitnet-cpu/src/attention.rs:97-209)."""
import sys

import numpy as np
import pytest

import oracle
from common import (D, HKV, HQ, THETA, assert_close, decode_workload, oracle_decode, seed)

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


def fresh_backend(monkeypatch, mode, rpg=None):
    import bitnetrs_amd

    monkeypatch.setenv("BNR_DECODE_MERGE", str(mode))
    if rpg:
        monkeypatch.setenv("BNR_DECODE_RPG", str(rpg))
    return bitnetrs_amd.HipBackend(0)


def decode_step(be, w, n_heads=HQ, n_kv=HKV, hd=D):
    import torch

    kc, vc = dev(w["k_cache"]), dev(w["v_cache"])
    out = torch.zeros(n_heads * hd, device="cuda")
    be.dev_decode_step(dev(w["q"]), dev(w["k"]), dev(w["v"]), w["pos"], n_heads, n_kv, hd, THETA,
                       kc, vc, w["cap"], out)
    return host(out), host(kc)


@pytest.mark.parametrize("mode,rpg", [(0, 1), (0, 2), (0, 8), (1, 1), (1, 2), (1, 3), (1, 5),
                                      (1, 6), (1, 7), (1, 8), (1, None), (3, None), (3, 1),
                                      (3, 2)])
def test_decode_merge_modes_consecutive(monkeypatch, mode, rpg):
    """Positions 300, 900, 2000, 64, 4095 in a row.  With 16*rpg rows per
    split these give 1..128 splits per kv head: merge rounds of 16, 32, 48
    and 64 splits, and two rounds above 64.  rpg None: the planner's
    choice (the smallest split that fits one workgroup per CU)."""
    be = fresh_backend(monkeypatch, mode, rpg)
    try:
        for i, pos in enumerate((300, 900, 2000, 64, 4095)):
            case(f"merge mode {mode} rpg {rpg} pos {pos}")
            w = decode_workload(60 + i, pos, cap=4096, q_scale=2.0)
            _, k_ref, kc_ref, _, out_ref = oracle_decode(w)
            out, kc = decode_step(be, w)
            np.testing.assert_array_equal(kc[:, pos], kc_ref[:, pos])
            assert_close(out, out_ref, f"mode {mode} rpg {rpg} pos {pos}")
    finally:
        be.close()


@pytest.mark.parametrize("mode", [0, 1, 3])
@pytest.mark.parametrize("n_heads,n_kv", [(8, 4), (4, 4), (8, 2)])
def test_decode_merge_group_sizes(monkeypatch, mode, n_heads, n_kv):
    """Both merges with 2 and 1 query heads per kv head and with 4 at two kv
    heads."""
    be = fresh_backend(monkeypatch, mode)
    try:
        for i, pos in enumerate((700, 1500)):
            case(f"merge mode {mode} heads {n_heads}/{n_kv} pos {pos}")
            w = decode_workload(70 + i, pos, cap=2048, n_heads=n_heads, n_kv=n_kv)
            out_ref = oracle_decode(w, n_heads, n_kv, D)[4]
            out, _ = decode_step(be, w, n_heads, n_kv)
            assert_close(out, out_ref, f"mode {mode} {n_heads}/{n_kv} pos {pos}")
    finally:
        be.close()


@pytest.mark.parametrize("mode", [0, 1, 3])
def test_decode_merge_ragged_batch(monkeypatch, mode):
    """A small batched launch (split counts differ per sequence, so workgroups
    past a sequence's count exit at once) under both merges, twice."""
    import torch

    be = fresh_backend(monkeypatch, mode)
    try:
        lens = np.array([100, 700, 1500], np.int32)
        B, cap = len(lens), 2048
        for rep in range(2):
            case(f"merge mode {mode} ragged batch {lens.tolist()} rep {rep}")
            q = oracle.normal(seed(80 + rep, 0), (B, HQ * D))
            k = oracle.normal(seed(80 + rep, 1), (B, HKV * D))
            v = oracle.normal(seed(80 + rep, 2), (B, HKV * D))
            kc = oracle.normal(seed(80 + rep, 3), (B, HKV, cap, D))
            vc = oracle.normal(seed(80 + rep, 4), (B, HKV, cap, D))
            out = torch.zeros(B, HQ * D, device="cuda")
            be.dev_decode_step_batched(dev(q), dev(k), dev(v), lens, HQ, HKV, D, THETA, dev(kc),
                                       dev(vc), cap, out)
            got = host(out)
            for b in range(B):
                w = {"q": q[b], "k": k[b], "v": v[b], "k_cache": kc[b], "v_cache": vc[b],
                     "pos": int(lens[b]), "cap": cap}
                assert_close(got[b], oracle_decode(w)[4], f"seq {b} len {lens[b]}")
    finally:
        be.close()


def test_deterministic_reference_merge_bit_identical(monkeypatch):
    """Mode 3 gives the same bits run after run: C2 (4095 cached rows, q x4),
    the same launch with planted rows that send two splits to the exact path,
    and a ragged batch, each run 5 times on rotated copies of the inputs."""
    import torch

    be = fresh_backend(monkeypatch, 3)
    try:
        w = decode_workload(2, 4095, cap=4096, q_scale=4.0)
        w2 = decode_workload(2, 4095, cap=4096, q_scale=4.0)
        qr = oracle_decode(w2)[0].reshape(HQ, D)  # rotated q
        for t in (200, 3100):
            w2["k_cache"][1, t] = (8.0 * qr[1 * (HQ // HKV)]).astype(f32)
        for label, ww in (("C2", w), ("C2 with exact-path splits", w2)):
            outs = []
            for rep in range(5):
                case(f"deterministic merge {label} run {rep}")
                out, _ = decode_step(be, ww)
                outs.append(out)
            assert_close(outs[0], oracle_decode(ww)[4], label)
            for o in outs[1:]:
                np.testing.assert_array_equal(o, outs[0])
        lens = np.array([130, 4095, 1, 2000], np.int32)
        B, cap = len(lens), 4096
        q = oracle.normal(seed(85, 0), (B, HQ * D))
        k = oracle.normal(seed(85, 1), (B, HKV * D))
        v = oracle.normal(seed(85, 2), (B, HKV * D))
        kc = oracle.normal(seed(85, 3), (B, HKV, cap, D))
        vc = oracle.normal(seed(85, 4), (B, HKV, cap, D))
        outs = []
        for rep in range(5):
            case(f"deterministic merge ragged batch run {rep}")
            out = torch.zeros(B, HQ * D, device="cuda")
            be.dev_decode_step_batched(dev(q), dev(k), dev(v), lens, HQ, HKV, D, THETA, dev(kc),
                                       dev(vc), cap, out)
            outs.append(host(out))
        for o in outs[1:]:
            np.testing.assert_array_equal(o, outs[0])
    finally:
        be.close()


def test_set_deterministic_host_path_bit_identical():
    """bnr_set_deterministic through the host-slice masked_attention (the
    trait path, completion words included): 4 runs at 3000 rows give the
    same bits and agree with the oracle; switched off again, the default
    merge still agrees with the oracle."""
    import bitnetrs_amd

    be = bitnetrs_amd.HipBackend(0)
    try:
        w = decode_workload(86, 3000, cap=4096, q_scale=4.0)
        q_rot, _, kc, vc, out_ref = oracle_decode(w)
        be.set_deterministic(True)
        outs = []
        for rep in range(4):
            case(f"set_deterministic host masked_attention run {rep}")
            be.mirror_invalidate()
            out = np.zeros(HQ * D, f32)
            be.masked_attention(q_rot, kc.reshape(-1), vc.reshape(-1), out, HQ, HKV, D, w["pos"])
            outs.append(out)
        assert_close(outs[0], out_ref, "deterministic host path")
        for o in outs[1:]:
            np.testing.assert_array_equal(o, outs[0])
        be.set_deterministic(False)
        be.mirror_invalidate()
        out = np.zeros(HQ * D, f32)
        be.masked_attention(q_rot, kc.reshape(-1), vc.reshape(-1), out, HQ, HKV, D, w["pos"])
        assert_close(out, out_ref, "default merge after switching back")
    finally:
        be.close()
