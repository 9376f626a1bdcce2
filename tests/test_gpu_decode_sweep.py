"""Seeded sweep of the fused decode step over the planner's range: contexts
from 1 to 9000 rows (every rpg 1..8 and 1..3 passes the planner picks),
1/2/4 query heads per kv head at 1, 2, 5 and 8 kv heads, and small batched
launches of 2..6 sequences with ragged lengths (split counts differ per
sequence).  Each output is checked against the oracle's rope_embed ->
store_kv -> masked_attention (bitnet-cpu/src/rope.rs:414-430,
bitnet-model/src/lib.rs:184-236, bitnet-cpu/src/attention.rs:97-209), the
appended rows bit for bit."""
import sys

import numpy as np
import pytest

import oracle
from common import D, THETA, assert_close, decode_workload, oracle_decode, seed

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


SINGLE = [  # (n_kv, group, position)
    (5, 4, 0), (5, 4, 1), (5, 4, 15), (5, 4, 16), (5, 4, 700), (5, 4, 1023), (5, 4, 1500),
    (5, 4, 2047), (5, 4, 2500), (5, 4, 3071), (5, 4, 4095), (5, 4, 5000), (5, 4, 6143),
    (5, 4, 8191), (5, 4, 9000), (1, 4, 3000), (2, 4, 2100), (8, 2, 1300), (8, 1, 777),
    (2, 2, 4500), (1, 1, 6000),
]


@pytest.mark.parametrize("n_kv,group,pos", SINGLE)
def test_decode_step_sweep(backend, n_kv, group, pos):
    case(f"decode sweep n_kv {n_kv} group {group} pos {pos}")
    import torch

    n_heads = n_kv * group
    cap = pos + 1 + (pos % 7)
    w = decode_workload(900 + pos % 97, pos, cap=cap, q_scale=2.0, n_heads=n_heads, n_kv=n_kv)
    _, k_ref, kc_ref, vc_ref, out_ref = oracle_decode(w, n_heads, n_kv, D)
    kc, vc = dev(w["k_cache"]), dev(w["v_cache"])
    out = torch.zeros(n_heads * D, device="cuda")
    backend.dev_decode_step(dev(w["q"]), dev(w["k"]), dev(w["v"]), pos, n_heads, n_kv, D, THETA,
                            kc, vc, cap, out)
    np.testing.assert_array_equal(host(kc)[:, pos], kc_ref[:, pos])
    np.testing.assert_array_equal(host(vc)[:, pos], vc_ref[:, pos])
    assert_close(host(out), out_ref, f"n_kv {n_kv} group {group} pos {pos}")


@pytest.mark.parametrize("trial", range(6))
def test_small_batched_decode_sweep(backend, trial):
    """2..6 sequences with lengths drawn from 1..6000: small launches merged
    in-kernel, whose split counts differ per sequence."""
    import torch

    rng = np.random.default_rng(seed(95, trial))
    B = int(rng.integers(2, 7))
    lens = rng.integers(0, 6000, size=B).astype(np.int32)
    n_kv, group = [(5, 4), (2, 4), (4, 2), (3, 1), (5, 4), (8, 4)][trial]
    n_heads = n_kv * group
    cap = int(lens.max()) + 3
    case(f"small batched sweep trial {trial}: lens {lens.tolist()} n_kv {n_kv} group {group}")
    q = oracle.normal(seed(96, trial), (B, n_heads * D))
    k = oracle.normal(seed(97, trial), (B, n_kv * D))
    v = oracle.normal(seed(98, trial), (B, n_kv * D))
    kc = oracle.normal(seed(99, trial), (B, n_kv, cap, D))
    vc = oracle.normal(seed(100, trial), (B, n_kv, cap, D))
    out = torch.zeros(B, n_heads * D, device="cuda")
    d_kc = dev(kc)
    backend.dev_decode_step_batched(dev(q), dev(k), dev(v), lens, n_heads, n_kv, D, THETA, d_kc,
                                    dev(vc), cap, out)
    got, gk = host(out), host(d_kc)
    for b in range(B):
        w = {"q": q[b], "k": k[b], "v": v[b], "k_cache": kc[b], "v_cache": vc[b],
             "pos": int(lens[b]), "cap": cap}
        _, k_ref, _, _, out_ref = oracle_decode(w, n_heads, n_kv, D)
        np.testing.assert_array_equal(gk[b][:, lens[b]], k_ref.reshape(n_kv, D))
        assert_close(got[b], out_ref, f"trial {trial} seq {b} len {lens[b]}")
