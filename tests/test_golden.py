"""The oracle against the committed golden fixtures (tests/golden/*.npz, written
by tests/golden/gen_golden.py), and the GPU path against the same fixtures."""
import hashlib
import os

import numpy as np
import pytest

import oracle
from common import assert_close, decode_workload, oracle_decode, oracle_prefill, prefill_workload

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    return np.load(os.path.join(GOLD, name), allow_pickle=False)


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def test_inputs_regenerate_from_seeds():
    g = load("decode_c1.npz")
    w = decode_workload(1, int(g["pos"]))
    assert sha(w["q"]) == str(g["sha_q"]) and sha(w["k"]) == str(g["sha_k"])
    assert sha(w["v"]) == str(g["sha_v"]) and sha(w["k_cache"]) == str(g["sha_kc"])
    assert sha(w["v_cache"]) == str(g["sha_vc"])


def test_oracle_decode_matches_fixture():
    g = load("decode_c1.npz")
    q_rot, k_rot, _, _, out = oracle_decode(decode_workload(1, int(g["pos"])))
    np.testing.assert_array_equal(q_rot, g["q_rot"])
    np.testing.assert_array_equal(k_rot, g["k_rot"])
    np.testing.assert_array_equal(out, g["out"])


def test_oracle_prefill_matches_fixture():
    g = load("prefill_small.npz")
    p = prefill_workload(36, int(g["n_tokens"]), int(g["n_heads"]), int(g["n_kv"]))
    assert sha(p["q"]) == str(g["sha_q"])
    q_r, k_r, cache, out = oracle_prefill(p, cap=int(g["cap"]), n_heads=int(g["n_heads"]),
                                          n_kv=int(g["n_kv"]))
    assert sha(q_r) == str(g["sha_q_rot"]) and sha(k_r) == str(g["sha_k_rot"])
    assert sha(cache.k(0)) == str(g["sha_k_cache"]) and sha(cache.v(0)) == str(g["sha_v_cache"])
    np.testing.assert_array_equal(out, g["out"])


def test_oracle_rope_rows_match_fixture():
    g = load("rope_rows.npz")
    c, s = oracle.rope_table(4096, 128, 500000.0)
    np.testing.assert_array_equal(c[g["rows"]], g["cos"])
    np.testing.assert_array_equal(s[g["rows"]], g["sin"])


@pytest.mark.gpu
def test_gpu_decode_matches_fixture(backend):
    import torch

    g = load("decode_c1.npz")
    pos = int(g["pos"])
    w = decode_workload(1, pos)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    out = torch.zeros(20 * 128, device="cuda")
    q_rot = torch.zeros(20 * 128, device="cuda")
    k_rot = torch.zeros(5 * 128, device="cuda")
    backend.dev_decode_step(dev(w["q"]), dev(w["k"]), dev(w["v"]), pos, 20, 5, 128, 500000.0,
                            dev(w["k_cache"]), dev(w["v_cache"]), 4096, out, q_rot, k_rot)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(q_rot.cpu().numpy(), g["q_rot"])
    np.testing.assert_array_equal(k_rot.cpu().numpy(), g["k_rot"])
    assert_close(out.cpu().numpy(), g["out"], "C1 vs fixture")


@pytest.mark.gpu
def test_gpu_prefill_matches_fixture(backend):
    import torch

    g = load("prefill_small.npz")
    n, hq, hkv, cap = int(g["n_tokens"]), int(g["n_heads"]), int(g["n_kv"]), int(g["cap"])
    p = prefill_workload(36, n, hq, hkv)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    kc = torch.zeros(hkv, cap, 128, device="cuda")
    vc = torch.zeros_like(kc)
    q, k = dev(p["q"]), dev(p["k"])
    out = torch.zeros(n, hq * 128, device="cuda")
    backend.dev_prefill(q, k, dev(p["v"]), n, 0, hq, hkv, 128, 500000.0, kc, vc, cap, out)
    torch.cuda.synchronize()
    assert sha(q.cpu().numpy()) == str(g["sha_q_rot"])
    assert sha(kc.cpu().numpy()) == str(g["sha_k_cache"])
    assert sha(vc.cpu().numpy()) == str(g["sha_v_cache"])
    assert_close(out.cpu().numpy(), g["out"], "prefill vs fixture")
