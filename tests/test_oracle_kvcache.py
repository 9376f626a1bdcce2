"""Pins of the oracle's KVCache and per-token layer sequence against the
reference's KVCache tests (bitnet-model/src/lib.rs:1325-1452, 1649-1700,
1753-1796) and the fp64 causal-attention definition."""
import numpy as np
import pytest

import oracle
from common import attention_f64, assert_close, oracle_prefill, prefill_workload

f32 = np.float32


def test_new_cache_is_empty():
    c = oracle.KVCache(2, 1, 4, 16)
    assert len(c) == 0 and c.layer_len(0) == 0
    assert c.k(0).size == 16 * 4


def test_store_kv_head_major_offsets():  # lib.rs:1680-1681, 218-228
    c = oracle.KVCache(1, 2, 4, 8)
    k = np.arange(8, dtype=f32)
    v = -np.arange(8, dtype=f32)
    c.store_kv(0, 0, k, v)
    c.store_kv(0, 1, k + 100, v - 100)
    K = c.k(0).reshape(2, 8, 4)
    np.testing.assert_array_equal(K[0, 0], [0, 1, 2, 3])
    np.testing.assert_array_equal(K[1, 0], [4, 5, 6, 7])
    np.testing.assert_array_equal(K[1, 1], [104, 105, 106, 107])
    np.testing.assert_array_equal(c.v(0).reshape(2, 8, 4)[0, 1], [-100, -101, -102, -103])
    assert c.layer_len(0) == 2


def test_store_kv_errors():  # lib.rs:197-216, 1395-1411
    c = oracle.KVCache(1, 1, 4, 2)
    kv = np.full(4, 0.25, f32)
    with pytest.raises(oracle.InvalidShape):
        c.store_kv(0, 0, np.zeros(3, f32), kv)
    with pytest.raises(oracle.InvalidShape):
        c.store_kv(0, 0, kv, np.zeros(5, f32))
    with pytest.raises(oracle.InvalidShape):  # gap
        c.store_kv(0, 1, kv, kv)
    c.store_kv(0, 0, kv, kv)
    c.store_kv(0, 1, kv, kv)
    with pytest.raises(oracle.InvalidShape, match="max_seq"):
        c.store_kv(0, 2, kv, kv)
    c.store_kv(0, 0, kv, kv)  # overwrite an existing row is allowed
    assert c.layer_len(0) == 2


def test_advance_and_clear():  # lib.rs:1347-1392, 1413-1422
    c = oracle.KVCache(2, 1, 4, 1)
    kv = np.full(4, 0.5, f32)
    c.store_kv(0, 0, kv, kv)
    c.advance()
    assert len(c) == 1
    with pytest.raises(oracle.BackendError, match="advance overflow"):
        c.advance()
    c.clear()
    assert len(c) == 0 and c.layer_len(0) == 0
    assert np.all(c.k(0) == 0) and np.all(c.v(0) == 0)


def test_layer_tokens_is_causal_attention():
    # The per-token sequence (rope -> store -> attention at cur_pos) equals
    # causal attention of the rotated q over the rotated keys 0..=i.
    n, hq, hkv, d = 24, 4, 2, 16
    w = prefill_workload(20, n, hq, hkv, d)
    q, k, cache, out = oracle_prefill(w, cap=32, n_heads=hq, n_kv=hkv, head_dim=d,
                                      theta=10000.0)
    assert cache.layer_len(0) == n
    kc, vc = cache.k(0), cache.v(0)
    np.testing.assert_array_equal(kc.reshape(hkv, 32, d)[:, :n].transpose(1, 0, 2).reshape(n, -1), k)
    for i in range(n):
        ref = attention_f64(q[i], kc, vc, hq, hkv, d, i)
        assert_close(out[i], ref, f"token {i}", atol=1e-5, rtol=1e-4)


def test_layer_tokens_decode_after_prefill():  # lib.rs:1770-1796
    n, hq, hkv, d = 10, 4, 1, 8
    w = prefill_workload(21, n + 1, hq, hkv, d)
    _, _, _, full = oracle_prefill(w, cap=16, n_heads=hq, n_kv=hkv, head_dim=d, theta=10000.0)
    be = oracle.CpuBackend()
    cache = oracle.KVCache(1, hkv, d, 16)
    first = {key: val[:n].copy() for key, val in w.items()}
    last = {key: val[n:].copy() for key, val in w.items()}
    oracle_prefill(first, cap=16, n_heads=hq, n_kv=hkv, head_dim=d, theta=10000.0, cache=cache,
                   backend=be)
    _, _, _, step = oracle_prefill(last, start_pos=n, n_heads=hq, n_kv=hkv, head_dim=d,
                                   theta=10000.0, cache=cache, backend=be)
    np.testing.assert_array_equal(step[0], full[n])
