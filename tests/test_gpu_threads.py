"""Concurrent use of one context.  Backend is Send + Sync
(bitnet-core/src/backend/mod.rs:128) and the engine shares it as
Arc<dyn Backend> (bitnet-model/src/device.rs:367-385), so the trait's &self
methods may run at the same time from several threads.  The C side
serialises a context's host entry points with its mutex; each thread's host
KV cache keeps its own HBM mirror.  Results are checked against the oracle's
per-token sequence rope_embed -> store_kv -> masked_attention
(bitnet-model/src/lib.rs:1004-1036)."""
import sys
import threading

import numpy as np
import pytest

import oracle
from common import D, HKV, HQ, THETA, assert_close, seed

pytestmark = pytest.mark.gpu
f32 = np.float32


def case(msg):
    print(f"[gpu case] {msg}", flush=True)
    sys.stdout.flush()


def sequence(cfg, n_steps, cap):
    """Inputs of n_steps decode tokens and the oracle's outputs for them."""
    be = oracle.CpuBackend()
    kc = np.zeros((HKV, cap, D), f32)
    vc = np.zeros_like(kc)
    steps = []
    for pos in range(n_steps):
        q = oracle.normal(seed(cfg, 3 * pos), (HQ * D,))
        k = oracle.normal(seed(cfg, 3 * pos + 1), (HKV * D,))
        v = oracle.normal(seed(cfg, 3 * pos + 2), (HKV * D,))
        qr, kr = q.copy(), k.copy()
        be.rope_embed(qr, kr, pos, D, HQ, HKV, THETA)
        kc[:, pos] = kr.reshape(HKV, D)
        vc[:, pos] = v.reshape(HKV, D)
        out = np.zeros(HQ * D, f32)
        be.masked_attention(qr, kc.reshape(-1), vc.reshape(-1), out, HQ, HKV, D, pos)
        steps.append((q, k, v, qr, kr, out))
    return steps


def test_host_entry_points_from_threads(backend):
    """Four threads share one context; each runs its own 24-token decode
    sequence through rope_embed and masked_attention on its own host cache."""
    case("host rope_embed + masked_attention from 4 threads sharing one context")
    backend.mirror_invalidate()  # recycled host addresses must not look in sync
    n_threads, n_steps, cap = 4, 24, 64
    refs = [sequence(700 + t, n_steps, cap) for t in range(n_threads)]
    errors = []

    def run(t):
        try:
            kc = np.zeros(HKV * cap * D, f32)
            vc = np.zeros_like(kc)
            k3, v3 = kc.reshape(HKV, cap, D), vc.reshape(HKV, cap, D)
            for pos, (q, k, v, qr, kr, out_ref) in enumerate(refs[t]):
                q, k = q.copy(), k.copy()
                backend.rope_embed(q, k, pos, D, HQ, HKV, THETA)
                np.testing.assert_array_equal(q, qr)
                np.testing.assert_array_equal(k, kr)
                k3[:, pos] = k.reshape(HKV, D)
                v3[:, pos] = v.reshape(HKV, D)
                out = np.zeros(HQ * D, f32)
                backend.masked_attention(q, kc, vc, out, HQ, HKV, D, pos)
                assert_close(out, out_ref, f"thread {t} pos {pos}")
        except Exception as e:  # reported by the main thread
            errors.append((t, repr(e)))

    threads = [threading.Thread(target=run, args=(t,)) for t in range(n_threads)]
    for th in threads:
        th.start()
    for th in threads:
        th.join(timeout=100)
    assert not any(th.is_alive() for th in threads), "a thread did not finish"
    assert not errors, errors


def test_native_caches_from_threads(backend):
    """Four threads share one context, each decoding through its own
    backend-owned KV cache (bnr_kv_decode)."""
    import bitnetrs_amd

    case("bnr_kv_decode from 4 threads, one native cache each")
    n_threads, n_steps, cap = 4, 16, 64
    refs = [sequence(710 + t, n_steps, cap) for t in range(n_threads)]
    caches = [bitnetrs_amd.NativeKVCache(backend, 1, HKV, D, cap) for _ in range(n_threads)]
    errors = []

    def run(t):
        try:
            for pos, (q, k, v, qr, kr, out_ref) in enumerate(refs[t]):
                q, k = q.copy(), k.copy()
                out = np.zeros(HQ * D, f32)
                caches[t].decode(0, q, k, v, pos, HQ, THETA, out)
                caches[t].advance()
                np.testing.assert_array_equal(q, qr)
                np.testing.assert_array_equal(k, kr)
                assert_close(out, out_ref, f"thread {t} pos {pos}")
            assert len(caches[t]) == n_steps
        except Exception as e:
            errors.append((t, repr(e)))

    try:
        threads = [threading.Thread(target=run, args=(t,)) for t in range(n_threads)]
        for th in threads:
            th.start()
        for th in threads:
            th.join(timeout=100)
        assert not any(th.is_alive() for th in threads), "a thread did not finish"
        assert not errors, errors
    finally:
        for kc in caches:
            kc.close()
