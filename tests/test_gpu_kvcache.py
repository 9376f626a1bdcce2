"""GPU parity of the library's backend-owned KV cache (``bnr_kv_cache``)
against the oracle's KVCache (bitnet-model/src/lib.rs:118-315) driven by the
reference's per-layer token sequence rope_embed -> store_kv ->
masked_attention (lib.rs:1004-1036): outputs within tolerance, rotated q/k
and cache rows bit for bit, the bookkeeping (layer lengths,
filled_positions) and store_kv / advance errors with the reference's kinds
and messages."""
import ctypes
import sys

import numpy as np
import pytest

import oracle
from common import (D, HKV, HQ, THETA, assert_close, error_from_parts, oracle_prefill, prefill_workload,
                    seed)

pytestmark = pytest.mark.gpu
f32 = np.float32


def case(msg):
    print(f"[gpu case] {msg}", flush=True)
    sys.stdout.flush()


def read_device(ptr: int, n: int) -> np.ndarray:
    """n floats at device address ptr, through the HIP runtime the library uses."""
    import torch

    import bitnetrs_amd

    torch.cuda.synchronize()
    L = bitnetrs_amd.load()
    out = np.empty(n, f32)
    rc = L.hipMemcpy(ctypes.c_void_p(out.ctypes.data), ctypes.c_void_p(ptr), ctypes.c_size_t(4 * n),
                     ctypes.c_int(2))  # hipMemcpyDeviceToHost
    assert rc == 0, rc
    return out


def dev(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda")


def host(t):
    import torch

    torch.cuda.synchronize()
    return t.cpu().numpy()


def token(cfg, layer, pos, n_heads=HQ, n_kv=HKV, hd=D):
    s = 1000 * cfg + 10 * layer
    return (oracle.normal(seed(s, pos), (n_heads * hd,)),
            oracle.normal(seed(s + 1, pos), (n_kv * hd,)),
            oracle.normal(seed(s + 2, pos), (n_kv * hd,)))


def ref_token(be, cache, layer, q, k, v, pos, n_heads, n_kv, hd):
    """The reference's three calls for one token of one layer."""
    be.rope_embed(q, k, pos, hd, n_heads, n_kv, THETA)
    cache.store_kv(layer, pos, k, v)
    out = np.zeros(n_heads * hd, f32)
    be.masked_attention(q, cache.k(layer), cache.v(layer), out, n_heads, n_kv, hd, pos)
    return out


@pytest.mark.parametrize("n_heads,n_kv,hd", [(HQ, HKV, D), (8, 2, 64)])
def test_native_cache_host_decode_matches_oracle(backend, n_heads, n_kv, hd):
    """Six tokens through two layers with bnr_kv_decode (host slices), the
    cache advanced after each token as the engine does."""
    import bitnetrs_amd

    n_layers, max_seq = 2, 64
    kc = bitnetrs_amd.NativeKVCache(backend, n_layers, n_kv, hd, max_seq)
    ref = oracle.KVCache(n_layers, n_kv, hd, max_seq)
    be = oracle.CpuBackend()
    try:
        for pos in range(6):
            for layer in range(n_layers):
                case(f"native cache host decode heads {n_heads}/{n_kv} d {hd} pos {pos} layer {layer}")
                q, k, v = token(50, layer, pos, n_heads, n_kv, hd)
                qr, kr = q.copy(), k.copy()
                out_ref = ref_token(be, ref, layer, qr, kr, v, pos, n_heads, n_kv, hd)
                out = np.zeros(n_heads * hd, f32)
                kc.decode(layer, q, k, v, pos, n_heads, THETA, out)
                np.testing.assert_array_equal(q, qr)
                np.testing.assert_array_equal(k, kr)
                assert_close(out, out_ref, f"pos {pos} layer {layer}")
                assert kc.layer_len(layer) == ref.layer_len(layer) == pos + 1
            kc.advance()
            ref.advance()
            assert len(kc) == len(ref) == pos + 1
        n = n_kv * max_seq * hd
        for layer in range(n_layers):
            kp, vp = kc.layer_ptrs(layer)
            np.testing.assert_array_equal(read_device(kp, n), ref.k(layer))
            np.testing.assert_array_equal(read_device(vp, n), ref.v(layer))
    finally:
        kc.close()


def test_native_cache_errors_match_oracle(backend):
    """store_kv's position rules, wrong lengths, a bad theta and the
    advance overflow: same error kind and message as the oracle; a failed
    call stores nothing.  Overwriting a stored row is allowed and does not
    extend the layer.  clear() zeroes rows and bookkeeping."""
    import bitnetrs_amd

    n_layers, max_seq = 2, 8
    kc = bitnetrs_amd.NativeKVCache(backend, n_layers, HKV, D, max_seq)
    ref = oracle.KVCache(n_layers, HKV, D, max_seq)
    be = oracle.CpuBackend()

    def both(pos, layer=0, v_len=HKV * D, theta=THETA):
        case(f"native cache error case pos {pos} layer {layer} v_len {v_len} theta {theta}")
        q, k, v = token(51, layer, pos)
        v = v[:v_len].copy()
        got = want = None
        try:
            kc.decode(layer, q.copy(), k.copy(), v, pos, HQ, theta, np.zeros(HQ * D, f32))
        except bitnetrs_amd.BitNetError as e:
            got = (type(e).__name__, str(e))
            assert error_from_parts() == (e.kind, str(e))
        try:
            qr, kr = q.copy(), k.copy()
            be.rope_embed(qr, kr, pos, D, HQ, HKV, theta)
            ref.store_kv(layer, pos, kr, v)
        except Exception as e:  # oracle error classes carry the reference's kind names
            want = (type(e).__name__, str(e))
        return got, want

    try:
        got, want = both(3)  # a gap: layer 0 holds no position yet
        assert got == ("InvalidShape", "invalid tensor shape: expected position <= "
                       "layer_len_positions (0), got position = 3"), got
        assert got[1] == want[1]
        assert kc.layer_len(0) == 0
        for p in range(3):
            assert both(p) == (None, None)
        got, want = both(8)  # position >= max_seq
        assert got[0] == "InvalidShape" and got[1] == want[1], (got, want)
        got, want = both(3, v_len=HKV * D - 1)  # store_kv's v length check
        assert got[0] == "InvalidShape" and got[1] == want[1], (got, want)
        got, _ = both(3, theta=-1.0)  # RopeCache::new rejects the table first
        assert got[0] == "InvalidConfig", got
        with pytest.raises(bitnetrs_amd.InvalidShape):
            kc.decode(n_layers, *token(51, 0, 0)[:2], token(51, 0, 0)[2], 0, HQ, THETA,
                      np.zeros(HQ * D, f32))
        assert both(1) == (None, None)  # overwrite a stored row
        assert kc.layer_len(0) == ref.layer_len(0) == 3
        for _ in range(max_seq):
            kc.advance()
            ref.advance()
        with pytest.raises(bitnetrs_amd.BackendError) as e:
            kc.advance()
        assert error_from_parts() == (e.value.kind, str(e.value))
        assert e.value.fields[0] == "HIP"
        with pytest.raises(Exception) as e_ref:
            ref.advance()
        assert str(e.value) == f"backend error (HIP): {e_ref.value}" or \
            str(e.value).endswith(str(e_ref.value)), (str(e.value), str(e_ref.value))
        assert len(kc) == max_seq
        kc.clear()
        assert len(kc) == 0 and kc.layer_len(0) == 0 and kc.layer_len(1) == 0
        kp, vp = kc.layer_ptrs(0)
        assert not np.any(read_device(kp, HKV * max_seq * D))
        assert not np.any(read_device(vp, HKV * max_seq * D))
    finally:
        kc.close()


def test_native_cache_device_prefill_then_decode(backend):
    """bnr_kv_dev_prefill of 300 tokens into layer 1 of a 2B-shaped cache
    (max_seq 4096), then bnr_kv_dev_decode of the next two positions: outputs
    against the reference's token loop, cache rows bit for bit."""
    import torch

    import bitnetrs_amd

    n_layers, max_seq, n = 2, 4096, 300
    kc = bitnetrs_amd.NativeKVCache(backend, n_layers, HKV, D, max_seq)
    try:
        case("native cache device prefill 300 tokens, layer 1")
        w = prefill_workload(52, n)
        ref = oracle.KVCache(n_layers, HKV, D, max_seq)
        be = oracle.CpuBackend()
        q_ref, k_ref, ref, out_ref = oracle_prefill(w, cache=ref, layer=1, backend=be)
        q, k = dev(w["q"]), dev(w["k"])
        out = torch.zeros(n, HQ * D, device="cuda")
        kc.dev_prefill(1, q, k, dev(w["v"]), n, 0, HQ, THETA, out)
        np.testing.assert_array_equal(host(q), q_ref)
        np.testing.assert_array_equal(host(k), k_ref)
        assert_close(host(out), out_ref, "prefill through the native cache")
        assert kc.layer_len(1) == n and kc.layer_len(0) == 0
        for pos in (n, n + 1):
            case(f"native cache device decode pos {pos}, layer 1")
            qh, kh, vh = token(53, 1, pos)
            out_d = torch.zeros(HQ * D, device="cuda")
            kc.dev_decode(1, dev(qh), dev(kh), dev(vh), pos, HQ, THETA, out_d)
            out_r = ref_token(be, ref, 1, qh.copy(), kh.copy(), vh, pos, HQ, HKV, D)
            assert_close(host(out_d), out_r, f"decode pos {pos}")
        assert kc.layer_len(1) == n + 2
        kp, vp = kc.layer_ptrs(1)
        cnt = HKV * max_seq * D
        np.testing.assert_array_equal(read_device(kp, cnt), ref.k(1))
        np.testing.assert_array_equal(read_device(vp, cnt), ref.v(1))
        with pytest.raises(bitnetrs_amd.InvalidShape):  # a gap in layer 0
            kc.dev_prefill(0, q, k, dev(w["v"]), n, 5, HQ, THETA, out)
    finally:
        kc.close()
