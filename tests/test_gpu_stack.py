"""The 30-layer attention stack (C5): 1024-token causal prefill then 256 decode
steps, 20/5 heads, d=128, seeded N(0,1) projections per layer and step.  The
whole stack runs on the GPU.  Every layer is checked against the oracle:
its cache (1280 appended rows) bit-exact with the oracle's rope_embed ->
store_kv rows, its 256 decode outputs with the oracle's masked_attention
over them, and its 1024 prefill outputs with the oracle's serial rope ->
store_kv -> masked_attention calls (bitnet-model/src/lib.rs:684-718)."""
import sys

import numpy as np
import pytest

import oracle
from common import D, HKV, HQ, THETA, assert_close_scaled, seed

pytestmark = pytest.mark.gpu

N_LAYERS, N_PRE, N_DEC = 30, 1024, 256


def stack_inputs(layer):
    return (oracle.normal(seed(5, 0) + 64 * layer, (N_PRE, HQ * D)),
            oracle.normal(seed(5, 1) + 64 * layer, (N_PRE, HKV * D)),
            oracle.normal(seed(5, 2) + 64 * layer, (N_PRE, HKV * D)),
            oracle.normal(seed(5, 3) + 64 * layer, (N_DEC, HQ * D)),
            oracle.normal(seed(5, 4) + 64 * layer, (N_DEC, HKV * D)),
            oracle.normal(seed(5, 5) + 64 * layer, (N_DEC, HKV * D)))


def test_stack_c5(backend):
    print("[gpu case] 30-layer stack: 1024 prefill + 256 decode", flush=True)
    import torch

    import bitnetrs_amd

    st = bitnetrs_amd.AttentionStack(backend, N_LAYERS, HQ, HKV, D, N_PRE + N_DEC, THETA)
    ins = [stack_inputs(l) for l in range(N_LAYERS)]
    dev = lambda xs: torch.from_numpy(np.ascontiguousarray(np.stack(xs))).cuda()  # noqa: E731
    qp, kp, vp = dev([i[0] for i in ins]), dev([i[1] for i in ins]), dev([i[2] for i in ins])
    qd, kd, vd = dev([i[3] for i in ins]), dev([i[4] for i in ins]), dev([i[5] for i in ins])
    out_p = torch.zeros(N_LAYERS, N_PRE, HQ * D, device="cuda")
    out_d = torch.zeros(N_LAYERS, N_DEC, HQ * D, device="cuda")
    st.prefill(qp, kp, vp, out_p)
    for s in range(N_DEC):
        st.decode(qd[:, s].contiguous(), kd[:, s].contiguous(), vd[:, s].contiguous(), out_d[:, s])
    torch.cuda.synchronize()
    assert st.position == N_PRE + N_DEC
    got_p, got_d = out_p.cpu().numpy(), out_d.cpu().numpy()
    be = oracle.CpuBackend()
    qz = np.zeros(HQ * D, np.float32)
    for layer in range(N_LAYERS):
        q, k, v, q2, k2, v2 = stack_inputs(layer)
        cache = oracle.KVCache(1, HKV, D, N_PRE + N_DEC)
        for t in range(N_PRE):  # prefill rows: rotation and append only
            kk = k[t].copy()
            be.rope_embed(qz.copy(), kk, t, D, HQ, HKV, THETA)
            cache.store_kv(0, t, kk, v[t])
        ref_d = np.zeros((N_DEC, HQ * D), np.float32)
        for s in range(N_DEC):
            qq, kk, pos = q2[s].copy(), k2[s].copy(), N_PRE + s
            be.rope_embed(qq, kk, pos, D, HQ, HKV, THETA)
            cache.store_kv(0, pos, kk, v2[s])
            be.masked_attention(qq, cache.k(0), cache.v(0), ref_d[s], HQ, HKV, D, pos)
        np.testing.assert_array_equal(st.cache.k[layer].cpu().numpy().reshape(-1), cache.k(0),
                                      err_msg=f"layer {layer} k cache")
        np.testing.assert_array_equal(st.cache.v[layer].cpu().numpy().reshape(-1), cache.v(0),
                                      err_msg=f"layer {layer} v cache")
        res = assert_close_scaled(got_d[layer], ref_d, f"layer {layer} decode")
        c2 = oracle.KVCache(1, HKV, D, N_PRE)
        ref_p = oracle.layer_tokens(oracle.CpuBackend(), c2, 0, q.copy(), k.copy(), v, 0, HQ, HKV,
                                    D, THETA)
        assert_close_scaled(got_p[layer], ref_p, f"layer {layer} prefill")
        print(f"[gpu case] layer {layer}: cache bit-exact, decode {res}", flush=True)
