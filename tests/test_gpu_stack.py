"""The 30-layer attention stack (C5): 1024-token causal prefill then 256 decode
steps, 20/5 heads, d=128, seeded N(0,1) projections per layer and step.  The
whole stack runs on the GPU; layers 0, 14 and 29 are replayed on the oracle
(1024 serial rope -> store_kv -> masked_attention calls, then 256 decode
calls) and compared element by element."""
import sys

import numpy as np
import pytest

import oracle
from common import D, HKV, HQ, THETA, assert_close, seed

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
    for layer in [0, 14, 29]:
        print(f"[gpu case] oracle replay of layer {layer}", flush=True)
        q, k, v, q2, k2, v2 = stack_inputs(layer)
        be = oracle.CpuBackend()
        cache = oracle.KVCache(1, HKV, D, N_PRE + N_DEC)
        ref_p = oracle.layer_tokens(be, cache, 0, q, k, v, 0, HQ, HKV, D, THETA)
        ref_d = oracle.layer_tokens(be, cache, 0, q2, k2, v2, N_PRE, HQ, HKV, D, THETA)
        assert_close(got_p[layer], ref_p, f"layer {layer} prefill")
        print(assert_close(got_d[layer], ref_d, f"layer {layer} decode"))
        np.testing.assert_array_equal(st.cache.k[layer].cpu().numpy().reshape(-1), cache.k(0))
        np.testing.assert_array_equal(st.cache.v[layer].cpu().numpy().reshape(-1), cache.v(0))
