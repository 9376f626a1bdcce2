"""Host-slice calls return when their kernels' completion words arrive, not
after a stream synchronisation.  If a word could arrive before the outputs it
covers, a call would return the previous call's outputs.  These tests make
back-to-back host-slice calls whose consecutive outputs differ -- rope_embed,
masked_attention (incremental mirror), rms_norm and sqrelu_gate, interleaved --
and check every one of them against the oracle as it returns."""
import sys

import numpy as np
import pytest

import oracle
from common import D, HKV, HQ, THETA, assert_close, seed

pytestmark = pytest.mark.gpu
f32 = np.float32


def case(msg):
    print(f"[gpu case] {msg}", flush=True)
    sys.stdout.flush()


def test_interleaved_host_calls_each_fresh(backend):
    case("host-slice calls back to back: 120 tokens of rope/attention with norm and gate between")
    backend.mirror_invalidate()
    ref = oracle.CpuBackend()
    cap, p0, n = 1024, 700, 120
    kc = oracle.normal(seed(60, 0), (HKV, cap, D))
    vc = oracle.normal(seed(60, 1), (HKV, cap, D))
    kcf, vcf = kc.reshape(-1), vc.reshape(-1)
    out = np.zeros(HQ * D, f32)
    # sync the mirror at p0 - 1 (rows 0..p0-1 uploaded once)
    backend.masked_attention(oracle.normal(seed(60, 2), (HQ * D,)), kcf, vcf, out, HQ, HKV, D,
                             p0 - 1)
    gamma = oracle.normal(seed(60, 3), (2560,))
    for t in range(n):
        pos = p0 + t
        q = oracle.normal(seed(61, 0) + t, (HQ * D,), scale=2.0)
        k = oracle.normal(seed(61, 1) + t, (HKV * D,))
        v = oracle.normal(seed(61, 2) + t, (HKV * D,))
        q_ref, k_ref = q.copy(), k.copy()
        ref.rope_embed(q_ref, k_ref, pos, D, HQ, HKV, THETA)
        backend.rope_embed(q, k, pos, D, HQ, HKV, THETA)
        np.testing.assert_array_equal(q, q_ref, err_msg=f"rope_embed q at {pos}")
        np.testing.assert_array_equal(k, k_ref, err_msg=f"rope_embed k at {pos}")
        kc[:, pos] = k.reshape(HKV, D)
        vc[:, pos] = v.reshape(HKV, D)
        out_ref = np.zeros(HQ * D, f32)
        oracle.masked_attention(q, kcf, vcf, out_ref, HQ, HKV, D, pos)
        out.fill(np.nan)
        backend.masked_attention(q, kcf, vcf, out, HQ, HKV, D, pos)
        assert_close(out, out_ref, f"masked_attention at {pos}")
        if t % 3 == 0:
            x = oracle.normal(seed(62, 0) + t, (2560,))
            y, y_ref = np.full(2560, np.nan, f32), np.zeros(2560, f32)
            oracle.rms_norm(x, gamma, 1e-5, y_ref)
            backend.rms_norm(x, gamma, 1e-5, y)
            # the norm's sum of squares is a tree, not the reference's lane order
            assert np.all(np.abs(y - y_ref) <= 2e-3 + 1e-3 * np.abs(y_ref)), f"rms_norm {t}"
            gate = oracle.normal(seed(62, 1) + t, (6912,))
            up = oracle.normal(seed(62, 2) + t, (6912,))
            o, o_ref = np.full(6912, np.nan, f32), np.zeros(6912, f32)
            oracle.sqrelu_gate(gate, up, o_ref)
            backend.sqrelu_gate(gate, up, o)
            np.testing.assert_array_equal(o, o_ref, err_msg=f"sqrelu_gate {t}")
