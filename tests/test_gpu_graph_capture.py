"""Stream-ordered device entry points under HIP graph capture: after one
uncaptured call on a cache of `cap` rows (any size), later calls on that
cache allocate nothing and synchronise nothing, so they can be captured --
here a prefill of the whole capacity after a 64-token warm-up, and decode
steps at positions far past the warm-up's.  Every replay is checked against
the same calls made eagerly, with eager work and synchronisations between
replays.  The eager results themselves are checked against the oracle in
test_gpu_parity.py."""
import sys

import numpy as np
import pytest

from common import D, HKV, HQ, THETA, decode_workload, prefill_workload

pytestmark = pytest.mark.gpu


def case(msg):
    print(f"[gpu case] {msg}", flush=True)
    sys.stdout.flush()


def dev(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda")


@pytest.mark.parametrize("cap,n,start", [(1024, 1024, 0), (2048, 2048, 0), (4096, 1568, 320)])
def test_prefill_at_capacity_captured(backend, cap, n, start):
    import torch

    case(f"captured prefill N={n} at {start} on cap {cap} after a 64-token warm-up")
    w = prefill_workload(70, n)
    q0, k0, v = dev(w["q"]), dev(w["k"]), dev(w["v"])
    kc = torch.zeros(HKV, cap, D, device="cuda")
    vc = torch.zeros_like(kc)
    # warm-up: 64 tokens on this cache (sizes the table and workspaces by cap)
    qw, kw = q0[:64].clone(), k0[:64].clone()
    ow = torch.zeros(64, HQ * D, device="cuda")
    backend.dev_prefill(qw, kw, v[:64], 64, 0, HQ, HKV, D, THETA, kc, vc, cap, ow)
    # captured straight after the warm-up: nothing larger ran on this cache
    q, k = q0.clone(), k0.clone()
    out = torch.zeros(n, HQ * D, device="cuda")
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        q.copy_(q0)
        k.copy_(k0)
        backend.dev_prefill(q, k, v, n, start, HQ, HKV, D, THETA, kc, vc, cap, out)
    # eager reference of the same call
    qe, ke = q0.clone(), k0.clone()
    out_ref = torch.zeros_like(out)
    kc.zero_()
    vc.zero_()
    backend.dev_prefill(qe, ke, v, n, start, HQ, HKV, D, THETA, kc, vc, cap, out_ref)
    torch.cuda.synchronize()
    q_ref, k_ref, kc_ref, vc_ref = qe.clone(), ke.clone(), kc.clone(), vc.clone()
    for r in range(3):
        out.fill_(float("nan"))
        kc.zero_()
        vc.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(q, q_ref) and torch.equal(k, k_ref), f"replay {r}: rotated q/k"
        assert torch.equal(kc, kc_ref) and torch.equal(vc, vc_ref), f"replay {r}: cache rows"
        diff = float((out - out_ref).abs().max())
        assert diff <= 1e-5 * max(1.0, float(out_ref.abs().max())), f"replay {r}: max diff {diff}"
        # eager work of the program between replays
        backend.dev_prefill(qw, kw, v[:64], 64, 0, HQ, HKV, D, THETA, kc, vc, cap, ow)
        torch.cuda.synchronize()
    del g


def prefill_workspace_bytes(cap, n_cu, group=HQ // HKV, n_kv=HKV):
    """Partial states the first prefill on a cache of `cap` rows reserves:
    the planner's budget of four (kv head, item) pairs per query tile, at
    most 8192, or two per resident workgroup of a stream-K launch (two per
    CU below group 8), whichever is more; group * 66 * 64 floats each."""
    tiles = (cap + 31) // 32
    per_cu = 1 if group >= 8 else 2
    items = max(min(4 * n_kv * tiles, 8192), 2 * n_cu * per_cu)
    return items * group * 66 * 64 * 4


@pytest.mark.parametrize("cap", [2048, 8192])
def test_prefill_workspace_reserved_by_cap(cap):
    """The first prefill on a cache reserves the workspace every later
    launch on it can need, and no more: device memory taken by a 64-token
    prefill in a fresh context is the partial-state workspace for `cap`
    plus small tables (RoPE rows, tickets)."""
    import torch

    import bitnetrs_amd

    case(f"prefill workspace reserved for cap {cap}")
    n_cu = torch.cuda.get_device_properties(0).multi_processor_count
    w = prefill_workload(71, 64)
    q, k, v = dev(w["q"]), dev(w["k"]), dev(w["v"])
    kc = torch.zeros(HKV, cap, D, device="cuda")
    vc = torch.zeros_like(kc)
    out = torch.zeros(64, HQ * D, device="cuda")
    be = bitnetrs_amd.HipBackend(0)
    try:
        torch.cuda.synchronize()
        free0 = torch.cuda.mem_get_info()[0]
        be.dev_prefill(q, k, v, 64, 0, HQ, HKV, D, THETA, kc, vc, cap, out)
        torch.cuda.synchronize()
        taken = free0 - torch.cuda.mem_get_info()[0]
    finally:
        be.close()
    want = prefill_workspace_bytes(cap, n_cu)
    assert want <= taken <= want + (16 << 20), f"cap {cap}: took {taken} B, workspace {want} B"


def test_decode_steps_captured_past_warmup(backend):
    import torch

    cap = 8192
    case(f"captured decode steps at positions 8000..8007, warm-up at 10, cap {cap}")
    w = decode_workload(71, 8007, cap=cap)
    kc0, vc0 = dev(w["k_cache"]), dev(w["v_cache"])
    gen = torch.Generator(device="cuda").manual_seed(71)
    n = 8
    qs = torch.randn(n, HQ * D, device="cuda", generator=gen)
    ks = torch.randn(n, HKV * D, device="cuda", generator=gen)
    vs = torch.randn(n, HKV * D, device="cuda", generator=gen)
    kc, vc = kc0.clone(), vc0.clone()
    out = torch.zeros(n, HQ * D, device="cuda")
    # warm-up at position 10 (the table and workspaces are sized by cap)
    backend.dev_decode_step(qs[0], ks[0], vs[0], 10, HQ, HKV, D, THETA, kc, vc, cap, out[0])
    kc.copy_(kc0)
    vc.copy_(vc0)

    def steps():
        for i in range(n):
            backend.dev_decode_step(qs[i], ks[i], vs[i], 8000 + i, HQ, HKV, D, THETA, kc, vc, cap,
                                    out[i])

    # captured straight after the warm-up, then the same steps eagerly
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        steps()
    steps()
    torch.cuda.synchronize()
    out_ref, kc_ref, vc_ref = out.clone(), kc.clone(), vc.clone()
    for r in range(3):
        kc.copy_(kc0)
        vc.copy_(vc0)
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(kc, kc_ref) and torch.equal(vc, vc_ref), f"replay {r}: cache rows"
        # the reference merge's atomics may reorder the last bits between runs
        diff = float((out - out_ref).abs().max())
        assert diff <= 1e-5 * max(1.0, float(out_ref.abs().max())), f"replay {r}: max diff {diff}"
        backend.dev_decode_step(qs[0], ks[0], vs[0], 10, HQ, HKV, D, THETA, kc, vc, cap, out[0])
        torch.cuda.synchronize()
    del g
