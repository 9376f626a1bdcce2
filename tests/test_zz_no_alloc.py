"""GPU parity of bnr_dev_decode_attention_noalloc, the decode entry point
that allocates nothing (its merge state lives in the library's per-GPU
device array), against the existing bnr_dev_decode_attention and against
the oracle's masked_attention (bitnet-cpu/src/attention.rs:97-209), on
consecutive calls with a smaller context second (the array keeps the last
call's state), with device free memory unchanged across the calls."""
import sys

import numpy as np
import pytest

import oracle
from common import D, HKV, HQ, assert_close_scaled, decode_workload

pytestmark = pytest.mark.gpu
f32 = np.float32


def case(msg):
    print(f"[gpu case] {msg}", flush=True)
    sys.stdout.flush()


def dev(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda")


def oracle_attention(w, n_heads, n_kv):
    out = np.zeros(n_heads * D, f32)
    oracle.masked_attention(w["q"], w["k_cache"].reshape(-1), w["v_cache"].reshape(-1), out,
                            n_heads, n_kv, D, w["pos"])
    return out


@pytest.mark.parametrize("n_heads,n_kv", [(HQ, HKV), (8, 2), (32, 32)])
def test_noalloc_matches_decode_attention(n_heads, n_kv):
    import torch

    import bitnetrs_amd

    be = bitnetrs_amd.HipBackend(0)
    try:
        # the larger context first, then a smaller one on the same array
        works = [decode_workload(90, 4095, cap=4096, q_scale=4.0, n_heads=n_heads, n_kv=n_kv),
                 decode_workload(91, 700, cap=4096, n_heads=n_heads, n_kv=n_kv)]
        bufs = []
        for w in works:
            # cached rows 0..pos, q taken as already rotated
            w["k_cache"][:, w["pos"]] = w["k"].reshape(n_kv, D)
            w["v_cache"][:, w["pos"]] = w["v"].reshape(n_kv, D)
            bufs.append((dev(w["q"]), dev(w["k_cache"]), dev(w["v_cache"]),
                         torch.zeros(n_heads * D, device="cuda"),
                         torch.zeros(n_heads * D, device="cuda")))
        # The existing entry point first: it launches the same kernels (the
        # runtime loads them on first use) and gives the reference outputs.
        for w, (q, kc, vc, _, out_ref) in zip(works, bufs):
            be.dev_decode_attention(q, kc, vc, 4096, out_ref, n_heads, n_kv, D, w["pos"])
        torch.cuda.synchronize()
        free0 = torch.cuda.mem_get_info()[0]
        for i, (w, (q, kc, vc, out_na, _)) in enumerate(zip(works, bufs)):
            case(f"no-alloc decode call {i}: heads {n_heads}/{n_kv} pos {w['pos']}")
            be.dev_decode_attention_noalloc(q, kc, vc, 4096, out_na, n_heads, n_kv, D, w["pos"])
        torch.cuda.synchronize()
        assert torch.cuda.mem_get_info()[0] == free0, "device memory changed across the calls"
        for i, (w, (q, kc, vc, out_na, out_ref)) in enumerate(zip(works, bufs)):
            got = out_na.cpu().numpy()
            assert_close_scaled(got, out_ref.cpu().numpy(), f"call {i} vs dev_decode_attention")
            assert_close_scaled(got, oracle_attention(w, n_heads, n_kv), f"call {i} vs oracle")
    finally:
        be.close()


def test_noalloc_limits_are_errors():
    import torch

    import bitnetrs_amd

    be = bitnetrs_amd.HipBackend(0)
    try:
        z = torch.zeros(64 * 4 * 16 * D, device="cuda")
        out = torch.zeros(64 * D, device="cuda")
        case("no-alloc limits")
        with pytest.raises(bitnetrs_amd.InvalidConfig):  # more than 32 query heads
            be.dev_decode_attention_noalloc(z[:64 * D], z, z, 16, out, 64, 16, D, 3)
        with pytest.raises(bitnetrs_amd.InvalidConfig):  # group size 8
            be.dev_decode_attention_noalloc(z[:8 * D], z, z, 16, out[:8 * D], 8, 1, D, 3)
        with pytest.raises(bitnetrs_amd.InvalidShape):  # position past the cache
            be.dev_decode_attention_noalloc(z[:8 * D], z, z, 16, out[:8 * D], 8, 2, D, 16)
    finally:
        be.close()


def test_noalloc_exact_path_then_plain():
    """The exact path through the scratch: planted rows score ~130 log2 units
    above the rest of their split (two heads), and in a third head the newest
    row points away from q, so every split of that head is flagged; the
    partial states and masks live in the scratch's ws_ml / ws_o regions.  A
    plain call follows on the same scratch (masks cleared by the first)."""
    import torch

    import bitnetrs_amd

    be = bitnetrs_amd.HipBackend(0)
    try:
        g = HQ // HKV
        w = decode_workload(92, 4095, cap=4096, q_scale=1.0)
        q = w["q"].reshape(HQ, D)
        for head, rows in [(0, [100, 2500]), (3, [4000])]:
            for t in rows:
                w["k_cache"][head, t] = (8.0 * q[head * g]).astype(f32)
        w["k_cache"][:, w["pos"]] = w["k"].reshape(HKV, D)
        w["v_cache"][:, w["pos"]] = w["v"].reshape(HKV, D)
        w["k_cache"][1, w["pos"]] = (-8.0 * q[1 * g]).astype(f32)  # newest row away from q
        plain = decode_workload(93, 1500, cap=4096)
        plain["k_cache"][:, plain["pos"]] = plain["k"].reshape(HKV, D)
        plain["v_cache"][:, plain["pos"]] = plain["v"].reshape(HKV, D)
        for i, ww in enumerate([w, plain]):
            case(f"no-alloc exact path: call {i} pos {ww['pos']}")
            out = torch.zeros(HQ * D, device="cuda")
            be.dev_decode_attention_noalloc(dev(ww["q"]), dev(ww["k_cache"]), dev(ww["v_cache"]), 4096,
                                            out, HQ, HKV, D, ww["pos"])
            torch.cuda.synchronize()
            assert_close_scaled(out.cpu().numpy(), oracle_attention(ww, HQ, HKV), f"call {i} vs oracle")
    finally:
        be.close()


def test_noalloc_scratch_has_one_owner():
    """The per-GPU scratch serves one (context, stream) pair: another context,
    or the owner on another stream, gets BackendError until the owner is
    destroyed; then the other context can claim it."""
    import torch

    import bitnetrs_amd

    w = decode_workload(94, 300, cap=512)
    w["k_cache"][:, w["pos"]] = w["k"].reshape(HKV, D)
    w["v_cache"][:, w["pos"]] = w["v"].reshape(HKV, D)
    q, kc, vc = dev(w["q"]), dev(w["k_cache"]), dev(w["v_cache"])
    out = torch.zeros(HQ * D, device="cuda")
    a, b = bitnetrs_amd.HipBackend(0), bitnetrs_amd.HipBackend(0)
    side = torch.cuda.Stream()
    try:
        case("no-alloc scratch owner")
        a.dev_decode_attention_noalloc(q, kc, vc, 512, out, HQ, HKV, D, w["pos"])
        with pytest.raises(bitnetrs_amd.BackendError):
            b.dev_decode_attention_noalloc(q, kc, vc, 512, out, HQ, HKV, D, w["pos"])
        with pytest.raises(bitnetrs_amd.BackendError):
            a.dev_decode_attention_noalloc(q, kc, vc, 512, out, HQ, HKV, D, w["pos"], stream=side)
        a.dev_decode_attention_noalloc(q, kc, vc, 512, out, HQ, HKV, D, w["pos"])  # still the owner
        torch.cuda.synchronize()
        a.close()
        b.dev_decode_attention_noalloc(q, kc, vc, 512, out, HQ, HKV, D, w["pos"])  # released
        torch.cuda.synchronize()
        assert_close_scaled(out.cpu().numpy(), oracle_attention(w, HQ, HKV), "new owner vs oracle")
    finally:
        a.close()
        b.close()
