"""GPU parity of the paths taken when the fast vector paths cannot be: the
norm-fused ternary GEMV with K not a multiple of 16 or with unaligned
activation vectors, and RoPE + KV append with a half head size not a
multiple of 4 or unaligned rows -- next to the aligned vector paths on the
same data.  References are the oracle's compositions of the reference's
functions (bitnet-cpu/src/norm.rs:76, bitnet-core/src/quant/absmax.rs:127,
bitnet-cpu/src/gemv.rs:251, bitnet-cpu/src/rope.rs:414-430,
bitnet-model/src/lib.rs:184-236)."""
import sys

import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu
f32 = np.float32
THETA = 500000.0


def case(msg):
    print(f"[gpu case] {msg}", flush=True)
    sys.stdout.flush()


def dev(a, offset=False):
    """Device copy of a; offset: placed 4 bytes past a 16-byte boundary."""
    import torch

    a = np.ascontiguousarray(a)
    if not offset:
        return torch.from_numpy(a).cuda()
    buf = torch.zeros(a.size + 1, dtype=torch.from_numpy(a[:0]).dtype, device="cuda")
    view = buf[1:]
    view.copy_(torch.from_numpy(a.reshape(-1)))
    return view


def host(t):
    import torch

    torch.cuda.synchronize()
    return t.cpu().numpy()


@pytest.mark.parametrize("mode", [0, 1, 2])
@pytest.mark.parametrize("k,offset", [(2560, False), (2560, True), (100, False), (1000, False),
                                      (4096, False), (4112, False), (6912, True)])
def test_norm_fused_gemv_paths(backend, mode, k, offset):
    _norm_fused_gemv_case(backend, mode, k, offset, [40, 23])


@pytest.mark.parametrize("mode", [1, 2])
@pytest.mark.parametrize("k", [2560, 6912])
@pytest.mark.parametrize("rows", [[5000, 3300], [9000, 7400]])
def test_norm_fused_gemv_rows_per_workgroup(backend, mode, k, rows):
    """As test_norm_fused_gemv_paths with matrices large enough that the
    launch takes 32 rows per workgroup (5000 + 3300 rows) or 64 (9000 + 7400
    rows), both ending mid-workgroup."""
    _norm_fused_gemv_case(backend, mode, k, False, rows)


def _norm_fused_gemv_case(backend, mode, k, offset, rows):
    """bnr_dev_ternary_gemv_norm_group against the oracle's norm -> quantise
    -> ternary GEMV, for two matrices with row counts that end mid-workgroup
    (K up to 4096 takes one 16-activation group per thread, longer K two).
    The sum of squares is a tree on the GPU, so an int8 activation may sit
    one step away where y*127/max falls on a half: each such flip moves an
    output by at most one step of its combined scale."""
    case(f"norm-fused gemv mode {mode} k {k} offset {offset} rows {rows}")
    import torch

    import bitnetrs_amd

    rng = np.random.default_rng(7000 + 10 * mode + k + offset)
    a = rng.standard_normal(k).astype(f32)
    b = rng.standard_normal(k).astype(f32)
    g = rng.uniform(0.5, 1.5, k).astype(f32)
    if mode == bitnetrs_amd._lib.BNR_GLUE_RESIDUAL:
        x = a.copy()
        oracle.axpy(1.0, b, x)
    elif mode == bitnetrs_amd._lib.BNR_GLUE_SQRELU:
        x = np.zeros(k, f32)
        oracle.sqrelu_gate(a, b, x)
    else:
        x = a
    y = np.zeros(k, f32)
    oracle.rms_norm(x, g, 1e-5, y)
    q, s = oracle.absmax_quantize_row(y)
    act_absmax = float(f32(s) * f32(127.0))
    scales = [0.05, 0.03]
    mats = [oracle.pack_rows(rng.integers(-1, 2, size=(m, k)).astype(np.int8)) for m in rows]
    refs = []
    for mat, m, sc in zip(mats, rows, scales):
        out = np.zeros(m, f32)
        oracle.ternary_gemv_preq(mat, sc, q, act_absmax, out, m, k)
        refs.append(out)

    weights = [dev(mt.reshape(-1)) for mt in mats]
    outs = [torch.full((m,), float("nan"), device="cuda") for m in rows]
    h_out = torch.full((k,), float("nan"), device="cuda")
    backend.dev_ternary_gemv_norm_group(
        weights, scales, mode, dev(a, offset), dev(b, offset), dev(g, offset), 1e-5,
        h_out if mode == bitnetrs_amd._lib.BNR_GLUE_RESIDUAL else None, outs, rows, k)
    if mode == bitnetrs_amd._lib.BNR_GLUE_RESIDUAL:
        np.testing.assert_array_equal(host(h_out), x)
    flips = max(2, k // 200)
    for got, ref, sc in zip(outs, refs, scales):
        got = host(got)
        assert np.all(np.isfinite(got))
        step = sc * act_absmax / 127.0
        assert np.max(np.abs(got.astype(np.float64) - ref)) <= flips * step * 1.0001 + 1e-6, \
            (np.max(np.abs(got - ref)), step)


@pytest.mark.parametrize("head_dim,offset", [(12, False), (128, True), (128, False), (64, False)])
def test_rope_append_paths(backend, head_dim, offset):
    _rope_append_case(backend, head_dim, offset, 4, 2)


@pytest.mark.parametrize("nh,nkv", [(16, 16), (32, 16), (40, 20)])
def test_rope_append_many_kv_heads(backend, nh, nkv):
    """As test_rope_append_paths at head_dim 128 with more than 8 kv heads: the
    v rows of a token then take more than one float4 per thread, and with
    more than 32 rotated heads the head loop a second pass."""
    _rope_append_case(backend, 128, False, nh, nkv)


def _rope_append_case(backend, head_dim, offset, nh, nkv):
    """bnr_dev_rope_append for 5 tokens at positions 7..11: q and k rotated in
    place and the cache rows written, bit for bit against the oracle's
    rope_embed and KVCache::store_kv."""
    case(f"rope_append head_dim {head_dim} offset {offset} heads {nh}/{nkv}")
    import torch

    n, start, cap = 5, 7, 16
    rng = np.random.default_rng(900 + head_dim + offset + 1000 * nkv)
    q = rng.standard_normal((n, nh * head_dim)).astype(f32)
    k = rng.standard_normal((n, nkv * head_dim)).astype(f32)
    v = rng.standard_normal((n, nkv * head_dim)).astype(f32)
    ref = oracle.CpuBackend()
    q_ref, k_ref = q.copy(), k.copy()
    for t in range(n):
        ref.rope_embed(q_ref[t], k_ref[t], start + t, head_dim, nh, nkv, THETA)
    dq, dk, dv = dev(q, offset), dev(k, offset), dev(v, offset)
    kc = torch.zeros(nkv, cap, head_dim, device="cuda")
    vc = torch.zeros_like(kc)
    backend.dev_rope_append(dq, dk, dv, n, start, nh, nkv, head_dim, THETA, kc, vc, cap)
    np.testing.assert_array_equal(host(dq).reshape(n, -1), q_ref)
    np.testing.assert_array_equal(host(dk).reshape(n, -1), k_ref)
    kc_h, vc_h = host(kc), host(vc)
    for t in range(n):
        for h in range(nkv):
            np.testing.assert_array_equal(kc_h[h, start + t], k_ref[t, h * head_dim:(h + 1) * head_dim])
            np.testing.assert_array_equal(vc_h[h, start + t], v[t, h * head_dim:(h + 1) * head_dim])
    assert not np.any(kc_h[:, :start]) and not np.any(kc_h[:, start + n:])
