"""GPU parity of the layer glue against the oracle: sqrelu gate, residual add
and absmax quantisation bit-exact; RMSNorm within the fp32 rounding of the
reference (its sum of squares is a tree here, 8 AVX2 lanes there); the fused
norm/quantise launch equal to RMSNorm followed by quantisation on the GPU."""
import sys

import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu
f32 = np.float32


def case(msg):
    print(f"[gpu case] {msg}", flush=True)
    sys.stdout.flush()


def dev(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    import torch

    torch.cuda.synchronize()
    return t.cpu().numpy()


def rms_bound(x, w, got, eps=1e-5):
    xd = x.astype(np.float64)
    exact = xd / np.sqrt(np.mean(xd * xd) + eps) * w
    return np.all(np.abs(got.astype(np.float64) - exact) <= (x.size * 2e-7 + 1e-6) * np.abs(exact) + 1e-12)


@pytest.mark.parametrize("n", [1, 7, 2560, 6912, 10001])
def test_rms_norm_host_and_device(backend, n):
    case(f"rms_norm n {n}")
    import torch

    rng = np.random.default_rng(n)
    x = (rng.standard_normal(n) * 2).astype(f32)
    w = rng.uniform(0.5, 1.5, n).astype(f32)
    ref = np.zeros(n, f32)
    oracle.rms_norm(x, w, 1e-5, ref)
    out = np.full(n, np.nan, f32)
    backend.rms_norm(x, w, 1e-5, out)
    assert rms_bound(x, w, out)
    assert np.all(np.abs(out - ref) <= 2e-3 + 1e-3 * np.abs(ref))
    d = torch.full((n,), float("nan"), device="cuda")
    backend.dev_rms_norm(dev(x), dev(w), 1e-5, d, n)
    np.testing.assert_array_equal(host(d), out)  # same kernel, same order


def test_rms_norm_errors_match_oracle(backend):
    case("rms_norm errors")
    import bitnetrs_amd

    z4 = np.zeros(4, f32)
    for args in [(z4, np.zeros(3, f32), 1e-5, z4), (z4, z4, 1e-5, np.zeros(5, f32)),
                 (z4, z4, 0.0, z4), (z4, z4, float("nan"), z4), (z4, z4, -2.5, z4)]:
        with pytest.raises(oracle.OracleError) as oe:
            oracle.rms_norm(*args)
        with pytest.raises(bitnetrs_amd.BitNetError) as ge:
            backend.rms_norm(*args)
        assert ge.value.kind == oe.value.kind and str(ge.value) == str(oe.value)
    backend.rms_norm(np.zeros(0, f32), np.zeros(0, f32), 1e-5, np.zeros(0, f32))


@pytest.mark.parametrize("n", [1, 6912, 10001])
def test_sqrelu_bit_exact(backend, n):
    case(f"sqrelu n {n}")
    import torch

    rng = np.random.default_rng(7 + n)
    g = (rng.standard_normal(n) * 3).astype(f32)
    g[::17] = -0.0
    g[::29] = np.nan
    u = (rng.standard_normal(n) * 3).astype(f32)
    ref = np.zeros(n, f32)
    oracle.sqrelu_gate(g, u, ref)
    out = np.full(n, np.nan, f32)
    backend.sqrelu_gate(g, u, out)
    np.testing.assert_array_equal(out, ref)
    d = torch.full((n,), float("nan"), device="cuda")
    backend.dev_sqrelu_gate(dev(g), dev(u), d, n)
    np.testing.assert_array_equal(host(d), ref)


def test_residual_bit_exact(backend):
    case("residual add")
    rng = np.random.default_rng(3)
    h = rng.standard_normal(2560).astype(f32)
    o = rng.standard_normal(2560).astype(f32)
    ref = h.copy()
    oracle.axpy(1.0, o, ref)  # axpy_f32_fast(1.0, o, h): fma(1, o, h) = o + h
    dh = dev(h)
    backend.dev_residual_add(dh, dev(o), 2560)
    np.testing.assert_array_equal(host(dh), ref)


@pytest.mark.parametrize("n", [1, 100, 2560, 6912, 10001])
def test_absmax_quantize_bit_exact(backend, n):
    case(f"absmax quantize n {n}")
    import torch

    rng = np.random.default_rng(50 + n)
    x = (rng.standard_normal(n) * rng.uniform(0.01, 20)).astype(f32)
    x[rng.integers(0, n, max(1, n // 30))] = 0.0
    q_ref, s_ref = oracle.absmax_quantize_row(x)
    q = torch.zeros(n, dtype=torch.int8, device="cuda")
    s = torch.zeros(1, device="cuda")
    backend.dev_absmax_quantize(dev(x), q, s, n)
    np.testing.assert_array_equal(host(q), q_ref)
    assert float(host(s)[0]) == s_ref


@pytest.mark.parametrize("mode,n,alias", [(0, 2560, False), (1, 2560, False), (2, 6912, False),
                                          (0, 10001, False), (1, 9000, False), (1, 9000, True),
                                          (1, 2561, True), (2, 37, False)])
def test_norm_quant_fused(backend, mode, n, alias):
    """The fused launch equals rms_norm followed by absmax_quantize on the GPU
    (bit for bit), and the oracle's composition to rounding.  alias: the
    residual stream is updated in place (h_out is a)."""
    case(f"norm_quant mode {mode} n {n} alias {alias}")
    import torch

    import bitnetrs_amd

    rng = np.random.default_rng(1000 * mode + n)
    a = rng.standard_normal(n).astype(f32)
    b = rng.standard_normal(n).astype(f32)
    g = rng.uniform(0.5, 1.5, n).astype(f32)
    if mode == bitnetrs_amd._lib.BNR_GLUE_RESIDUAL:
        x = a.copy()
        oracle.axpy(1.0, b, x)
    elif mode == bitnetrs_amd._lib.BNR_GLUE_SQRELU:
        x = np.zeros(n, f32)
        oracle.sqrelu_gate(a, b, x)
    else:
        x = a
    y_ref = np.zeros(n, f32)
    oracle.rms_norm(x, g, 1e-5, y_ref)
    q_ref, s_ref = oracle.absmax_quantize_row(y_ref)

    da, db, dg = dev(a), dev(b), dev(g)
    h_out = da if alias else torch.full((n,), float("nan"), device="cuda")
    q = torch.zeros(n, dtype=torch.int8, device="cuda")
    aa = torch.zeros(1, device="cuda")
    backend.dev_norm_quant(mode, da, db, dg, 1e-5, n, h_out, q, aa)
    if mode == bitnetrs_amd._lib.BNR_GLUE_RESIDUAL:
        np.testing.assert_array_equal(host(h_out), x)
    # GPU composition: x on the GPU -> rms_norm -> absmax quantise
    y = torch.zeros(n, device="cuda")
    backend.dev_rms_norm(dev(x), dg, 1e-5, y, n)
    q2 = torch.zeros(n, dtype=torch.int8, device="cuda")
    s2 = torch.zeros(1, device="cuda")
    backend.dev_absmax_quantize(y, q2, s2, n)
    np.testing.assert_array_equal(host(q), host(q2))
    assert float(host(aa)[0]) == float(f32(host(s2)[0]) * f32(127.0))
    # oracle: y to rounding, so q may differ by one where y*127/max sits on a half
    diff = host(q).astype(int) - q_ref.astype(int)
    assert np.all(np.abs(diff) <= 1) and np.count_nonzero(diff) <= max(2, n // 200)
    assert abs(float(host(aa)[0]) - s_ref * 127.0) <= 1e-5 * s_ref * 127.0
