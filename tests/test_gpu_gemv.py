"""GPU parity of the W2A8 ternary GEMV (Backend::ternary_gemv_preq) against
the oracle, through the C ABI.  Integer accumulation is exact and the scale
is applied with one f32 multiply, so outputs must be bit-identical."""
import sys

import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu
f32 = np.float32


def case(msg):
    print(f"[gpu case] {msg}", flush=True)
    sys.stdout.flush()


def workload(seed, m, k, garbage=0.0):
    rng = np.random.default_rng(seed)
    w = oracle.pack_rows(rng.integers(-1, 2, size=(m, k)).astype(np.int8)) if m else \
        np.zeros((0, (k + 3) // 4), np.uint8)
    w = np.ascontiguousarray(w.reshape(-1))
    if garbage:
        mask = rng.random(w.size) < garbage  # any byte, including code 0b11 (decodes to 0)
        w[mask] = rng.integers(0, 256, int(mask.sum()))
    act = rng.integers(-128, 128, size=k).astype(np.int8)
    ws, aa = f32(rng.uniform(0.05, 2.0)), f32(rng.uniform(0.5, 40.0))
    return w, act, ws, aa


def ref(w, ws, act, aa, m, k):
    out = np.full(m, np.nan, f32)
    oracle.ternary_gemv_preq(w, ws, act, aa, out, m, k)
    return out


SHAPES = [(2560, 2560), (640, 2560), (6912, 2560), (2560, 6912),  # 2B projections
          (1, 1), (3, 5), (17, 64), (33, 63), (16, 4097), (5, 10000), (100, 130)]


@pytest.mark.parametrize("m,k", SHAPES)
def test_host_gemv_bit_exact(backend, m, k):
    case(f"ternary gemv host m {m} k {k}")
    w, act, ws, aa = workload(1000 + m + 7 * k, m, k, garbage=0.05)
    out = np.full(m, np.nan, f32)
    backend.ternary_gemv_preq(w, ws, act, aa, out, m, k)
    np.testing.assert_array_equal(out, ref(w, ws, act, aa, m, k))


@pytest.mark.parametrize("m,k,offset", [(2560, 2560, 0), (6912, 2560, 0), (2560, 6912, 0),
                                        (700, 2560, 1), (300, 999, 0), (64, 6912, 3)])
def test_device_gemv_bit_exact(backend, m, k, offset):
    """offset > 0 shifts the weight and activation pointers off 16-byte
    alignment, which takes the byte-wise load path."""
    case(f"ternary gemv device m {m} k {k} offset {offset}")
    import torch

    w, act, ws, aa = workload(2000 + m + k + offset, m, k)
    wbuf = torch.zeros(w.size + offset, dtype=torch.uint8, device="cuda")
    abuf = torch.zeros(act.size + offset, dtype=torch.int8, device="cuda")
    wbuf[offset:] = torch.from_numpy(w).cuda()
    abuf[offset:] = torch.from_numpy(act).cuda()
    out = torch.full((m,), float("nan"), device="cuda")
    backend.dev_ternary_gemv_preq(wbuf[offset:], ws, abuf[offset:], aa, out, m, k)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(out.cpu().numpy(), ref(w, ws, act, aa, m, k))


def test_gemv_extremes(backend):
    case("ternary gemv extremes")
    k = 6912
    w = oracle.pack_rows(np.stack([-np.ones(k, np.int8), np.ones(k, np.int8),
                                   np.zeros(k, np.int8)])).reshape(-1)
    act = np.full(k, -128, np.int8)
    out = np.zeros(3, f32)
    backend.ternary_gemv_preq(w, 1.0, act, 127.0, out, 3, k)
    np.testing.assert_array_equal(out, [884736.0, -884736.0, 0.0])


def test_gemv_empty_dims(backend):
    case("ternary gemv empty dims")
    out = np.full(4, np.nan, f32)
    backend.ternary_gemv_preq(np.zeros(0, np.uint8), 1.0, np.zeros(0, np.int8), 1.0, out, 4, 0)
    np.testing.assert_array_equal(out, np.zeros(4, f32))  # empty dot = 0 (gemv.rs row loop)
    backend.ternary_gemv_preq(np.zeros(0, np.uint8), 1.0, np.zeros(5, np.int8), 1.0,
                              np.zeros(0, f32), 0, 5)


def test_gemv_errors_match_oracle(backend):
    case("ternary gemv errors")
    import bitnetrs_amd

    w, act, ws, aa = workload(5, 4, 10)
    out = np.zeros(4, f32)
    bad = [
        (np.zeros(5, np.uint8), ws, act, aa, out, 4, 10),   # weight length
        (w, ws, np.zeros(9, np.int8), aa, out, 4, 10),      # activation length
        (w, ws, act, aa, np.zeros(3, f32), 4, 10),          # output length
        (w, 0.0, act, aa, out, 4, 10),                       # weight scale
        (w, float("inf"), act, aa, out, 4, 10),
        (w, ws, act, -1.0, out, 4, 10),                      # activation scale
        (w, ws, act, float("nan"), out, 4, 10),
        (np.zeros(5, np.uint8), 0.0, act, aa, out, 4, 10),  # shape checked before scale
    ]
    kinds = {oracle.InvalidShape: bitnetrs_amd.InvalidShape,
             oracle.QuantizationError: bitnetrs_amd.QuantizationError}
    for args in bad:
        with pytest.raises(oracle.OracleError) as oe:
            oracle.ternary_gemv_preq(*args)
        with pytest.raises(bitnetrs_amd.BitNetError) as ge:
            backend.ternary_gemv_preq(*args)
        assert type(ge.value) is kinds[type(oe.value)]
        assert str(ge.value) == str(oe.value)


def test_gemv_weight_mirror_and_invalidate(backend):
    case("ternary gemv weight mirror")
    m, k = 48, 200
    w, act, ws, aa = workload(9, m, k)
    out = np.zeros(m, f32)
    backend.ternary_gemv_preq(w, ws, act, aa, out, m, k)
    np.testing.assert_array_equal(out, ref(w, ws, act, aa, m, k))
    # new activations, same (mirrored) weights
    act2 = np.ascontiguousarray(act[::-1])
    backend.ternary_gemv_preq(w, ws, act2, aa, out, m, k)
    np.testing.assert_array_equal(out, ref(w, ws, act2, aa, m, k))
    # weights rewritten in place: the mirror is stale until invalidated
    w[:] = oracle.pack_rows(-np.ones((m, k), np.int8)).reshape(-1)
    backend.mirror_invalidate()
    backend.ternary_gemv_preq(w, ws, act, aa, out, m, k)
    np.testing.assert_array_equal(out, ref(w, ws, act, aa, m, k))


def test_gemv_same_address_new_matrix(backend):
    """A different matrix at the same address and length (a freed host buffer
    reused by the allocator) is detected by the mirror's content sample."""
    case("ternary gemv same-address matrix")
    m, k = 2560, 6912
    w, act, ws, aa = workload(11, m, k)
    out = np.zeros(m, f32)
    backend.ternary_gemv_preq(w, ws, act, aa, out, m, k)
    np.testing.assert_array_equal(out, ref(w, ws, act, aa, m, k))
    w2, _, _, _ = workload(12, m, k)
    w[:] = w2
    backend.ternary_gemv_preq(w, ws, act, aa, out, m, k)
    np.testing.assert_array_equal(out, ref(w, ws, act, aa, m, k))


@pytest.mark.parametrize("shapes,k", [([2560, 640, 640], 2560), ([6912, 6912], 2560),
                                      ([37, 0, 5, 16, 1, 3, 2, 100], 999)])
def test_device_gemv_group_bit_exact(backend, shapes, k):
    """One launch for matrices sharing the activation (q/k/v, gate/up),
    including an empty matrix and a group of eight with odd sizes."""
    case(f"ternary gemv group {shapes} k {k}")
    import torch

    rng = np.random.default_rng(len(shapes) * 1000 + k)
    act = rng.integers(-128, 128, size=k).astype(np.int8)
    aa = f32(7.5)
    ws, dws, outs, refs, scales = [], [], [], [], []
    for i, m in enumerate(shapes):
        w, _, s_, _ = workload(3000 + 17 * i + k, m, k, garbage=0.02)
        ws.append(w)
        scales.append(s_)
        dws.append(torch.from_numpy(w).cuda() if w.size else torch.zeros(16, dtype=torch.uint8, device="cuda"))
        outs.append(torch.full((max(m, 1),), float("nan"), device="cuda"))
        refs.append(ref(w, s_, act, aa, m, k))
    backend.dev_ternary_gemv_preq_group(dws, scales, torch.from_numpy(act).cuda(), aa, outs,
                                        shapes, k)
    torch.cuda.synchronize()
    for m, o, r in zip(shapes, outs, refs):
        np.testing.assert_array_equal(o.cpu().numpy()[:m], r)


def test_device_gemv_group_errors(backend):
    case("ternary gemv group errors")
    import bitnetrs_amd
    import torch

    a = torch.zeros(8, dtype=torch.int8, device="cuda")
    w = torch.zeros(64, dtype=torch.uint8, device="cuda")
    o = torch.zeros(8, device="cuda")
    with pytest.raises(bitnetrs_amd.InvalidConfig):
        backend.dev_ternary_gemv_preq_group([w] * 9, [1.0] * 9, a, 1.0, [o] * 9, [8] * 9, 8)
    with pytest.raises(bitnetrs_amd.QuantizationError, match="weight_scale must be finite > 0, got 0"):
        backend.dev_ternary_gemv_preq_group([w, w], [1.0, 0.0], a, 1.0, [o, o], [8, 8], 8)
