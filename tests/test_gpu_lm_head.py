"""GPU parity of the i8-weight LM head (Backend::lm_head_matmul_i8_into)
against the oracle, through the C ABI.  fp32 sums in a different order than
the reference's AVX2 lanes: each logit must lie within the fp32 rounding
bound of the exact (fp64) value, 4*K*eps*sum|w*h|*scale, and within
|gpu - oracle| <= 2e-3 + 1e-3*|oracle|."""
import sys

import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu
f32 = np.float32


def case(msg):
    print(f"[gpu case] {msg}", flush=True)
    sys.stdout.flush()


def workload(seed, v, h):
    rng = np.random.default_rng(seed)
    hid = rng.standard_normal(h).astype(f32)
    w = rng.integers(-128, 128, size=(v, h)).astype(np.int8)
    sc = rng.uniform(0.001, 0.03, size=v).astype(f32)
    return hid, w, sc


def check(got, hid, w, sc):
    v, h = w.shape
    ref = np.full(v, np.nan, f32)
    oracle.lm_head_matmul_i8(hid, w, sc, ref, v, h)
    exact = (w.astype(np.float64) @ hid.astype(np.float64)) * sc
    mag = (np.abs(w).astype(np.float64) @ np.abs(hid).astype(np.float64)) * sc
    bound = 4 * max(h, 1) * np.finfo(f32).eps * mag + 1e-30
    assert np.all(np.abs(got.astype(np.float64) - exact) <= bound)
    err = np.abs(got - ref)
    assert np.all(err <= 2e-3 + 1e-3 * np.abs(ref)), float(err.max())
    return float(err.max())


@pytest.mark.parametrize("v,h", [(128256, 2560), (1000, 2560), (129, 100), (300, 4100), (7, 9000)])
def test_host_lm_head(backend, v, h):
    case(f"lm head host vocab {v} hidden {h}")
    hid, w, sc = workload(v + h, v, h)
    out = np.full(v, np.nan, f32)
    backend.lm_head_matmul_i8_into(hid, w.reshape(-1), sc, out, v, h)
    print(f"max |gpu - oracle| {check(out, hid, w, sc):.3e}")


@pytest.mark.parametrize("v,h,offset", [(128256, 2560, 0), (5000, 2560, 4), (333, 2048, 1)])
def test_device_lm_head(backend, v, h, offset):
    """offset shifts the weight pointer by bytes (and hidden by floats) off
    16-byte alignment: the element-wise load path."""
    case(f"lm head device vocab {v} hidden {h} offset {offset}")
    import torch

    hid, w, sc = workload(7 * v + h, v, h)
    wb = torch.zeros(w.size + offset, dtype=torch.int8, device="cuda")
    wb[offset:] = torch.from_numpy(w.reshape(-1)).cuda()
    hb = torch.zeros(h + offset, device="cuda")
    hb[offset:] = torch.from_numpy(hid).cuda()
    out = torch.full((v,), float("nan"), device="cuda")
    backend.dev_lm_head_matmul_i8(hb[offset:], wb[offset:], torch.from_numpy(sc).cuda(), out, v, h)
    torch.cuda.synchronize()
    check(out.cpu().numpy(), hid, w, sc)


def test_lm_head_shape_errors_match_oracle(backend):
    case("lm head errors")
    import bitnetrs_amd

    w = np.zeros(12, np.int8)
    args = [(np.zeros(5, f32), w, np.ones(3, f32), np.zeros(3, f32), 3, 4),
            (np.zeros(4, f32), w, np.ones(2, f32), np.zeros(3, f32), 3, 4),
            (np.zeros(4, f32), w, np.ones(3, f32), np.zeros(4, f32), 3, 4),
            (np.zeros(4, f32), w, np.ones(3, f32), np.zeros(3, f32), 2, 4)]
    for a in args:
        with pytest.raises(oracle.InvalidShape) as oe:
            oracle.lm_head_matmul_i8(*a)
        with pytest.raises(bitnetrs_amd.InvalidShape) as ge:
            backend.lm_head_matmul_i8_into(*a)
        assert str(ge.value) == str(oe.value)
