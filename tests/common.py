"""Shared helpers for the test suite: tolerance rule, seeded workloads, fp64
brute force.

Tolerance (fp32 I/O): per element |gpu - ref| <= ATOL + RTOL * |ref| with
ATOL = 2e-3, RTOL = 1e-3 (allclose semantics); max-abs and max-rel are
reported separately in the failure message.  Attention outputs are also
held to a bound on the output's scale, |gpu - ref| <= SCALE_FLOOR +
SCALE_REL * max|ref| (assert_close_scaled): tight enough that a missing or
extra attended row fails it at the long contexts tested, where the
per-element rule alone would not.
"""
from __future__ import annotations

import numpy as np

import oracle

ATOL = 2e-3
RTOL = 1e-3
SCALE_FLOOR = 1e-5
SCALE_REL = 1e-4

# BitNet b1.58 2B attention shape (bitnet-core/src/config.rs:161-173).
HQ, HKV, D, THETA = 20, 5, 128, 500000.0


# BitNetError's Display format of each variant the path returns
# (bitnet-core/src/error.rs:17-55), by the library's status code.
RUST_DISPLAY = {
    1: "invalid tensor shape: expected {0}, got {1}",  # InvalidShape { expected, got }
    2: "invalid model configuration: {0}",  # InvalidConfig(String)
    3: "backend error ({0}): {1}",  # BackendError { backend, message }
    4: "unsupported device: {0}",  # UnsupportedDevice(String)
    5: "quantization error: {0}",  # QuantizationError(String)
}


def error_from_parts() -> tuple:
    """(status, Display) of the calling thread's last library error, the
    Display rebuilt from bnr_last_error_parts' fields with the Rust format
    string -- what a binding that constructs the variant prints.  Checks that
    a one-field variant leaves the second field empty and that the rebuilt
    text equals bnr_last_error()."""
    import ctypes

    from bitnetrs_amd import _lib

    lib = _lib.load()
    first, second = ctypes.c_char_p(), ctypes.c_char_p()
    kind = lib.bnr_last_error_parts(ctypes.byref(first), ctypes.byref(second))
    a, b = first.value.decode(), second.value.decode()
    if kind == 0:
        return 0, ""
    if kind not in (1, 3):
        assert b == "", (kind, a, b)
    assert a != "", (kind, a, b)
    text = RUST_DISPLAY[kind].format(a, b)
    assert text == lib.bnr_last_error().decode(), (text, lib.bnr_last_error())
    return kind, text


def seed(cfg: int, tensor_id: int) -> int:
    """Seed of tensor `tensor_id` of workload `cfg`: 0xB17E7000 + 16*cfg + id."""
    return 0xB17E7000 + 16 * cfg + tensor_id


def assert_close(got, ref, what: str = "", atol: float = ATOL, rtol: float = RTOL) -> dict:
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert got.shape == ref.shape, f"{what}: shape {got.shape} != {ref.shape}"
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    err = np.abs(got - ref)
    max_abs = float(err.max()) if err.size else 0.0
    rel = err / np.maximum(np.abs(ref), 1e-30)
    max_rel = float(rel.max()) if rel.size else 0.0
    bad = err > atol + rtol * np.abs(ref)
    n_bad = int(bad.sum())
    assert n_bad == 0, (f"{what}: {n_bad}/{err.size} elements outside "
                        f"|d| <= {atol} + {rtol}|ref| (max_abs={max_abs:.3e}, "
                        f"max_rel={max_rel:.3e})")
    return {"max_abs": max_abs, "max_rel": max_rel}


def assert_close_scaled(got, ref, what: str = "", floor: float = SCALE_FLOOR,
                        rel: float = SCALE_REL) -> dict:
    """The per-element rule of assert_close, plus |gpu - ref| <= floor +
    rel * max|ref| over the whole output."""
    res = assert_close(got, ref, what)
    ref64 = np.asarray(ref, dtype=np.float64)
    bound = floor + rel * (float(np.abs(ref64).max()) if ref64.size else 0.0)
    assert res["max_abs"] <= bound, (f"{what}: max_abs {res['max_abs']:.3e} above the output-scale "
                                     f"bound {bound:.3e} ({floor} + {rel} max|ref|)")
    return res


# ----------------------------------------------------------------------------
# fp64 brute force (independent of the oracle's code)
# ----------------------------------------------------------------------------

def attention_f64(q, k_cache, v_cache, n_heads, n_kv_heads, head_dim, cur_pos):
    """Scaled dot-product GQA attention over rows 0..=cur_pos in float64;
    the caches are head-major with per-head stride len/n_kv."""
    q = np.asarray(q, np.float64).reshape(n_heads, head_dim)
    stride = k_cache.size // n_kv_heads
    L = cur_pos + 1
    K = np.stack([np.asarray(k_cache[h * stride:h * stride + L * head_dim], np.float64)
                  .reshape(L, head_dim) for h in range(n_kv_heads)])
    V = np.stack([np.asarray(v_cache[h * stride:h * stride + L * head_dim], np.float64)
                  .reshape(L, head_dim) for h in range(n_kv_heads)])
    g = n_heads // n_kv_heads
    out = np.empty((n_heads, head_dim))
    for h in range(n_heads):
        s = K[h // g] @ q[h] / np.sqrt(head_dim)
        p = np.exp(s - s.max())
        p /= p.sum()
        out[h] = p @ V[h // g]
    return out.reshape(-1)


# ----------------------------------------------------------------------------
# Seeded workloads
# ----------------------------------------------------------------------------

def decode_workload(cfg: int, pos: int, cap: int = 4096, q_scale: float = 1.0,
                    n_heads: int = HQ, n_kv: int = HKV, head_dim: int = D):
    """One decode step at `pos`: cached rows 0..pos-1 ~ N(0,1) (taken as
    already rotated), raw q ~ N(0,1)*q_scale, raw k and v ~ N(0,1).
    Returns dict with head-major host caches [n_kv, cap, d] (rows >= pos are
    zero)."""
    kc = np.zeros((n_kv, cap, head_dim), np.float32)
    vc = np.zeros_like(kc)
    if pos:
        kc[:, :pos] = oracle.normal(seed(cfg, 3), (n_kv, pos, head_dim))
        vc[:, :pos] = oracle.normal(seed(cfg, 4), (n_kv, pos, head_dim))
    return {
        "q": oracle.normal(seed(cfg, 0), (n_heads * head_dim,), q_scale),
        "k": oracle.normal(seed(cfg, 1), (n_kv * head_dim,)),
        "v": oracle.normal(seed(cfg, 2), (n_kv * head_dim,)),
        "k_cache": kc, "v_cache": vc, "pos": pos, "cap": cap,
    }


def oracle_decode(w, n_heads=HQ, n_kv=HKV, head_dim=D, theta=THETA):
    """Reference call sequence for one token: rope_embed -> store_kv ->
    masked_attention (bitnet-model/src/lib.rs:1004-1036).  Returns
    (q_rot, k_rot, k_cache, v_cache, out) without modifying `w`."""
    be = oracle.CpuBackend()
    q = w["q"].copy()
    k = w["k"].copy()
    be.rope_embed(q, k, w["pos"], head_dim, n_heads, n_kv, theta)
    kc = w["k_cache"].copy()
    vc = w["v_cache"].copy()
    kc[:, w["pos"]] = k.reshape(n_kv, head_dim)
    vc[:, w["pos"]] = w["v"].reshape(n_kv, head_dim)
    out = np.zeros(n_heads * head_dim, np.float32)
    be.masked_attention(q, kc.reshape(-1), vc.reshape(-1), out, n_heads, n_kv, head_dim,
                        w["pos"])
    return q, k, kc, vc, out


def prefill_workload(cfg: int, n_tokens: int, n_heads: int = HQ, n_kv: int = HKV,
                     head_dim: int = D):
    return {
        "q": oracle.normal(seed(cfg, 0), (n_tokens, n_heads * head_dim)),
        "k": oracle.normal(seed(cfg, 1), (n_tokens, n_kv * head_dim)),
        "v": oracle.normal(seed(cfg, 2), (n_tokens, n_kv * head_dim)),
    }


def oracle_prefill(w, start_pos=0, cap=None, n_heads=HQ, n_kv=HKV, head_dim=D, theta=THETA,
                   cache=None, layer=0, backend=None):
    """n_tokens serial rope -> store_kv -> masked_attention calls of one layer
    (bitnet-model/src/lib.rs:684-718).  Returns (q_rot, k_rot, KVCache, out)."""
    n = w["q"].shape[0]
    cap = cap or max(start_pos + n, 1)
    if cache is None:
        cache = oracle.KVCache(1, n_kv, head_dim, cap)
    if backend is None:
        backend = oracle.CpuBackend()
    q = w["q"].copy()
    k = w["k"].copy()
    out = oracle.layer_tokens(backend, cache, layer, q, k, w["v"], start_pos, n_heads, n_kv,
                              head_dim, theta)
    return q, k, cache, out


def batched_lengths(n: int = 32, lo: int = 128, hi: int = 4096, cfg: int = 4):
    """Cached lengths ~ U[lo, hi) (half-open, as Rust's gen_range) from a
    seeded PCG64 stream."""
    rng = np.random.default_rng(seed(cfg, 15))
    return rng.integers(lo, hi, size=n).astype(np.int32)


# ----------------------------------------------------------------------------
# Whole decode token through the layer stack (oracle composition)
# ----------------------------------------------------------------------------

def make_decode_model(seed, hidden, n_heads, n_kv, head_dim, ffn, n_layers, vocab):
    """Seeded synthetic BitNet weights: ternary projections (packed rows),
    absmean scales, RMSNorm weights, i8 LM head with per-row scales."""
    rng = np.random.default_rng(seed)
    q_dim, kv_dim = n_heads * head_dim, n_kv * head_dim
    shapes = [(q_dim, hidden), (kv_dim, hidden), (kv_dim, hidden), (hidden, q_dim),
              (ffn, hidden), (ffn, hidden), (hidden, ffn)]
    layers = []
    for _ in range(n_layers):
        mats = [oracle.pack_rows(rng.integers(-1, 2, size=s).astype(np.int8)) for s in shapes]
        scales = [float(np.float32(rng.uniform(0.02, 0.08))) for _ in shapes]
        norms = [rng.uniform(0.8, 1.2, size=n).astype(np.float32)
                 for n in (hidden, q_dim, hidden, ffn)]
        layers.append({"mats": mats, "shapes": shapes, "scales": scales, "norms": norms})
    return {"layers": layers, "final_norm": rng.uniform(0.8, 1.2, hidden).astype(np.float32),
            "lm_w": rng.integers(-128, 128, size=(vocab, hidden)).astype(np.int8),
            "lm_scales": rng.uniform(0.001, 0.01, vocab).astype(np.float32),
            "dims": (hidden, n_heads, n_kv, head_dim, ffn, n_layers, vocab)}


def oracle_decode_token(model, h, position, cache, backend, theta=THETA, eps=1e-5):
    """BitNetModel::forward_into's decode path for one token
    (bitnet-model/src/lib.rs:946-1163) composed from the oracle's pinned
    functions.  h [hidden] is updated in place; returns the logits."""
    hidden, n_heads, n_kv, hd, ffn, n_layers, vocab = model["dims"]
    f32 = np.float32

    def gemv(mat, shape, scale, x_q, absmax):
        out = np.zeros(shape[0], f32)
        oracle.ternary_gemv_preq(mat, scale, x_q, absmax, out, shape[0], shape[1])
        return out

    def norm_quant(x, g):
        y = np.zeros(x.size, f32)
        oracle.rms_norm(x, g, eps, y)
        q, sc = oracle.absmax_quantize_row(y)
        return q, float(f32(f32(sc) * f32(127.0)))

    for li, L in enumerate(model["layers"]):
        m, sh, sc, nm = L["mats"], L["shapes"], L["scales"], L["norms"]
        xq, aa = norm_quant(h, nm[0])
        q, k, v = (gemv(m[i], sh[i], sc[i], xq, aa) for i in range(3))
        backend.rope_embed(q, k, position, hd, n_heads, n_kv, theta)
        cache.store_kv(li, position, k, v)
        attn = np.zeros(n_heads * hd, f32)
        backend.masked_attention(q, cache.k(li), cache.v(li), attn, n_heads, n_kv, hd, position)
        xq, aa = norm_quant(attn, nm[1])
        o = gemv(m[3], sh[3], sc[3], xq, aa)
        oracle.axpy(1.0, o, h)
        xq, aa = norm_quant(h, nm[2])
        gate, up = gemv(m[4], sh[4], sc[4], xq, aa), gemv(m[5], sh[5], sc[5], xq, aa)
        inner = np.zeros(ffn, f32)
        oracle.sqrelu_gate(gate, up, inner)
        xq, aa = norm_quant(inner, nm[3])
        down = gemv(m[6], sh[6], sc[6], xq, aa)
        oracle.axpy(1.0, down, h)
    cache.advance()
    fin = np.zeros(hidden, f32)
    oracle.rms_norm(h, model["final_norm"], eps, fin)
    logits = np.zeros(vocab, f32)
    oracle.lm_head_matmul_i8(fin, model["lm_w"], model["lm_scales"], logits, vocab, hidden)
    return logits
