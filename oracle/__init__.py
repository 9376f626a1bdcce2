"""ctypes view of the CPU restatement of bitnetrs's GQA attention hot path.

TEST INFRASTRUCTURE ONLY: imported by ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py``, always as the checker or the
reported CPU baseline, never as the thing measured or shipped.

Each wrapper names the reference function (file:line) whose arithmetic the C
code in ``bnr_oracle.c`` restates.  Errors are raised as the same exception
classes the product binding uses, so a test can compare error *kinds*.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libbnr_oracle.so")

OK, INVALID_SHAPE, INVALID_CONFIG, BACKEND_ERROR, QUANTIZATION_ERROR = 0, 1, 2, 3, 5


class OracleError(Exception):
    """Base class; ``kind`` is the status code (bitnet-core/src/error.rs:12-55)."""

    kind = -1


class InvalidShape(OracleError):
    kind = INVALID_SHAPE


class InvalidConfig(OracleError):
    kind = INVALID_CONFIG


class BackendError(OracleError):
    kind = BACKEND_ERROR


class QuantizationError(OracleError):
    kind = QUANTIZATION_ERROR


_ERR = {INVALID_SHAPE: InvalidShape, INVALID_CONFIG: InvalidConfig, BACKEND_ERROR: BackendError,
        QUANTIZATION_ERROR: QuantizationError}


def build() -> str:
    """Compile the oracle with its Makefile (gcc, no GPU needed)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = ctypes.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


_f = ctypes.POINTER(ctypes.c_float)
_sz = ctypes.c_size_t


def _declare(L: ctypes.CDLL) -> None:
    L.bnro_last_error.restype = ctypes.c_char_p
    L.bnro_fill_normal.argtypes = [ctypes.c_uint64, _f, _sz, ctypes.c_float]
    L.bnro_dot_f32.argtypes = [_f, _f, _sz]
    L.bnro_dot_f32.restype = ctypes.c_float
    L.bnro_axpy_f32.argtypes = [ctypes.c_float, _f, _f, _sz]
    L.bnro_softmax_f32.argtypes = [_f, _sz]
    L.bnro_force_scalar.argtypes = [ctypes.c_int]
    L.bnro_rope_table.argtypes = [_sz, _sz, ctypes.c_float, _f, _f]
    L.bnro_apply_rope.argtypes = [_f, _sz, _f, _sz, _sz, _sz, _sz, _sz, ctypes.c_float]
    L.bnro_apply_rope_cached.argtypes = [_f, _sz, _f, _sz, _sz, _sz, _sz, _f, _f, _sz, _sz]
    L.bnro_masked_attention.argtypes = [_f, _sz, _f, _sz, _f, _sz, _f, _sz, _sz, _sz, _sz, _sz]
    L.bnro_backend_new.restype = ctypes.c_void_p
    L.bnro_backend_free.argtypes = [ctypes.c_void_p]
    L.bnro_backend_rope_embed.argtypes = [ctypes.c_void_p, _f, _sz, _f, _sz, _sz, _sz, _sz, _sz, ctypes.c_float]
    L.bnro_backend_rope_state.argtypes = [ctypes.c_void_p, ctypes.POINTER(_sz), ctypes.POINTER(_sz), _f]
    L.bnro_kv_new.argtypes = [_sz, _sz, _sz, _sz]
    L.bnro_kv_new.restype = ctypes.c_void_p
    L.bnro_kv_free.argtypes = [ctypes.c_void_p]
    L.bnro_kv_store.argtypes = [ctypes.c_void_p, _sz, _sz, _f, _sz, _f, _sz]
    L.bnro_kv_advance.argtypes = [ctypes.c_void_p]
    L.bnro_kv_clear.argtypes = [ctypes.c_void_p]
    L.bnro_kv_len.argtypes = [ctypes.c_void_p]
    L.bnro_kv_len.restype = _sz
    L.bnro_kv_layer_len.argtypes = [ctypes.c_void_p, _sz]
    L.bnro_kv_layer_len.restype = _sz
    L.bnro_kv_k.argtypes = [ctypes.c_void_p, _sz]
    L.bnro_kv_k.restype = _f
    L.bnro_kv_v.argtypes = [ctypes.c_void_p, _sz]
    L.bnro_kv_v.restype = _f
    L.bnro_kv_backing_len.argtypes = [ctypes.c_void_p]
    L.bnro_kv_backing_len.restype = _sz
    L.bnro_layer_tokens.argtypes = [ctypes.c_void_p, ctypes.c_void_p, _sz, _f, _f, _f, _sz, _sz,
                                    _sz, _sz, _sz, ctypes.c_float, _f]
    L.bnro_set_threads.argtypes = [ctypes.c_int]
    L.bnro_get_threads.restype = ctypes.c_int
    _u8 = ctypes.c_void_p
    L.bnro_pack_ternary.argtypes = [_u8, _sz, _u8]
    L.bnro_dot_packed_ternary_i8.argtypes = [_u8, _u8, _sz]
    L.bnro_dot_packed_ternary_i8.restype = ctypes.c_int32
    L.bnro_ternary_gemv_preq.argtypes = [_u8, _sz, ctypes.c_float, _u8, _sz, ctypes.c_float, _f,
                                         _sz, _sz, _sz]
    L.bnro_dot_f32_i8w.argtypes = [_u8, _f, _sz]
    L.bnro_dot_f32_i8w.restype = ctypes.c_float
    L.bnro_lm_head_matmul_i8.argtypes = [_f, _sz, _u8, _sz, _f, _sz, _f, _sz, _sz, _sz]
    L.bnro_sum_squares_f32.argtypes = [_f, _sz]
    L.bnro_sum_squares_f32.restype = ctypes.c_float
    L.bnro_rms_norm.argtypes = [_f, _sz, _f, _sz, ctypes.c_float, _f, _sz]
    L.bnro_absmax_quantize_row.argtypes = [_f, _sz, _u8, _sz, ctypes.POINTER(ctypes.c_float)]
    L.bnro_sqrelu_gate.argtypes = [_f, _sz, _f, _sz, _f, _sz]


def _check(status: int) -> None:
    if status != OK:
        msg = lib().bnro_last_error().decode()
        raise _ERR.get(status, OracleError)(msg)


def _ptr(a: np.ndarray):
    if a.dtype != np.float32 or not a.flags.c_contiguous:
        raise TypeError("oracle arrays must be C-contiguous float32")
    if a.size == 0:
        return _f()
    return a.ctypes.data_as(_f)


# ----------------------------------------------------------------------------
# inputs
# ----------------------------------------------------------------------------

def normal(seed: int, shape, scale: float = 1.0) -> np.ndarray:
    """Seeded N(0,1)*scale float32 array (SplitMix64 -> Box-Muller in f64)."""
    out = np.empty(shape, dtype=np.float32)
    lib().bnro_fill_normal(ctypes.c_uint64(seed & (2**64 - 1)), _ptr(out), out.size, scale)
    return out


# ----------------------------------------------------------------------------
# primitives
# ----------------------------------------------------------------------------

def dot(a: np.ndarray, b: np.ndarray) -> float:
    """simd::dot_f32_f32_fast  bitnet-cpu/src/simd.rs:711-720."""
    return lib().bnro_dot_f32(_ptr(a), _ptr(b), a.size)


def axpy(alpha: float, x: np.ndarray, out: np.ndarray) -> None:
    """simd::axpy_f32_fast  bitnet-cpu/src/simd.rs:772-782 (in place on out)."""
    lib().bnro_axpy_f32(alpha, _ptr(x), _ptr(out), x.size)


def softmax(x: np.ndarray) -> None:
    """ops::softmax_f32  bitnet-core/src/backend/ops.rs:206-226 (in place)."""
    lib().bnro_softmax_f32(_ptr(x), x.size)


def force_scalar(on: bool) -> None:
    lib().bnro_force_scalar(1 if on else 0)


def set_threads(n: int) -> None:
    lib().bnro_set_threads(n)


def get_threads() -> int:
    return lib().bnro_get_threads()


# ----------------------------------------------------------------------------
# RoPE
# ----------------------------------------------------------------------------

def rope_table(max_seq: int, head_dim: int, theta: float):
    """RopeCache::new  bitnet-cpu/src/rope.rs:100-153 -> (cos, sin) [max_seq, d/2]."""
    half = max(head_dim // 2, 0)
    c = np.zeros((max(max_seq, 0), half), np.float32)
    s = np.zeros_like(c)
    _check(lib().bnro_rope_table(max_seq, head_dim, theta, _ptr(c) if c.size else _f(),
                                 _ptr(s) if s.size else _f()))
    return c, s


def apply_rope(q, k, position, head_dim, n_heads, n_kv_heads, theta) -> None:
    """apply_rope (uncached)  bitnet-cpu/src/rope.rs:227-292 (in place)."""
    _check(lib().bnro_apply_rope(_ptr(q), q.size, _ptr(k), k.size, position, head_dim,
                                 n_heads, n_kv_heads, theta))


def apply_rope_cached(q, k, position, n_heads, n_kv_heads, cos, sin, head_dim) -> None:
    """apply_rope_cached  bitnet-cpu/src/rope.rs:312-355 (in place)."""
    _check(lib().bnro_apply_rope_cached(_ptr(q), q.size, _ptr(k), k.size, position, n_heads,
                                        n_kv_heads, _ptr(cos), _ptr(sin), cos.shape[0],
                                        head_dim))


# ----------------------------------------------------------------------------
# attention
# ----------------------------------------------------------------------------

def masked_attention(q, k_cache, v_cache, output, n_heads, n_kv_heads, head_dim, cur_pos) -> None:
    """attention::masked_attention  bitnet-cpu/src/attention.rs:97-209."""
    _check(lib().bnro_masked_attention(_ptr(q), q.size, _ptr(k_cache), k_cache.size,
                                       _ptr(v_cache), v_cache.size, _ptr(output), output.size,
                                       n_heads, n_kv_heads, head_dim, cur_pos))


class CpuBackend:
    """CpuBackend's rope_embed / masked_attention (bitnet-cpu/src/lib.rs:289-347)."""

    def __init__(self):
        self._h = lib().bnro_backend_new()

    def __del__(self):
        if getattr(self, "_h", None):
            lib().bnro_backend_free(self._h)
            self._h = None

    def rope_embed(self, q, k, position, head_dim, n_heads, n_kv_heads, theta) -> None:
        _check(lib().bnro_backend_rope_embed(self._h, _ptr(q), q.size, _ptr(k), k.size, position,
                                             head_dim, n_heads, n_kv_heads, theta))

    def rope_state(self):
        ms, hd, th = _sz(), _sz(), ctypes.c_float()
        if not lib().bnro_backend_rope_state(self._h, ctypes.byref(ms), ctypes.byref(hd),
                                             ctypes.byref(th)):
            return None
        return ms.value, hd.value, th.value

    def masked_attention(self, q, k_cache, v_cache, output, n_heads, n_kv_heads, head_dim,
                         cur_pos) -> None:
        masked_attention(q, k_cache, v_cache, output, n_heads, n_kv_heads, head_dim, cur_pos)


class KVCache:
    """KVCache  bitnet-model/src/lib.rs:118-292 (head-major per layer)."""

    def __init__(self, n_layers, n_kv_heads, head_dim, max_seq):
        self.n_layers, self.n_kv_heads, self.head_dim, self.max_seq = (
            n_layers, n_kv_heads, head_dim, max_seq)
        self._h = lib().bnro_kv_new(n_layers, n_kv_heads, head_dim, max_seq)

    def __del__(self):
        if getattr(self, "_h", None):
            lib().bnro_kv_free(self._h)
            self._h = None

    def store_kv(self, layer, position, k_vec, v_vec) -> None:
        _check(lib().bnro_kv_store(self._h, layer, position, _ptr(k_vec), k_vec.size,
                                   _ptr(v_vec), v_vec.size))

    def advance(self) -> None:
        _check(lib().bnro_kv_advance(self._h))

    def clear(self) -> None:
        lib().bnro_kv_clear(self._h)

    def __len__(self) -> int:
        return lib().bnro_kv_len(self._h)

    def layer_len(self, layer) -> int:
        return lib().bnro_kv_layer_len(self._h, layer)

    def _view(self, p):
        n = lib().bnro_kv_backing_len(self._h)
        return np.ctypeslib.as_array(p, shape=(n,))

    def k(self, layer) -> np.ndarray:
        """Whole backing buffer of layer (a live view), as k_slice returns."""
        return self._view(lib().bnro_kv_k(self._h, layer))

    def v(self, layer) -> np.ndarray:
        return self._view(lib().bnro_kv_v(self._h, layer))


def layer_tokens(backend: CpuBackend, cache: KVCache, layer, q_raw, k_raw, v_raw, start_pos,
                 n_heads, n_kv_heads, head_dim, theta) -> np.ndarray:
    """Per-token rope -> store_kv -> masked_attention sequence of one layer
    (BitNetModel::forward, bitnet-model/src/lib.rs:684-718).  q_raw/k_raw are
    rotated in place; returns out [n_tokens, n_heads*head_dim]."""
    n = q_raw.shape[0]
    out = np.zeros((n, n_heads * head_dim), np.float32)
    _check(lib().bnro_layer_tokens(backend._h, cache._h, layer, _ptr(q_raw), _ptr(k_raw),
                                   _ptr(v_raw), n, start_pos, n_heads, n_kv_heads, head_dim,
                                   theta, _ptr(out)))
    return out


# ----------------------------------------------------------------------------
# W2A8 ternary GEMV
# ----------------------------------------------------------------------------

def _bytes_ptr(a: np.ndarray, dtype) -> ctypes.c_void_p:
    if a.dtype != dtype or not a.flags.c_contiguous:
        raise TypeError(f"oracle arrays must be C-contiguous {np.dtype(dtype).name}")
    return ctypes.c_void_p(a.ctypes.data if a.size else 0)


def pack_ternary(w: np.ndarray) -> np.ndarray:
    """pack_ternary (bitnet-core/src/quant/ternary.rs:266-286) of one row."""
    w = np.ascontiguousarray(w, np.int8)
    out = np.zeros((w.size + 3) // 4, np.uint8)
    _check(lib().bnro_pack_ternary(_bytes_ptr(w, np.int8), w.size, _bytes_ptr(out, np.uint8)))
    return out


def pack_rows(w: np.ndarray) -> np.ndarray:
    """Row-aligned packing of a [rows, cols] ternary matrix (each row padded
    to ceil(cols/4) bytes), as the model's weight loader stores it."""
    return np.stack([pack_ternary(r) for r in np.asarray(w, np.int8)]) if len(w) else \
        np.zeros((0, (np.asarray(w).shape[1] + 3) // 4), np.uint8)


def dot_packed_ternary_i8(packed: np.ndarray, act: np.ndarray, n: int) -> int:
    return int(lib().bnro_dot_packed_ternary_i8(_bytes_ptr(packed, np.uint8),
                                                _bytes_ptr(act, np.int8), n))


def ternary_gemv_preq(weight_packed, weight_scale, activation_q, act_absmax, output,
                      out_features, in_features) -> None:
    """CpuBackend::ternary_gemv_preq (bitnet-cpu/src/lib.rs:519-538 ->
    gemv::ternary_gemv_quantised, gemv.rs:251-310)."""
    w = np.ascontiguousarray(weight_packed, np.uint8).reshape(-1)
    a = np.ascontiguousarray(activation_q, np.int8).reshape(-1)
    _check(lib().bnro_ternary_gemv_preq(_bytes_ptr(w, np.uint8), w.size, weight_scale,
                                        _bytes_ptr(a, np.int8), a.size, act_absmax,
                                        _ptr(output), output.size, out_features, in_features))


# ----------------------------------------------------------------------------
# LM head with i8 weights
# ----------------------------------------------------------------------------

def dot_f32_i8w(w: np.ndarray, hidden: np.ndarray) -> float:
    """simd::dot_f32_i8w_fast (bitnet-cpu/src/simd.rs:1255-1269)."""
    w = np.ascontiguousarray(w, np.int8)
    return float(lib().bnro_dot_f32_i8w(_bytes_ptr(w, np.int8), _ptr(hidden), w.size))


def lm_head_matmul_i8(hidden, weights_i8, scales, output, vocab_size, hidden_size) -> None:
    """CpuBackend::lm_head_matmul_i8_into (bitnet-cpu/src/lib.rs:544-575)."""
    w = np.ascontiguousarray(weights_i8, np.int8).reshape(-1)
    _check(lib().bnro_lm_head_matmul_i8(_ptr(hidden), hidden.size, _bytes_ptr(w, np.int8), w.size,
                                        _ptr(scales), scales.size, _ptr(output), output.size,
                                        vocab_size, hidden_size))


# ----------------------------------------------------------------------------
# Layer glue
# ----------------------------------------------------------------------------

def sum_squares(x: np.ndarray) -> float:
    return float(lib().bnro_sum_squares_f32(_ptr(x), x.size))


def rms_norm(input, weight, eps, output) -> None:
    """norm::rms_norm (bitnet-cpu/src/norm.rs:76-136)."""
    _check(lib().bnro_rms_norm(_ptr(input), input.size, _ptr(weight), weight.size, eps,
                               _ptr(output), output.size))


def absmax_quantize_row(x: np.ndarray, out: np.ndarray = None):
    """absmax_quantize_row_into (bitnet-core/src/quant/absmax.rs:127-170);
    returns (q, scale) with scale = max|x| / 127."""
    if out is None:
        out = np.zeros(x.size, np.int8)
    sc = ctypes.c_float()
    _check(lib().bnro_absmax_quantize_row(_ptr(x), x.size, _bytes_ptr(out, np.int8), out.size,
                                          ctypes.byref(sc)))
    return out, float(np.float32(sc.value))


def sqrelu_gate(gate, up, out) -> None:
    """CpuBackend::sqrelu_gate (bitnet-cpu/src/lib.rs:494-509)."""
    _check(lib().bnro_sqrelu_gate(_ptr(gate), gate.size, _ptr(up), up.size, _ptr(out), out.size))
