"""Host-side mirror of the reference's Backend trait for the attention path.

``HipBackend`` exposes the two trait methods this library replaces,
``rope_embed`` (bitnet-core/src/backend/mod.rs:251-260) and
``masked_attention`` (mod.rs:301-311), with the trait's argument order,
in-place semantics and error kinds (``InvalidShape`` / ``InvalidConfig`` /
``BackendError``), plus the device-pointer entry points of the C ABI that
keep the KV cache resident in HBM.  All compute runs in libbitnet_hip.so on
the GPU; nothing here computes on the CPU.

Device entry points take ``torch`` CUDA tensors only as device memory; the
library sees raw pointers and the current HIP stream.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _lib
from ._lib import (BNR_MIRROR_FULL, BNR_MIRROR_INCREMENTAL, BackendError, BitNetError,
                   InvalidConfig, InvalidShape, QuantizationError, UnsupportedDevice)

__all__ = ["HipBackend", "DeviceKVCache", "NativeKVCache", "BitNetError", "InvalidShape", "InvalidConfig",
           "BackendError", "UnsupportedDevice", "QuantizationError", "BNR_MIRROR_FULL",
           "BNR_MIRROR_INCREMENTAL"]

_fp = ctypes.POINTER(ctypes.c_float)


def _host(a: np.ndarray, name: str):
    if not isinstance(a, np.ndarray) or a.dtype != np.float32 or not a.flags.c_contiguous:
        raise TypeError(f"{name} must be a C-contiguous float32 numpy array")
    return a.ctypes.data_as(_fp) if a.size else _fp()


def _host_bytes(a: np.ndarray, dtype, name: str):
    if not isinstance(a, np.ndarray) or a.dtype != dtype or not a.flags.c_contiguous:
        raise TypeError(f"{name} must be a C-contiguous {np.dtype(dtype).name} numpy array")
    return ctypes.c_void_p(a.ctypes.data if a.size else 0)


def _dev(t, name: str, allow_none: bool = False, dtype=None):
    if t is None:
        if allow_none:
            return None
        raise TypeError(f"{name} is required")
    import torch

    dtype = dtype or torch.float32
    if not (isinstance(t, torch.Tensor) and t.is_cuda and t.dtype == dtype
            and t.is_contiguous()):
        raise TypeError(f"{name} must be a contiguous {dtype} CUDA tensor")
    return ctypes.c_void_p(t.data_ptr())


def _stream(stream):
    if stream is None:
        import torch

        return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    if isinstance(stream, int):
        return ctypes.c_void_p(stream)
    return ctypes.c_void_p(stream.cuda_stream)


class HipBackend:
    """The HIP backend: CudaBackend's shape (bitnet-gpu-cuda/src/lib.rs:83-272)
    with rope_embed / masked_attention implemented on gfx950."""

    def __init__(self, device_id: int = 0):
        self._L = _lib.load()
        h = ctypes.c_void_p()
        _lib.check(self._L.bnr_create(int(device_id), ctypes.byref(h)))
        self._h = h
        self.device_id = device_id

    # lifecycle ------------------------------------------------------------
    def close(self) -> None:
        if getattr(self, "_h", None):
            self._L.bnr_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def device_name(self) -> str:
        return self._L.bnr_device_name(self._h).decode()

    # trait-shaped host entry points ----------------------------------------
    def rope_embed(self, q: np.ndarray, k: np.ndarray, position: int, head_dim: int,
                   n_heads: int, n_kv_heads: int, theta: float) -> None:
        """Backend::rope_embed: rotate q [n_heads*d] and k [n_kv_heads*d] in place."""
        _lib.check(self._L.bnr_rope_embed(self._h, _host(q, "q"), q.size, _host(k, "k"), k.size,
                                          position, head_dim, n_heads, n_kv_heads, theta))

    def masked_attention(self, q: np.ndarray, k_cache: np.ndarray, v_cache: np.ndarray,
                         output: np.ndarray, n_heads: int, n_kv_heads: int, head_dim: int,
                         cur_pos: int) -> None:
        """Backend::masked_attention over head-major host caches; output overwritten."""
        _lib.check(self._L.bnr_masked_attention(
            self._h, _host(q, "q"), q.size, _host(k_cache, "k_cache"), k_cache.size,
            _host(v_cache, "v_cache"), v_cache.size, _host(output, "output"), output.size,
            n_heads, n_kv_heads, head_dim, cur_pos))

    def ternary_gemv_preq(self, weight_packed: np.ndarray, weight_scale: float,
                          activation_q: np.ndarray, act_absmax: float, output: np.ndarray,
                          out_features: int, in_features: int) -> None:
        """Backend::ternary_gemv_preq (bitnet-core/src/backend/mod.rs:459-468): packed
        2-bit weights (uint8, mirrored in HBM on first use), int8 activations,
        output overwritten."""
        _lib.check(self._L.bnr_ternary_gemv_preq(
            self._h, _host_bytes(weight_packed, np.uint8, "weight_packed"), weight_packed.size,
            weight_scale, _host_bytes(activation_q, np.int8, "activation_q"), activation_q.size,
            act_absmax, _host(output, "output"), output.size, out_features, in_features))

    def lm_head_matmul_i8_into(self, hidden: np.ndarray, weights_i8: np.ndarray,
                               scales: np.ndarray, output: np.ndarray, vocab_size: int,
                               hidden_size: int) -> None:
        """Backend::lm_head_matmul_i8_into (bitnet-core/src/backend/mod.rs:486-509)."""
        _lib.check(self._L.bnr_lm_head_matmul_i8_into(
            self._h, _host(hidden, "hidden"), hidden.size,
            _host_bytes(weights_i8, np.int8, "weights_i8"), weights_i8.size,
            _host(scales, "scales"), scales.size, _host(output, "output"), output.size,
            vocab_size, hidden_size))

    def rms_norm(self, input: np.ndarray, weight: np.ndarray, eps: float,
                 output: np.ndarray) -> None:
        """Backend::rms_norm (CpuBackend: bitnet-cpu/src/norm.rs:76-136)."""
        _lib.check(self._L.bnr_rms_norm(self._h, _host(input, "input"), input.size,
                                        _host(weight, "weight"), weight.size, eps,
                                        _host(output, "output"), output.size))

    def sqrelu_gate(self, gate: np.ndarray, up: np.ndarray, out: np.ndarray) -> None:
        """Backend::sqrelu_gate (CpuBackend: bitnet-cpu/src/lib.rs:494-509)."""
        _lib.check(self._L.bnr_sqrelu_gate(self._h, _host(gate, "gate"), gate.size,
                                           _host(up, "up"), up.size, _host(out, "out"), out.size))

    def set_mirror_mode(self, mode: int) -> None:
        _lib.check(self._L.bnr_set_mirror_mode(self._h, mode))

    def set_deterministic(self, on: bool = True) -> None:
        """Decode launches merge their splits in a fixed order: the same
        inputs give the same output bits on every run (slower)."""
        _lib.check(self._L.bnr_set_deterministic(self._h, int(bool(on))))

    def mirror_invalidate(self) -> None:
        _lib.check(self._L.bnr_mirror_invalidate(self._h))

    # device entry points ---------------------------------------------------
    def dev_rope_append(self, q, k, v, n_tokens, start_pos, n_heads, n_kv_heads, head_dim, theta,
                        k_cache, v_cache, cap, stream=None) -> None:
        _lib.check(self._L.bnr_dev_rope_append(
            self._h, _dev(q, "q"), _dev(k, "k"), _dev(v, "v"), n_tokens, start_pos, n_heads,
            n_kv_heads, head_dim, theta, _dev(k_cache, "k_cache"), _dev(v_cache, "v_cache"), cap,
            _stream(stream)))

    def dev_decode_attention(self, q, k_cache, v_cache, cap, out, n_heads, n_kv_heads, head_dim,
                             cur_pos, stream=None) -> None:
        _lib.check(self._L.bnr_dev_decode_attention(
            self._h, _dev(q, "q"), _dev(k_cache, "k_cache"), _dev(v_cache, "v_cache"), cap,
            _dev(out, "out"), n_heads, n_kv_heads, head_dim, cur_pos, _stream(stream)))

    def dev_stream_read(self, a, b, stream=None) -> None:
        """Plain streaming read of two float32 CUDA tensors (measurement)."""
        _lib.check(self._L.bnr_dev_stream_read(self._h, _dev(a, "a"), a.numel() * 4, _dev(b, "b"),
                                               b.numel() * 4, _stream(stream)))

    def dev_stream_read_shape(self, a, b, threads: int, loads_per_lane: int,
                              nontemporal: bool = False, stream=None) -> None:
        """The streaming read in a chosen shape: workgroups of `threads`, each
        lane with `loads_per_lane` 16-byte loads in flight (measurement)."""
        _lib.check(self._L.bnr_dev_stream_read_shape(
            self._h, _dev(a, "a"), a.numel() * 4, _dev(b, "b"), b.numel() * 4, threads,
            loads_per_lane, int(nontemporal), _stream(stream)))

    def dev_decode_attention_noalloc(self, q, k_cache, v_cache, cap, out, n_heads, n_kv_heads,
                                     head_dim, cur_pos, stream=None) -> None:
        """dev_decode_attention without any device allocation (the merge state
        lives in the library's per-GPU device array); overlapping calls on one
        GPU race."""
        _lib.check(self._L.bnr_dev_decode_attention_noalloc(
            self._h, _dev(q, "q"), _dev(k_cache, "k_cache"), _dev(v_cache, "v_cache"), cap,
            _dev(out, "out"), n_heads, n_kv_heads, head_dim, cur_pos, _stream(stream)))

    def dev_decode_step(self, q, k, v, position, n_heads, n_kv_heads, head_dim, theta, k_cache,
                        v_cache, cap, out, q_rot=None, k_rot=None, stream=None) -> None:
        _lib.check(self._L.bnr_dev_decode_step(
            self._h, _dev(q, "q"), _dev(k, "k"), _dev(v, "v"), position, n_heads, n_kv_heads,
            head_dim, theta, _dev(k_cache, "k_cache"), _dev(v_cache, "v_cache"), cap,
            _dev(out, "out"), _dev(q_rot, "q_rot", True), _dev(k_rot, "k_rot", True),
            _stream(stream)))

    def dev_decode_step_batched(self, q, k, v, positions, n_heads, n_kv_heads, head_dim, theta,
                                k_caches, v_caches, cap, out, stream=None) -> None:
        pos = np.ascontiguousarray(np.asarray(positions, dtype=np.int32))
        _lib.check(self._L.bnr_dev_decode_step_batched(
            self._h, _dev(q, "q"), _dev(k, "k"), _dev(v, "v"),
            pos.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)), pos.size, n_heads, n_kv_heads,
            head_dim, theta, _dev(k_caches, "k_caches"), _dev(v_caches, "v_caches"), cap,
            _dev(out, "out"), _stream(stream)))

    def dev_prefill_attention(self, q, k_cache, v_cache, cap, out, n_tokens, start_pos, n_heads,
                              n_kv_heads, head_dim, stream=None) -> None:
        _lib.check(self._L.bnr_dev_prefill_attention(
            self._h, _dev(q, "q"), _dev(k_cache, "k_cache"), _dev(v_cache, "v_cache"), cap,
            _dev(out, "out"), n_tokens, start_pos, n_heads, n_kv_heads, head_dim,
            _stream(stream)))

    def dev_prefill(self, q, k, v, n_tokens, start_pos, n_heads, n_kv_heads, head_dim, theta,
                    k_cache, v_cache, cap, out, stream=None) -> None:
        _lib.check(self._L.bnr_dev_prefill(
            self._h, _dev(q, "q"), _dev(k, "k"), _dev(v, "v"), n_tokens, start_pos, n_heads,
            n_kv_heads, head_dim, theta, _dev(k_cache, "k_cache"), _dev(v_cache, "v_cache"), cap,
            _dev(out, "out"), _stream(stream)))

    def dev_ternary_gemv_preq(self, weight_packed, weight_scale, activation_q, act_absmax, output,
                              out_features, in_features, stream=None) -> None:
        import torch

        _lib.check(self._L.bnr_dev_ternary_gemv_preq(
            self._h, _dev(weight_packed, "weight_packed", dtype=torch.uint8), weight_scale,
            _dev(activation_q, "activation_q", dtype=torch.int8), act_absmax,
            _dev(output, "output"), out_features, in_features, _stream(stream)))

    def dev_ternary_gemv_preq_group(self, weights, weight_scales, activation_q, act_absmax,
                                    outputs, out_features, in_features, stream=None) -> None:
        """Several ternary GEMVs sharing one activation vector, one launch."""
        import torch

        n = len(weights)
        wp = (ctypes.c_void_p * n)(*[_dev(w, "weight", dtype=torch.uint8).value for w in weights])
        op = (ctypes.c_void_p * n)(*[_dev(o, "output").value for o in outputs])
        sc = (ctypes.c_float * n)(*[float(x) for x in weight_scales])
        mf = (ctypes.c_size_t * n)(*[int(x) for x in out_features])
        _lib.check(self._L.bnr_dev_ternary_gemv_preq_group(
            self._h, n, wp, sc, _dev(activation_q, "activation_q", dtype=torch.int8), act_absmax,
            op, mf, in_features, _stream(stream)))

    def dev_lm_head_matmul_i8(self, hidden, weights_i8, scales, output, vocab_size, hidden_size,
                              stream=None) -> None:
        import torch

        _lib.check(self._L.bnr_dev_lm_head_matmul_i8(
            self._h, _dev(hidden, "hidden"), _dev(weights_i8, "weights_i8", dtype=torch.int8),
            _dev(scales, "scales"), _dev(output, "output"), vocab_size, hidden_size,
            _stream(stream)))

    def dev_ternary_gemv_preq_group_devscale(self, weights, weight_scales, activation_q,
                                             act_absmax, outputs, out_features, in_features,
                                             stream=None) -> None:
        """Grouped ternary GEMV with the activation scale in device memory."""
        import torch

        n = len(weights)
        wp = (ctypes.c_void_p * n)(*[_dev(w, "weight", dtype=torch.uint8).value for w in weights])
        op = (ctypes.c_void_p * n)(*[_dev(o, "output").value for o in outputs])
        sc = (ctypes.c_float * n)(*[float(x) for x in weight_scales])
        mf = (ctypes.c_size_t * n)(*[int(x) for x in out_features])
        _lib.check(self._L.bnr_dev_ternary_gemv_preq_group_devscale(
            self._h, n, wp, sc, _dev(activation_q, "activation_q", dtype=torch.int8),
            _dev(act_absmax, "act_absmax"), op, mf, in_features, _stream(stream)))

    def dev_ternary_gemv_norm_group(self, weights, weight_scales, mode, a, b, gamma, eps, h_out,
                                    outputs, out_features, in_features, stream=None) -> None:
        """Grouped ternary GEMV whose prologue forms x (mode), RMSNorms and
        quantises it: the glue launch folded into the projection."""
        import torch

        n = len(weights)
        wp = (ctypes.c_void_p * n)(*[_dev(w, "weight", dtype=torch.uint8).value for w in weights])
        op = (ctypes.c_void_p * n)(*[_dev(o, "output").value for o in outputs])
        sc = (ctypes.c_float * n)(*[float(x) for x in weight_scales])
        mf = (ctypes.c_size_t * n)(*[int(x) for x in out_features])
        _lib.check(self._L.bnr_dev_ternary_gemv_norm_group(
            self._h, n, wp, sc, int(mode), _dev(a, "a"), _dev(b, "b", True), _dev(gamma, "gamma"),
            eps, _dev(h_out, "h_out", True), op, mf, in_features, _stream(stream)))

    def dev_rms_norm(self, input, weight, eps, output, n, stream=None) -> None:
        _lib.check(self._L.bnr_dev_rms_norm(self._h, _dev(input, "input"), _dev(weight, "weight"),
                                            eps, _dev(output, "output"), n, _stream(stream)))

    def dev_sqrelu_gate(self, gate, up, out, n, stream=None) -> None:
        _lib.check(self._L.bnr_dev_sqrelu_gate(self._h, _dev(gate, "gate"), _dev(up, "up"),
                                               _dev(out, "out"), n, _stream(stream)))

    def dev_residual_add(self, h, delta, n, stream=None) -> None:
        _lib.check(self._L.bnr_dev_residual_add(self._h, _dev(h, "h"), _dev(delta, "delta"), n,
                                                _stream(stream)))

    def dev_absmax_quantize(self, x, q_out, scale_out, n, stream=None) -> None:
        import torch

        _lib.check(self._L.bnr_dev_absmax_quantize(
            self._h, _dev(x, "x"), _dev(q_out, "q_out", dtype=torch.int8),
            _dev(scale_out, "scale_out"), n, _stream(stream)))

    def dev_norm_quant(self, mode, a, b, gamma, eps, n, h_out, q_out, act_absmax,
                       stream=None) -> None:
        """x = a | a + b (-> h_out) | sqrelu(a) * b; RMSNorm with gamma; int8
        absmax quantisation into q_out with act_absmax (device float)."""
        import torch

        _lib.check(self._L.bnr_dev_norm_quant(
            self._h, int(mode), _dev(a, "a"), _dev(b, "b", True), _dev(gamma, "gamma"), eps, n,
            _dev(h_out, "h_out", True), _dev(q_out, "q_out", dtype=torch.int8),
            _dev(act_absmax, "act_absmax"), _stream(stream)))

    def dev_synchronize(self, stream=None) -> None:
        _lib.check(self._L.bnr_dev_synchronize(self._h, _stream(stream)))


class DeviceKVCache:
    """HBM-resident KV cache with KVCache's bookkeeping (bitnet-model/src/lib.rs:
    118-292): per layer, head-major ``[n_kv_heads, max_seq, head_dim]`` K and V
    buffers, per-layer lengths and ``filled_positions``."""

    def __init__(self, n_layers: int, n_kv_heads: int, head_dim: int, max_seq: int,
                 device: str = "cuda"):
        import torch

        self.n_layers, self.n_kv_heads, self.head_dim, self.max_seq = (
            n_layers, n_kv_heads, head_dim, max_seq)
        shape = (n_kv_heads, max_seq, head_dim)
        self.k = [torch.zeros(shape, dtype=torch.float32, device=device) for _ in range(n_layers)]
        self.v = [torch.zeros(shape, dtype=torch.float32, device=device) for _ in range(n_layers)]
        self.layer_lengths = [0] * n_layers
        self.filled_positions = 0

    def check_store(self, layer: int, position: int, n_tokens: int = 1) -> None:
        """store_kv's position rules (lib.rs:209-216) for n_tokens rows from position."""
        last = position + n_tokens - 1
        if last >= self.max_seq:
            raise InvalidShape(f"position < max_seq ({self.max_seq})", f"position = {last}")
        if position > self.layer_lengths[layer]:
            raise InvalidShape(f"position <= layer_len_positions ({self.layer_lengths[layer]})",
                               f"position = {position}")

    def mark_stored(self, layer: int, position: int, n_tokens: int = 1) -> None:
        self.layer_lengths[layer] = max(self.layer_lengths[layer], position + n_tokens)

    def advance(self, n: int = 1) -> None:
        if self.filled_positions + n > self.max_seq:
            raise BackendError("HIP", f"KVCache::advance overflow: filled_positions="
                                      f"{self.filled_positions} max_seq={self.max_seq}")
        self.filled_positions += n

    def clear(self) -> None:
        for t in self.k + self.v:
            t.zero_()
        self.layer_lengths = [0] * self.n_layers
        self.filled_positions = 0

    def __len__(self) -> int:
        return self.filled_positions


class NativeKVCache:
    """The library's backend-owned KV cache (``bnr_kv_cache``): KVCache
    (bitnet-model/src/lib.rs:118-315) with its buffers in HBM, owned and
    bookkept by libbitnet_hip.so -- what a Rust caller binds.  Rows are
    written by :meth:`decode` / :meth:`dev_decode` / :meth:`dev_prefill`,
    which apply store_kv's position rules."""

    def __init__(self, backend: HipBackend, n_layers: int, n_kv_heads: int, head_dim: int,
                 max_seq: int):
        self._be = backend
        self._L = backend._L
        h = ctypes.c_void_p()
        _lib.check(self._L.bnr_kv_cache_create(backend._h, n_layers, n_kv_heads, head_dim,
                                               max_seq, ctypes.byref(h)))
        self._h = h
        self.n_layers, self.n_kv_heads, self.head_dim, self.max_seq = (
            n_layers, n_kv_heads, head_dim, max_seq)

    def close(self) -> None:
        if getattr(self, "_h", None):
            self._L.bnr_kv_cache_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __len__(self) -> int:
        return int(self._L.bnr_kv_cache_len(self._h))

    def advance(self, n: int = 1) -> None:
        _lib.check(self._L.bnr_kv_cache_advance(self._h, n))

    def clear(self) -> None:
        _lib.check(self._L.bnr_kv_cache_clear(self._h))

    def layer_len(self, layer: int) -> int:
        n = ctypes.c_size_t()
        _lib.check(self._L.bnr_kv_cache_layer_len(self._h, layer, ctypes.byref(n)))
        return n.value

    def layer_ptrs(self, layer: int):
        """Device addresses (K, V) of a layer's ``[n_kv, max_seq, head_dim]`` caches."""
        k, v = ctypes.c_void_p(), ctypes.c_void_p()
        _lib.check(self._L.bnr_kv_cache_layer(self._h, layer, ctypes.byref(k), ctypes.byref(v)))
        return k.value, v.value

    def decode(self, layer: int, q: np.ndarray, k: np.ndarray, v: np.ndarray, position: int,
               n_heads: int, theta: float, output: np.ndarray) -> None:
        """rope_embed -> store_kv -> masked_attention for one token of one layer
        from host slices; q and k are rotated in place."""
        _lib.check(self._L.bnr_kv_decode(
            self._be._h, self._h, layer, _host(q, "q"), q.size, _host(k, "k"), k.size,
            _host(v, "v"), v.size, position, n_heads, theta, _host(output, "output"),
            output.size))

    def dev_decode(self, layer: int, q, k, v, position: int, n_heads: int, theta: float, out,
                   stream=None) -> None:
        _lib.check(self._L.bnr_kv_dev_decode(
            self._be._h, self._h, layer, _dev(q, "q"), _dev(k, "k"), _dev(v, "v"), position,
            n_heads, theta, _dev(out, "out"), _stream(stream)))

    def dev_prefill(self, layer: int, q, k, v, n_tokens: int, start_pos: int, n_heads: int,
                    theta: float, out, stream=None) -> None:
        _lib.check(self._L.bnr_kv_dev_prefill(
            self._be._h, self._h, layer, _dev(q, "q"), _dev(k, "k"), _dev(v, "v"), n_tokens,
            start_pos, n_heads, theta, _dev(out, "out"), _stream(stream)))
