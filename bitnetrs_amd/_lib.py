"""ctypes binding of ``libbitnet_hip.so`` (declarations: ``include/bitnet_hip.h``).

The library is built in-tree by ``bitnetrs_amd/csrc/Makefile`` (see
``bitnetrs_amd.build``).  Loading fails loudly when it is missing: there is
no CPU fallback anywhere in this package.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG_DIR, "libbitnet_hip.so")
CSRC = os.path.join(PKG_DIR, "csrc")
HEADER = os.path.join(os.path.dirname(PKG_DIR), "include", "bitnet_hip.h")

BNR_OK = 0
BNR_INVALID_SHAPE = 1
BNR_INVALID_CONFIG = 2
BNR_BACKEND_ERROR = 3
BNR_UNSUPPORTED_DEVICE = 4
BNR_QUANTIZATION_ERROR = 5

BNR_MIRROR_INCREMENTAL = 0
BNR_MIRROR_FULL = 1

BNR_GLUE_PLAIN = 0
BNR_GLUE_RESIDUAL = 1
BNR_GLUE_SQRELU = 2


class BitNetError(Exception):
    """Mirror of bitnet_core::error::BitNetError (bitnet-core/src/error.rs:12-55).

    ``fields`` holds the variant's own fields as the library reports them
    (``bnr_last_error_parts``); ``str()`` is the variant's Display text,
    rebuilt from them.
    """

    kind = -1
    FORMAT = "{0}"

    def __init__(self, *fields: str):
        self.fields = fields
        super().__init__(self.FORMAT.format(*fields))


class InvalidShape(BitNetError):
    kind = BNR_INVALID_SHAPE
    FORMAT = "invalid tensor shape: expected {0}, got {1}"

    @property
    def expected(self) -> str:
        return self.fields[0]

    @property
    def got(self) -> str:
        return self.fields[1]


class InvalidConfig(BitNetError):
    kind = BNR_INVALID_CONFIG
    FORMAT = "invalid model configuration: {0}"


class BackendError(BitNetError):
    kind = BNR_BACKEND_ERROR
    FORMAT = "backend error ({0}): {1}"


class UnsupportedDevice(BitNetError):
    kind = BNR_UNSUPPORTED_DEVICE
    FORMAT = "unsupported device: {0}"


class QuantizationError(BitNetError):
    kind = BNR_QUANTIZATION_ERROR
    FORMAT = "quantization error: {0}"


ERRORS = {
    BNR_INVALID_SHAPE: InvalidShape,
    BNR_INVALID_CONFIG: InvalidConfig,
    BNR_BACKEND_ERROR: BackendError,
    BNR_UNSUPPORTED_DEVICE: UnsupportedDevice,
    BNR_QUANTIZATION_ERROR: QuantizationError,
}


def build(verbose: bool = False) -> str:
    """Compile libbitnet_hip.so for gfx950 with hipcc (works without a GPU)."""
    out = None if verbose else subprocess.DEVNULL
    subprocess.run(["make", "-B", "-s", "-C", CSRC], check=True, stdout=out)
    return LIB_PATH


_c = ctypes
_f = _c.POINTER(_c.c_float)
_sz = _c.c_size_t
_vp = _c.c_void_p
_i32p = _c.POINTER(_c.c_int32)

# name -> (restype, argtypes); one entry per function in include/bitnet_hip.h
SIGNATURES = {
    "bnr_last_error": (_c.c_char_p, []),
    "bnr_last_error_parts": (_c.c_int, [_c.POINTER(_c.c_char_p), _c.POINTER(_c.c_char_p)]),
    "bnr_abi_version": (_c.c_uint32, []),
    "bnr_create": (_c.c_int, [_c.c_int, _c.POINTER(_vp)]),
    "bnr_destroy": (None, [_vp]),
    "bnr_device_name": (_c.c_char_p, [_vp]),
    "bnr_rope_embed": (_c.c_int, [_vp, _f, _sz, _f, _sz, _sz, _sz, _sz, _sz, _c.c_float]),
    "bnr_masked_attention": (_c.c_int, [_vp, _f, _sz, _f, _sz, _f, _sz, _f, _sz, _sz, _sz, _sz,
                                        _sz]),
    "bnr_set_mirror_mode": (_c.c_int, [_vp, _c.c_int]),
    "bnr_set_deterministic": (_c.c_int, [_vp, _c.c_int]),
    "bnr_mirror_invalidate": (_c.c_int, [_vp]),
    "bnr_dev_rope_append": (_c.c_int, [_vp, _vp, _vp, _vp, _sz, _sz, _sz, _sz, _sz, _c.c_float,
                                       _vp, _vp, _sz, _vp]),
    "bnr_dev_decode_attention": (_c.c_int, [_vp, _vp, _vp, _vp, _sz, _vp, _sz, _sz, _sz, _sz,
                                            _vp]),
    "bnr_dev_stream_read": (_c.c_int, [_vp, _vp, _sz, _vp, _sz, _vp]),
    "bnr_dev_stream_read_shape": (_c.c_int, [_vp, _vp, _sz, _vp, _sz, _c.c_int, _c.c_int,
                                             _c.c_int, _vp]),
    "bnr_dev_decode_attention_noalloc": (_c.c_int, [_vp, _vp, _vp, _vp, _sz, _vp, _sz, _sz, _sz,
                                                    _sz, _vp]),
    "bnr_dev_decode_step": (_c.c_int, [_vp, _vp, _vp, _vp, _sz, _sz, _sz, _sz, _c.c_float, _vp,
                                       _vp, _sz, _vp, _vp, _vp, _vp]),
    "bnr_dev_decode_step_batched": (_c.c_int, [_vp, _vp, _vp, _vp, _i32p, _sz, _sz, _sz, _sz,
                                               _c.c_float, _vp, _vp, _sz, _vp, _vp]),
    "bnr_dev_prefill_attention": (_c.c_int, [_vp, _vp, _vp, _vp, _sz, _vp, _sz, _sz, _sz, _sz,
                                             _sz, _vp]),
    "bnr_dev_prefill": (_c.c_int, [_vp, _vp, _vp, _vp, _sz, _sz, _sz, _sz, _sz, _c.c_float, _vp,
                                   _vp, _sz, _vp, _vp]),
    "bnr_ternary_gemv_preq": (_c.c_int, [_vp, _vp, _sz, _c.c_float, _vp, _sz, _c.c_float, _f,
                                         _sz, _sz, _sz]),
    "bnr_dev_ternary_gemv_preq": (_c.c_int, [_vp, _vp, _c.c_float, _vp, _c.c_float, _vp, _sz,
                                             _sz, _vp]),
    "bnr_dev_ternary_gemv_preq_group": (_c.c_int, [_vp, _sz, _c.POINTER(_vp), _f, _vp,
                                                   _c.c_float, _c.POINTER(_vp),
                                                   _c.POINTER(_sz), _sz, _vp]),
    "bnr_lm_head_matmul_i8_into": (_c.c_int, [_vp, _f, _sz, _vp, _sz, _f, _sz, _f, _sz, _sz,
                                              _sz]),
    "bnr_dev_lm_head_matmul_i8": (_c.c_int, [_vp, _vp, _vp, _vp, _vp, _sz, _sz, _vp]),
    "bnr_dev_ternary_gemv_preq_group_devscale": (_c.c_int, [_vp, _sz, _c.POINTER(_vp), _f, _vp,
                                                            _vp, _c.POINTER(_vp),
                                                            _c.POINTER(_sz), _sz, _vp]),
    "bnr_rms_norm": (_c.c_int, [_vp, _f, _sz, _f, _sz, _c.c_float, _f, _sz]),
    "bnr_sqrelu_gate": (_c.c_int, [_vp, _f, _sz, _f, _sz, _f, _sz]),
    "bnr_dev_rms_norm": (_c.c_int, [_vp, _vp, _vp, _c.c_float, _vp, _sz, _vp]),
    "bnr_dev_sqrelu_gate": (_c.c_int, [_vp, _vp, _vp, _vp, _sz, _vp]),
    "bnr_dev_residual_add": (_c.c_int, [_vp, _vp, _vp, _sz, _vp]),
    "bnr_dev_absmax_quantize": (_c.c_int, [_vp, _vp, _vp, _vp, _sz, _vp]),
    "bnr_dev_norm_quant": (_c.c_int, [_vp, _c.c_int, _vp, _vp, _vp, _c.c_float, _sz, _vp, _vp,
                                      _vp, _vp]),
    "bnr_dev_ternary_gemv_norm_group": (_c.c_int, [_vp, _sz, _c.POINTER(_vp), _f, _c.c_int, _vp,
                                                   _vp, _vp, _c.c_float, _vp, _c.POINTER(_vp),
                                                   _c.POINTER(_sz), _sz, _vp]),
    "bnr_dev_synchronize": (_c.c_int, [_vp, _vp]),
    "bnr_kv_cache_create": (_c.c_int, [_vp, _sz, _sz, _sz, _sz, _c.POINTER(_vp)]),
    "bnr_kv_cache_destroy": (None, [_vp]),
    "bnr_kv_cache_clear": (_c.c_int, [_vp]),
    "bnr_kv_cache_advance": (_c.c_int, [_vp, _sz]),
    "bnr_kv_cache_len": (_sz, [_vp]),
    "bnr_kv_cache_layer_len": (_c.c_int, [_vp, _sz, _c.POINTER(_sz)]),
    "bnr_kv_cache_layer": (_c.c_int, [_vp, _sz, _c.POINTER(_vp), _c.POINTER(_vp)]),
    "bnr_kv_decode": (_c.c_int, [_vp, _vp, _sz, _f, _sz, _f, _sz, _f, _sz, _sz, _sz, _c.c_float,
                                 _f, _sz]),
    "bnr_kv_dev_decode": (_c.c_int, [_vp, _vp, _sz, _vp, _vp, _vp, _sz, _sz, _c.c_float, _vp,
                                     _vp]),
    "bnr_kv_dev_prefill": (_c.c_int, [_vp, _vp, _sz, _vp, _vp, _vp, _sz, _sz, _sz, _c.c_float,
                                      _vp, _vp]),
}

_lib = None


def load() -> ctypes.CDLL:
    """Load the in-tree library (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `make -C {CSRC}` "
                "(or __graft_entry__.build()); there is no fallback path")
        # PyTorch wheels bundle their own HIP runtime, which the dynamic
        # loader also hands to this library (libamdhip64.so.7) when torch is
        # loaded first: one runtime then serves tensors and library calls.
        # Loaded the other way round, the process holds two runtimes and
        # torch finds no GPU.  So torch, when installed, goes first.
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


# Fields each variant takes from bnr_last_error_parts (first, second).
_N_FIELDS = {BNR_INVALID_SHAPE: 2, BNR_BACKEND_ERROR: 2}


def last_error() -> BitNetError:
    """The calling thread's last error, rebuilt from its fields."""
    lib = load()
    first, second = _c.c_char_p(), _c.c_char_p()
    kind = lib.bnr_last_error_parts(_c.byref(first), _c.byref(second))
    parts = [(first.value or b"").decode(), (second.value or b"").decode()]
    cls = ERRORS.get(kind)
    if cls is None:
        return BitNetError(lib.bnr_last_error().decode())
    return cls(*parts[:_N_FIELDS.get(kind, 1)])


def check(status: int) -> None:
    """Raise the BitNetError subclass for a non-zero status."""
    if status != BNR_OK:
        err = last_error()
        if err.kind != status:  # cannot happen: the library records every failure
            raise BitNetError(f"status {status} with last error {err!s}")
        raise err
