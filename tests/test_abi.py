"""The C-ABI library loads (no GPU needed) and exports every function the
public header declares; the ctypes table matches the header."""
import ast
import ctypes
import os
import re
import subprocess

import pytest

import bitnetrs_amd
from bitnetrs_amd import _lib
from common import error_from_parts

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_functions(path=_lib.HEADER):
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(bnr_\w+)\s*\(", text)))


def test_header_declares_entry_points():
    names = header_functions()
    assert "bnr_rope_embed" in names and "bnr_masked_attention" in names
    assert len(names) >= 15


def test_library_exports_every_header_symbol():
    lib = _lib.load()
    missing = [n for n in header_functions() if not hasattr(lib, n)]
    assert not missing, f"not exported: {missing}"


def test_exported_symbols_are_c_linkage():
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    for n in header_functions():
        assert n in exported, f"{n} is not an unmangled exported symbol"


def test_ctypes_table_matches_header():
    assert sorted(_lib.SIGNATURES) == header_functions()


def test_abi_version_and_no_device_error():
    lib = _lib.load()
    assert lib.bnr_abi_version() >> 16 == 1
    try:
        import torch

        has_gpu = torch.cuda.is_available()
    except Exception:
        has_gpu = False
    if has_gpu:
        pytest.skip("a GPU is present")
    with pytest.raises(bitnetrs_amd.UnsupportedDevice) as e:
        bitnetrs_amd.HipBackend(0)
    assert "device" in lib.bnr_last_error().decode()
    assert error_from_parts() == (_lib.BNR_UNSUPPORTED_DEVICE,
                                  "unsupported device: no HIP device available")
    assert e.value.fields == ("no HIP device available",)
    assert str(e.value) == lib.bnr_last_error().decode()


def test_error_parts_rebuild_each_variant_without_gpu():
    """bnr_last_error_parts gives each variant's fields: a binding that builds
    the variant from them prints bnr_last_error()'s text exactly."""
    lib = _lib.load()
    assert lib.bnr_create(0, None) == _lib.BNR_BACKEND_ERROR
    assert error_from_parts() == (_lib.BNR_BACKEND_ERROR,
                                  "backend error (HIP): bnr_create: out is NULL")
    assert lib.bnr_rope_embed(None, None, 0, None, 0, 0, 8, 1, 1, 1e4) == _lib.BNR_BACKEND_ERROR
    kind, text = error_from_parts()
    assert kind == _lib.BNR_BACKEND_ERROR and text.startswith("backend error (HIP): ")
    with pytest.raises(bitnetrs_amd.BackendError) as e:
        _lib.check(lib.bnr_rope_embed(None, None, 0, None, 0, 0, 8, 1, 1, 1e4))
    assert e.value.fields[0] == "HIP" and str(e.value) == text
    # null out-pointers are allowed; the status is still returned
    assert lib.bnr_last_error_parts(None, None) == _lib.BNR_BACKEND_ERROR


def test_null_context_is_an_error_not_a_crash():
    lib = _lib.load()
    assert lib.bnr_masked_attention(None, None, 0, None, 0, None, 0, None, 0, 1, 1, 4, 0) != 0
    assert lib.bnr_rope_embed(None, None, 0, None, 0, 0, 8, 1, 1, 1e4) == _lib.BNR_BACKEND_ERROR
    lib.bnr_destroy(None)


def test_integration_rust_extern_block_matches_header():
    # The Rust extern block of the integration guide at the repository root
    # declares exactly the header's functions.
    text = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    block = text.split("extern \"C\" {", 1)[1].split("\n}\n", 1)[0]
    rust = sorted(set(re.findall(r"fn (bnr_\w+)\s*\(", block)))
    assert rust == header_functions()


def test_one_hip_runtime_after_load():
    """Loading the library in a fresh process leaves one HIP runtime mapped
    (torch's bundled one serves the library too), so torch still sees the GPU
    after the library was loaded first.  No GPU is touched."""
    code = ("import sys; sys.path.insert(0, %r); import bitnetrs_amd; bitnetrs_amd.load(); "
            "print(sorted({l.split()[-1] for l in open('/proc/self/maps') if 'libamdhip64' in l}))"
            % os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
    out = subprocess.run(["python3", "-c", code], capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stderr
    maps = ast.literal_eval(out.stdout.strip().splitlines()[-1])
    assert len(maps) == 1, maps
