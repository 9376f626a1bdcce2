"""The prefill work-item order (prefill_map / prefill_order, shared by the
kernels and the host planner's dispatch replay) is a bijection onto the
(query tile, key chunk) pairs, with the chunk counts and partial-state slots
the merge expects, and with non-increasing chunk lengths in the
longest-first order.  A host-only harness is built with hipcc against the
library and run over 2550 shapes (150 launch shapes x 17 chunk sizes, no GPU
needed)."""
import os
import shutil
import subprocess

import pytest

from bitnetrs_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not available")
def test_prefill_item_order(tmp_path):
    _lib.load()  # the library is built
    lib_dir = os.path.dirname(_lib.LIB_PATH)
    exe = tmp_path / "prefill_order_check"
    subprocess.run([HIPCC, "-O1", "-std=c++17", "-I", os.path.join(ROOT, "bitnetrs_amd", "csrc"),
                    "-o", str(exe), os.path.join(ROOT, "tests", "native", "prefill_order_check.cpp"),
                    "-L", lib_dir, "-lbitnet_hip", f"-Wl,-rpath,{lib_dir}"],
                   check=True, capture_output=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0 and out.stdout.startswith("ok"), out.stdout + out.stderr
