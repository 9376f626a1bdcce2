"""The stream-K prefill runs (prefill_streamk_units / sk_seg / sk_u0 /
sk_wg_of, shared by the kernel and the host): every (kv head, query tile,
key tile) unit is taken exactly once, runs are contiguous and equal to
within one unit, a query tile's parts are the runs the merge expects with
distinct partial-state slots.  A host-only harness is built with hipcc
against the library and walks every run of 2058 launches (14 token counts
x 7 start positions x 3 kv-head counts x 7 workgroup counts; no GPU
needed)."""
import os
import shutil
import subprocess

import pytest

from bitnetrs_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not available")
def test_prefill_streamk_runs(tmp_path):
    _lib.load()  # the library is built
    lib_dir = os.path.dirname(_lib.LIB_PATH)
    exe = tmp_path / "prefill_streamk_check"
    subprocess.run([HIPCC, "-O1", "-std=c++17", "-I", os.path.join(ROOT, "bitnetrs_amd", "csrc"),
                    "-o", str(exe), os.path.join(ROOT, "tests", "native", "prefill_streamk_check.cpp"),
                    "-L", lib_dir, "-lbitnet_hip", f"-Wl,-rpath,{lib_dir}"],
                   check=True, capture_output=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0 and out.stdout.startswith("ok"), out.stdout + out.stderr
