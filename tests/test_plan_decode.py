"""The split-K decode planner (bnr::plan_decode): split sizes and counts
consistent with the rows; for the reference merge (default) the smallest
split whose workgroups fit the launch's target; for the forced ticket and
two-launch merges the two-launch merge only where its kernels exist and
small launches at the cheapest split by the planner's time estimate; the
plans of the 2B shape.  A host-only harness is built with hipcc against the
library and run over 10800 seeded launches (no GPU needed)."""
import os
import shutil
import subprocess

import pytest

from bitnetrs_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not available")
def test_decode_plans(tmp_path):
    _lib.load()  # the library is built
    lib_dir = os.path.dirname(_lib.LIB_PATH)
    exe = tmp_path / "plan_decode_check"
    subprocess.run([HIPCC, "-O1", "-std=c++17", "-I", os.path.join(ROOT, "bitnetrs_amd", "csrc"),
                    "-o", str(exe), os.path.join(ROOT, "tests", "native", "plan_decode_check.cpp"),
                    "-L", lib_dir, "-lbitnet_hip", f"-Wl,-rpath,{lib_dir}"],
                   check=True, capture_output=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0 and out.stdout.startswith("ok"), out.stdout + out.stderr
