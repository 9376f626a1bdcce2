"""The chunked-prefill workspace bound (bnr::prefill_item_budget): every
chunk size the planner picks fits the (kv head, item) pairs the workspace
is sized for on that cache capacity.  A host-only harness is built with
hipcc against the library and run over 816 seeded launches (caches of 96
to 8192 rows, 1 to 8 kv heads; no GPU needed)."""
import os
import shutil
import subprocess

import pytest

from bitnetrs_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not available")
def test_prefill_workspace_budget(tmp_path):
    _lib.load()  # the library is built
    lib_dir = os.path.dirname(_lib.LIB_PATH)
    exe = tmp_path / "prefill_ws_check"
    subprocess.run([HIPCC, "-O1", "-std=c++17", "-I", os.path.join(ROOT, "bitnetrs_amd", "csrc"),
                    "-o", str(exe), os.path.join(ROOT, "tests", "native", "prefill_ws_check.cpp"),
                    "-L", lib_dir, "-lbitnet_hip", f"-Wl,-rpath,{lib_dir}"],
                   check=True, capture_output=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0 and out.stdout.startswith("ok"), out.stdout + out.stderr


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not available")
def test_prefill_paired_plans(tmp_path):
    """Paired 16-query plans (bnr::plan_prefill_pairs) over 1600 seeded
    shapes: key-tile coverage, chunk order, bins of at most two pieces within
    tau, the grid mapping, disjoint partial-state slots within the budget,
    and the stack shape's 51 bins of at most 21 key tiles (host only)."""
    _lib.load()
    lib_dir = os.path.dirname(_lib.LIB_PATH)
    exe = tmp_path / "prefill_pair_check"
    subprocess.run([HIPCC, "-O1", "-std=c++17", "-I", os.path.join(ROOT, "bitnetrs_amd", "csrc"),
                    "-o", str(exe), os.path.join(ROOT, "tests", "native", "prefill_pair_check.cpp"),
                    "-L", lib_dir, "-lbitnet_hip", f"-Wl,-rpath,{lib_dir}"],
                   check=True, capture_output=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0 and out.stdout.startswith("ok"), out.stdout + out.stderr
