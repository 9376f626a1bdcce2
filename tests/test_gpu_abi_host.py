"""The C ABI driven from a plain C program (tests/native/abi_host_check.c),
with no Python or PyTorch in that process, as a Rust backend crate's extern
"C" block would drive it: the reference's per-token rope_embed -> store_kv
-> masked_attention sequence (bitnet-model/src/lib.rs:1004-1036) on host
slices for 48 tokens of the 2B shape, against the oracle's CpuBackend (rotated
q/k bit for bit, outputs within tolerance), plus an error case of each entry
point.  The program is built by __graft_entry__.build() (tests/native/
Makefile)."""
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EXE = os.path.join(ROOT, "tests", "native", "abi_host_check")


def test_plain_c_host_matches_oracle():
    print("[gpu case] plain C host program: rope_embed + masked_attention, 48 tokens", flush=True)
    sys.stdout.flush()
    assert os.path.exists(EXE), f"{EXE} is missing: run __graft_entry__.build() first"
    out = subprocess.run([EXE], capture_output=True, text=True, timeout=100)
    assert out.returncode == 0 and out.stdout.startswith("ok 48 "), out.stdout + out.stderr
