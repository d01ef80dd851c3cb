"""The dense prefill kernel's host work list (prefill_split_plan in
csrc/kernels/prefill.hip): coverage, piece order and slot numbering over random
chunk sets, checked by a host-only program built with hipcc (no GPU needed)."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


def test_prefill_work_list_invariants(tmp_path):
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(hipcc):
        pytest.skip("hipcc is not available")
    exe = tmp_path / "prefill_plan_check"
    src = os.path.join(HERE, "native", "prefill_plan_check.cpp")
    r = subprocess.run([hipcc, "-O1", "-std=c++17", "--offload-arch=gfx950", "-Xclang", "-target-feature",
                        "-Xclang", "-packed-fp32-ops", src, "-o", str(exe)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout[-2000:]
    # the random set must exercise every schedule
    split = int(r.stdout.split(" of 3000")[0].split()[-1])
    multi = int(r.stdout.split(" run several")[0].split()[-1])
    assert 0 < split < 3000, r.stdout
    assert 0 < multi < 3000 - split, r.stdout
