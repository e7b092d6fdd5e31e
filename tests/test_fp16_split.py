"""Exhaustive host check of the fp16 hi/lo split of the prefill's matrix-core
operands (tests/fp16_split_check.cpp): for a row scaled so its maximum lies
in [2^14, 2^15), hi = rn16(x) and lo = rn16(x - hi) hold every element of
[2^-3, 2^15) to within 2^-22 of itself (22 significant bits) and smaller
ones to within 2^-25; all floats of [0, 2^15) checked."""
import shutil
import subprocess
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent


@pytest.mark.skipif(shutil.which("hipcc") is None, reason="hipcc not on PATH")
def test_fp16_split_exhaustive(tmp_path):
    exe = tmp_path / "fp16_split_check"
    subprocess.run(["hipcc", "--offload-host-only", "-O2", "-std=c++17", "-ffp-contract=off",
                    str(REPO / "tests" / "fp16_split_check.cpp"), "-lpthread", "-o", str(exe)], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=600)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
