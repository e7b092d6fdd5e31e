"""Exhaustive host check of the device polynomial exp (qh_vec.hpp).

exp_approx must equal the oracle's restatement of the reference's
exp_approx (avx_math.h:10-61) on all 2^32 float bit patterns, and the
attention kernels' exp_approx_nonpos must equal exp_approx on every x <= 0
and every NaN (the softmax arguments s - max s they feed it).  The device
helpers are compiled for the host by hipcc (host pass only); the check runs
in a few seconds on the host's cores.
"""
import shutil
import subprocess
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent
ORACLE_LIB = REPO / "oracle" / "build" / "liboracle.so"


@pytest.mark.skipif(shutil.which("hipcc") is None, reason="hipcc not on PATH")
def test_exp_forms_exhaustive(tmp_path):
    assert ORACLE_LIB.exists(), "oracle not built (make -C oracle)"
    exe = tmp_path / "exp_forms_check"
    subprocess.run(["hipcc", "--offload-host-only", "-O2", "-mfma", "-std=c++17", "-ffp-contract=off",
                    "-I", str(REPO / "project-ia_amd" / "csrc"), str(REPO / "tests" / "exp_forms_check.cpp"),
                    "-L", str(ORACLE_LIB.parent), "-loracle", "-Wl,-rpath," + str(ORACLE_LIB.parent),
                    "-lpthread", "-o", str(exe)], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=600)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "0 of 4294967296 differ" in r.stdout
