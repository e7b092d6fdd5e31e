"""Host check of the GEMV's second-digit-level rule (qh_digits.hpp).

The rule's functions are compiled for the host by hipcc (host pass only)
and applied to blocks quantized as the device quantizes them; the checker
(tests/digits_rule_check.cpp) asserts the documented properties: N(0,1)
blocks never take level 2, 1..6 outliers of 1e3..1e5 always do, a block
left on level 1 keeps 3 * (max >> 6) outside any 6 of its elements, and a
level-2 block holds every element within 2^21 of its maximum exactly.
"""
import shutil
import subprocess
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent


@pytest.mark.skipif(shutil.which("hipcc") is None, reason="hipcc not on PATH")
def test_digits_rule_properties(tmp_path):
    exe = tmp_path / "digits_rule_check"
    subprocess.run(["hipcc", "--offload-host-only", "-O2", "-std=c++17", "-ffp-contract=off",
                    "-I", str(REPO / "project-ia_amd" / "csrc"), str(REPO / "tests" / "digits_rule_check.cpp"),
                    "-o", str(exe)], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=600)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
