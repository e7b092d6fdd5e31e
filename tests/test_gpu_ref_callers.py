"""The reference's own C tests of the hot-path ops and of q_sample_token,
compiled unchanged from the reference's tests/ against this repository's
include/qorus.h and linked to libqorus_hip.so (oracle/Makefile, target
`callers`): the drop-in check of the boundary.  Each program is also linked
to the reference's own library (oracle/_ref), and the two runs must end the
same way: the same exit status and, where the program prints them, the same
counts of passed, failed and crashed cases.  (test_matmul_adversarial fails
24 of its 30 cases against the reference's own library too: its tensors
leave nb[0] = 0, which the GEMV's validation rejects, and it then compares
the untouched, uninitialized output buffer.  Both runs set glibc's
MALLOC_PERTURB_, so such a buffer holds a fixed byte pattern instead of
whatever the heap held before, and the counts do not depend on the two
libraries' heap layouts.)

The binaries are built in the build container, where the reference sources
are; where they were not built the test is skipped.  test_dequantize reads
the reference's fixtures from ./test_data (the copies in tests/golden).
"""
import os
import re
import subprocess
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

REPO = Path(__file__).resolve().parent.parent
CALLERS = REPO / "oracle" / "_ref" / "callers"
CALLERS_REF = REPO / "oracle" / "_ref" / "callers_ref"
NAMES = ["test_matmul", "test_matmul_adversarial", "test_ops", "test_dequantize", "test_dequantize_adversarial",
         "test_matmul_f32", "test_add_f32", "test_mul_f32", "test_rmsnorm_adversarial", "test_rope_adversarial",
         "test_silu_adversarial", "test_softmax_adversarial", "test_causal_mask_f32", "test_main"]


COUNTS = re.compile(r"Tests (Passed|Failed|Crashed):\s+(\d+)")


def run(exe, cwd):
    env = dict(os.environ, MALLOC_PERTURB_="165")
    p = subprocess.run([str(exe)], cwd=cwd, env=env, capture_output=True, text=True, timeout=120)
    out = p.stdout + p.stderr
    return p.returncode, dict(COUNTS.findall(out)), out[-3000:]


@pytest.mark.parametrize("name", NAMES)
def test_reference_caller(tmp_path, name):
    exe, exe_ref = CALLERS / name, CALLERS_REF / name
    if not exe.exists() or not exe_ref.exists():
        pytest.skip("reference callers not built (make -C oracle callers needs the reference sources)")
    os.symlink(REPO / "tests" / "golden", tmp_path / "test_data")
    rc, counts, tail = run(exe, tmp_path)
    rc_ref, counts_ref, tail_ref = run(exe_ref, tmp_path)
    print(f"{name}: hip rc={rc} {counts} | reference rc={rc_ref} {counts_ref}")
    assert rc == rc_ref, f"{name}: exit {rc}, reference library {rc_ref}\n{tail}\n--- reference ---\n{tail_ref}"
    assert counts == counts_ref, (counts, counts_ref)
