"""The library's host code under AddressSanitizer + UndefinedBehaviorSanitizer.

`make -C project-ia_amd asan` builds build/asan/libqorus_hip.so: the same
sources with every host-side translation unit instrumented (`-Xarch_host
-fsanitize=address,undefined`, aborting on the first report; device code as
in the main build).  The CPU tests of the other files (C-API validation
order and codes, the tokenizer, the model-file loader, the sampler's host
checks, ...) then run in a child process against that build, with the
sanitizer runtime preloaded into Python: any heap/stack overflow,
use-after-free or undefined behaviour on those paths aborts the child.
This is the counterpart of the reference's Release + DEBUG (ASan + UBSan)
matrix of its op tests (its Makefile, target test-validation).
"""
import os
import subprocess
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent
PKG = REPO / "project-ia_amd"
CLANG = Path("/opt/rocm/llvm/bin/clang++")


def asan_runtime():
    if not CLANG.exists():
        return None
    p = subprocess.run([str(CLANG), "-print-file-name=libclang_rt.asan-x86_64.so"], capture_output=True, text=True)
    rt = Path(p.stdout.strip())
    return rt if rt.is_absolute() and rt.exists() else None


def test_cpu_suite_under_host_sanitizers():
    rt = asan_runtime()
    if rt is None:
        pytest.skip("no clang AddressSanitizer runtime in this image")
    b = subprocess.run(["make", "-C", str(PKG), "-j8", "asan"], capture_output=True, text=True, timeout=900)
    assert b.returncode == 0, b.stdout[-3000:] + b.stderr[-3000:]
    lib = PKG / "build" / "asan" / "libqorus_hip.so"
    assert lib.exists()
    env = dict(os.environ, QORUS_HIP_LIB=str(lib), LD_PRELOAD=str(rt),
               ASAN_OPTIONS="detect_leaks=0:abort_on_error=1",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    r = subprocess.run([sys.executable, "-m", "pytest", str(REPO / "tests"), "-x", "-q", "-m", "not gpu",
                        "-p", "no:cacheprovider", "--ignore", __file__],
                       cwd=REPO, env=env, capture_output=True, text=True, timeout=900)
    tail = (r.stdout + r.stderr)[-6000:]
    print(tail)
    assert r.returncode == 0, tail
    assert "AddressSanitizer" not in r.stdout + r.stderr and "runtime error" not in r.stdout + r.stderr, tail
