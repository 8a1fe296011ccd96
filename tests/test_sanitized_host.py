"""The C ABI's host code under AddressSanitizer and UndefinedBehaviorSanitizer.

Opt-in (AITER_AMD_SANITIZE=1; it builds a second library, about a minute):
builds aiter_amd/_build_san/libaiter_amd_san.so with host-only sanitizers
and runs the CPU ABI tests (argument checks, workspace layouts, the
reference-shaped ctypes entry points, error strings) in a child process that
loads it with clang's ASan runtime preloaded. Any sanitizer report fails the
child, and so the test."""
import os
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent


@pytest.mark.skipif(os.environ.get("AITER_AMD_SANITIZE") != "1",
                    reason="opt-in: AITER_AMD_SANITIZE=1 builds the sanitized library")
def test_abi_host_code_under_sanitizers():
    from aiter_amd import build as B

    lib = B.build_sanitized(verbose=False)
    env = dict(os.environ)
    env.update(ASAN_OPTIONS="detect_leaks=0:halt_on_error=1",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1",
               LD_PRELOAD=str(B.sanitizer_runtime()), AITER_AMD_LIB=str(lib))
    env.pop("AITER_AMD_SANITIZE", None)
    res = subprocess.run([sys.executable, "-m", "pytest", "-q", "-x", "-m", "not gpu",
                          "tests/test_abi_cpu.py"], cwd=ROOT, env=env, capture_output=True,
                         text=True, timeout=900)
    tail = (res.stdout + res.stderr)[-4000:]
    assert res.returncode == 0, tail
    assert "ERROR: AddressSanitizer" not in tail and "runtime error" not in tail, tail
