"""ThreadSanitizer run of the host runtime (CPU, no GPU needed).

tests/tsan/Makefile builds runtime.hip's host code with -fsanitize=thread and
links the stress driver tests/tsan/registry_stress.cpp: 8 threads create and
free tensors, wrap one buffer from every thread at once, wrap library tensors'
data and free wrapper and owner in both orders, flip their own precision mode
and read their own errors.  Every check in the driver must hold and
ThreadSanitizer must report nothing (a planted race in the registry lock is
reported by this same build).
"""
import os
import shutil
import subprocess

import pytest

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "tsan")


def test_runtime_registry_under_tsan():
    if not os.path.exists("/opt/rocm/llvm/bin/clang++") or shutil.which("make") is None:
        pytest.skip("needs the ROCm clang toolchain and make")
    b = subprocess.run(["make", "-s", "-C", HERE], capture_output=True, text=True, timeout=600)
    assert b.returncode == 0, b.stderr[-3000:]
    env = dict(os.environ, TSAN_OPTIONS="halt_on_error=0 exitcode=66")
    r = subprocess.run([os.path.join(HERE, "_build", "registry_stress")], capture_output=True, text=True,
                       timeout=300, env=env)
    assert "ThreadSanitizer" not in r.stderr, r.stderr[-4000:]
    assert r.returncode == 0 and "0 failed checks" in r.stdout, (r.returncode, r.stdout, r.stderr[-2000:])
