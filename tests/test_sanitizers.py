"""The host library (GGUF reader, config reader, synthetic writer) and the
oracle built with AddressSanitizer + UndefinedBehaviorSanitizer, with the CPU
tests that drive them (ABI, oracle against the reference's fixtures, damaged
GGUF images) run on those builds in a child process.  Any invalid access or
undefined behaviour aborts the child."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def gcc_runtime(name):
    r = subprocess.run(["gcc", f"-print-file-name={name}"], capture_output=True, text=True)
    path = r.stdout.strip()
    return path if os.path.isabs(path) and os.path.exists(path) else None


@pytest.mark.skipif(gcc_runtime("libasan.so") is None, reason="gcc's AddressSanitizer runtime is not installed")
def test_host_and_oracle_tests_clean_under_asan_ubsan(tmp_path):
    for d, sub in (("forword.c_amd", "host"), ("oracle", "oracle")):
        out = tmp_path / sub
        r = subprocess.run(["make", "-s", "-C", os.path.join(ROOT, d), "san", f"SAN_DIR={out}"],
                           capture_output=True, text=True)
        assert r.returncode == 0, r.stderr
    env = dict(os.environ)
    env.update(LD_PRELOAD=gcc_runtime("libasan.so"), ASAN_OPTIONS="detect_leaks=0:abort_on_error=1",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1",
               FW_HOST_LIB=str(tmp_path / "host" / "libfw_host.so"),
               FW_CPU_LIB=str(tmp_path / "oracle" / "libfwcpu.so"))
    tests = [os.path.join(ROOT, "tests", t) for t in ("test_abi.py", "test_oracle.py", "test_gguf_corrupt.py")]
    r = subprocess.run([sys.executable, "-m", "pytest", "-x", "-q", "-m", "not gpu", "-p", "no:cacheprovider"] + tests,
                       capture_output=True, text=True, env=env, cwd=ROOT, timeout=900)
    tail = (r.stdout + r.stderr)[-3000:]
    assert r.returncode == 0, tail
    assert "ERROR: AddressSanitizer" not in r.stderr and "runtime error:" not in r.stderr, tail
