"""The product's host code under sanitizers (no GPU): the threaded block
quantiser, the synthetic generator and the fp16 scale codec, driven from
several caller threads at once (tests/cpp/host_sanitize.cpp), built with
ThreadSanitizer and with AddressSanitizer + UndefinedBehaviorSanitizer by
tests/cpp/Makefile (`make -C tests/cpp sanitize`, run by build())."""
import os
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.parametrize("kind", ["tsan", "asan"])
def test_host_code_clean_under_sanitizer(kind):
    binary = os.path.join(HERE, "cpp", "_build", f"host_sanitize_{kind}")
    assert os.path.exists(binary), "build first: make -C tests/cpp sanitize"
    env = dict(os.environ)
    env["TSAN_OPTIONS"] = "halt_on_error=1"
    env["ASAN_OPTIONS"] = "detect_leaks=1:halt_on_error=1"
    r = subprocess.run([binary], capture_output=True, text=True, timeout=300, env=env)
    out = r.stdout + r.stderr
    assert r.returncode == 0, out
    assert "all passed" in r.stdout
    assert "Sanitizer" not in out, out
