"""The C++ host API (include/nutllm_gpu.hpp) without a GPU: the host-side
checks of tests/cpp/host_api_test.cpp (quantiser KATs, storage formula,
error types and messages, config validation)."""
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
BINARY = os.path.join(HERE, "cpp", "_build", "host_api_test")


def test_cpp_host_api_cpu_checks():
    assert os.path.exists(BINARY), "build first: make -C tests/cpp"
    r = subprocess.run([BINARY, os.path.join(HERE, "golden"), "--cpu-only"],
                       capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "all passed" in r.stdout
