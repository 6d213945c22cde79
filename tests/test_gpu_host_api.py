"""The C++ host API (include/nutllm_gpu.hpp) on the GPU: tests/cpp/
host_api_test.cpp runs as a child process and checks the reference's
llama2.c fixture ([1, 0, 3] -> [4, 5] in INT8 and INT4), prefill against
the decode loop, the decode / prefill / generate exceptions and messages,
and the quantised matvec through the C ABI."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
BINARY = os.path.join(HERE, "cpp", "_build", "host_api_test")


def test_cpp_host_api_on_device(gpu):
    assert os.path.exists(BINARY), "build first: make -C tests/cpp"
    print("running", BINARY, flush=True)
    r = subprocess.run([BINARY, os.path.join(HERE, "golden")],
                       capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "all passed" in r.stdout
