"""The drop-in adapter (nutllm_amd/adapter/reference_dropin.cpp) compiled
against the reference's own headers, linked with the reference's sources
(their CPU definitions of the replaced functions renamed to cpu_*) and
libnutllm_hip.so into oracle/_ref/dropin_test by oracle/Makefile.

Without a GPU: the reference's argument checks raise the reference's
exception types and messages before any device work, and a call that needs
the device raises std::runtime_error (no CPU fallback).
"""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BINARY = os.path.join(ROOT, "oracle", "_ref", "dropin_test")
FIXTURE = os.path.join(ROOT, "tests", "golden", "tiny-llama2.bin")


@pytest.mark.skipif(not os.path.exists(BINARY) and
                    not os.path.isdir("/root/reference/src"),
                    reason="needs the reference sources to build")
def test_dropin_builds_against_reference_headers():
    if os.path.isdir("/root/reference/src"):
        subprocess.run(["make", "-C", os.path.join(ROOT, "oracle"), "dropin"],
                       check=True, capture_output=True)
    assert os.path.exists(BINARY)
    r = subprocess.run([BINARY, FIXTURE, "--no-device"], capture_output=True,
                       text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "PASS" in r.stdout
