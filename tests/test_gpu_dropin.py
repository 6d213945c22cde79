"""The reference's own entry points on the device (drop-in adapter): the
llama2.c fixture through the reference's loader and generate_tokens_cached
gives [4, 5]; prefill_quantized / decode_quantized_token hidden states and
the caller's KVCache rows, greedy and sampled generate_tokens_cached ids,
matvec_quantized[_threaded], matvec_threaded and matmul_threaded agree with
the reference's CPU definitions in the same program (rel-L2 1e-5, ids
identical). oracle/_ref/dropin_test is built on the host by
__graft_entry__.build()."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BINARY = os.path.join(ROOT, "oracle", "_ref", "dropin_test")
FIXTURE = os.path.join(ROOT, "tests", "golden", "tiny-llama2.bin")


def test_reference_entry_points_on_device(gpu):
    assert os.path.exists(BINARY), "build() did not produce oracle/_ref/dropin_test"
    r = subprocess.run([BINARY, FIXTURE], capture_output=True, text=True,
                       timeout=300)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "PASS: 0 failure(s)" in r.stdout
