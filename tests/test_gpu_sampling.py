"""Temperature / top-p sampling (choose_token, src/generate.cpp:31-72) on
the device path against the ids the compiled reference sampled with the
same model, prompt, temperature, top-p and seed (tests/golden/sampled.json):
16 ids identical for each setting; the reference's argument error."""
import json
import os

import numpy as np
import pytest

from nutllm_amd import workloads as W

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module")
def runs():
    with open(os.path.join(GOLDEN, "sampled.json")) as f:
        return json.load(f)


@pytest.mark.parametrize("name", ["tiny_int8", "tinyllama_int4"])
def test_sampled_ids_match_reference(gpu, runs, name):
    model, prompt, _ = W.build_run(name)
    dev = model.to_device()
    try:
        for r in (r for r in runs if r["run"] == name):
            assert r["prompt"] == prompt.tolist()
            ids, stats = dev.generate_sampled(prompt, 16, r["temperature"], r["top_p"],
                                              r["seed"])
            print(f"{name} T={r['temperature']} p={r['top_p']} seed={r['seed']}: "
                  f"{ids[:6]}...", flush=True)
            assert ids == r["ids"], r
            assert stats.generated_tokens == len(ids)
    finally:
        dev.close()


def test_sampling_arguments(gpu):
    model, prompt, _ = W.build_run("tiny_int8")
    dev = model.to_device()
    try:
        with pytest.raises(gpu.InvalidArgument,
                           match="^sampling: invalid temperature or top-p$"):
            dev.generate_sampled(prompt, 4, 1.0, 1.5, 1)
        with pytest.raises(gpu.InvalidArgument,
                           match="^sampling: invalid temperature or top-p$"):
            dev.generate_sampled(prompt, 4, float("inf"), 0.9, 1)
        # temperature 0 is the greedy branch
        greedy, _ = dev.generate(prompt, 8)
        assert dev.generate_sampled(prompt, 8, 0.0, 0.9, 5)[0] == greedy
    finally:
        dev.close()
