"""The fp32 model path on the GPU against the reference's own outputs
(tests/golden/fp32_*.npz, written by the compiled reference's
prefill_tokens / decode_token, src/kvcache.cpp:237-284, on the same seeded
[in x out] weights with non-unit norm weights): every prefill row, every
decode step's hidden state and the K/V cache within rel-L2 1e-5; the
reference's errors for bad input."""
import os

import numpy as np
import pytest

from nutllm_amd import workloads as W

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
TOL = 1e-5


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


@pytest.mark.parametrize("shape,tied", [("tiny", False), ("tiny", True), ("step_gqa2", False)],
                         ids=["tiny", "tiny-tied", "dim256"])
def test_fp32_path_matches_reference(gpu, shape, tied):
    g = np.load(os.path.join(GOLDEN, f"fp32_{shape}{'_tied' if tied else ''}.npz"))
    seed = int(g["seed"])
    model = W.build_fp32(shape, seed, max_seq=64, norm_seed=seed + 100, tied=tied)
    c = model.config
    dev = model.to_device()
    cache = gpu.KVCache(c)
    try:
        rows = dev.prefill(cache, g["prompt"])
        errs = [rel_l2(rows[i], g["rows"][i]) for i in range(len(g["prompt"]))]
        print(f"{shape}: prefill rows rel-L2 max {max(errs):.2e}", flush=True)
        assert max(errs) <= TOL
        for i, token in enumerate(g["tokens"]):
            err = rel_l2(dev.decode(cache, int(token)), g["hidden"][i])
            assert err <= TOL, (i, err)
        n = len(g["prompt"]) + len(g["tokens"])
        assert cache.length() == n
        k, v = cache.read_positions(0, n)
        kvh = c.kv_heads or c.heads
        ref_k = g["keys"].reshape(c.layers, kvh, c.max_seq, c.head_dim)[:, :, :n]
        ref_v = g["values"].reshape(c.layers, kvh, c.max_seq, c.head_dim)[:, :, :n]
        assert rel_l2(k, ref_k) <= TOL and rel_l2(v, ref_v) <= TOL
    finally:
        cache.close()
        dev.close()


def test_fp32_path_errors(gpu):
    model = W.build_fp32("tiny", 21, max_seq=64)
    c = model.config
    dev = model.to_device()
    cache = gpu.KVCache(c)
    try:
        with pytest.raises(gpu.OutOfRange, match="^kv cache: token id out of range$"):
            dev.decode(cache, c.vocab_size)
        with pytest.raises(gpu.InvalidArgument, match="^kv cache: invalid prefill length$"):
            dev.prefill(cache, np.zeros(0, np.int32))
        # a bad id anywhere in the prompt fails before any layer runs
        with pytest.raises(gpu.OutOfRange, match="^kv cache: token id out of range$"):
            dev.prefill(cache, np.array([3, 4, -1], np.int32))
        assert cache.length() == 0
        cache.set_length(c.max_seq)
        with pytest.raises(gpu.LengthError, match="^kv cache: context is full$"):
            dev.decode(cache, 0)
        other = gpu.KVCache(W.make_config("tiny", max_seq=32))
        with pytest.raises(gpu.InvalidArgument, match="^kv cache: model configuration mismatch$"):
            dev.decode(other, 0)
        other.close()
    finally:
        cache.close()
        dev.close()
