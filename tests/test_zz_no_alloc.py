"""nut_decode_noalloc against nut_decode (the existing entry point) on the
same model: the same step kernels, with the split-attention partials and
counters in the library's per-device scratch array instead of model-owned
allocations. Bar: rel-L2 <= 1e-5 on the hidden state and K/V rows (the
fp32 bar of decode_quantized_token, src/quant_model.cpp:158-206); the two
paths run the same arithmetic, so they are expected to agree bit for bit.

Two calls in a row, the second with a smaller input (a shorter context,
then a smaller model), so the second call finds the first call's scratch
contents; every call leaves the library's count of device allocations
(nut_device_allocations) unchanged; plus the limits: bad tokens fail as
nut_decode does, a model the step kernels cannot run is rejected.
"""
import numpy as np
import pytest

from nutllm_amd import workloads as W

pytestmark = pytest.mark.gpu

TOL = 1e-5


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def run_pair(gpu, dev, c, prompt, tokens, out):
    """Prefill two caches the same way, then decode `tokens` on one with
    nut_decode and on the other with nut_decode_noalloc."""
    dev.set_path(1)
    ca, cb = gpu.KVCache(c), gpu.KVCache(c)
    dev.prefill(ca, prompt)
    dev.prefill(cb, prompt)
    for i, token in enumerate(tokens):
        ha = dev.decode(ca, token)
        before = gpu.device_allocations()
        dev.decode_noalloc(cb, token, out)
        made = gpu.device_allocations() - before
        print(f"nut_decode_noalloc made {made} device allocations", flush=True)
        assert made == 0
        hb = out.download(np.float32, c.dim)
        err = rel_l2(hb, ha)
        print(f"context {len(prompt) + i}: hidden rel-L2 {err:.2e}, "
              f"bitwise {np.array_equal(ha, hb)}", flush=True)
        assert err <= TOL
        assert cb.length() == ca.length() == len(prompt) + i + 1
        pos = len(prompt) + i
        for layer in (0, c.layers - 1):
            for kvh in range(c.kv_heads):
                ka, va = ca.key_value(layer, kvh, pos)
                kb, vb = cb.key_value(layer, kvh, pos)
                assert rel_l2(kb, ka) <= TOL and rel_l2(vb, va) <= TOL
    ca.close(), cb.close()


def test_decode_noalloc_matches_decode(gpu):
    model = W.build("tinyllama", 1, 3, 1024)
    c = model.config
    dev = model.to_device()
    out = gpu.DeviceArray(4 * c.dim)
    try:
        # first call at a 700-token context (every split in use), then a
        # smaller input: a 3-token context
        run_pair(gpu, dev, c, gpu.synth_tokens(5, c.vocab_size, 700), [7, 123], out)
        run_pair(gpu, dev, c, gpu.synth_tokens(6, c.vocab_size, 3), [9, 31999], out)
        # errors as nut_decode raises them, before any work
        cache = gpu.KVCache(c)
        with pytest.raises(gpu.OutOfRange, match="token out of range"):
            dev.decode_noalloc(cache, c.vocab_size, out)
        cache.set_length(c.max_seq)
        with pytest.raises(gpu.LengthError, match="context is full"):
            dev.decode_noalloc(cache, 0, out)
        cache.close()
    finally:
        out.close()
        dev.set_path(0)
        dev.close()
    # a smaller model on the same scratch array
    small = W.build("step_gqa2", 0, 6)
    sc = small.config
    dev = small.to_device()
    out = gpu.DeviceArray(4 * sc.dim)
    try:
        run_pair(gpu, dev, sc, gpu.synth_tokens(8, sc.vocab_size, 40), [3, 4], out)
    finally:
        out.close()
        dev.set_path(0)
        dev.close()


def test_decode_noalloc_rejects_models_off_the_step_kernels(gpu):
    """The tiny model (head_dim 16) has no step-kernel instantiation."""
    model = W.build("tiny", 0, 0)
    dev = model.to_device()
    cache = gpu.KVCache(model.config)
    try:
        with pytest.raises(gpu.InvalidArgument, match="no-alloc decode"):
            dev.decode_noalloc(cache, 1, None)
    finally:
        cache.close()
        dev.close()
