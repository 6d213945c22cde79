"""The long-prompt configurations at full size against the reference.

Fixtures tests/golden/tinyllama_int8_2k.npz and llama7b_int4.npz were
written by tests/golden/make_golden.py from the reference's own path
(oracle/_ref: prefill_quantized as per-token decode_quantized_token, then
generate_tokens_cached, src/quant_model.cpp:158-220 and
src/generate.cpp:174-216) over the same seeded weights:

* TinyLlama-shape INT8, 2048-token prompt, 128 greedy tokens at KV lengths
  2048-2175 (token kernel with split attention on the device);
* Llama-2-7B-shape INT4, 512-token prompt, 128 greedy tokens.

The device prefills with the batched MFMA path (bar: rel-L2 2e-3 for the
hidden state and K/V rows) and must reproduce all 128 greedy ids. A
two-layer model at the 7B widths is also checked against the oracle at the
fp32 bar (1e-5) on the step kernels and at 2e-3 on the batched prefill,
and its classifier argmax through the wide kernel's INT8 screen on rows
built to defeat a screen that ignored the fp32 logits or non-finite rows.
"""
import dataclasses
import hashlib
import os

import numpy as np
import pytest

import oracle as O
from nutllm_amd import workloads as W
from screening import screen_twin

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
TOL = 1e-5
PREFILL_TOL = 2e-3


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def weight_digest(model):
    h = hashlib.sha256()
    h.update(model.embeddings.tobytes())
    h.update(model.lm_head.tobytes())
    for mats in model.layers:
        for name in O.PROJECTIONS:
            h.update(mats[name][0].tobytes())
            h.update(mats[name][1].tobytes())
    return h.hexdigest()


@pytest.mark.parametrize("name", ["tinyllama_int8_2k", "llama7b_int4"])
def test_long_run_matches_reference(gpu, name):
    g = np.load(os.path.join(GOLDEN, f"{name}.npz"))
    model, prompt, gen = W.build_run(name)
    assert np.array_equal(prompt, g["prompt"])
    assert weight_digest(model) == str(g["digest"])
    c = model.config
    dev = model.to_device()
    try:
        assert dev.storage_bytes() == int(g["storage_bytes"])
        cache = gpu.KVCache(c)
        h = dev.prefill(cache, prompt)
        err = rel_l2(h, g["hidden"])
        worst = 0.0
        for (l, kvh, p), rk, rv in zip(g["kv_index"], g["keys"], g["values"]):
            k, v = cache.key_value(int(l), int(kvh), int(p))
            worst = max(worst, rel_l2(k, rk), rel_l2(v, rv))
        print(f"{name}: prefill hidden rel-L2 {err:.2e}, K/V rows worst "
              f"{worst:.2e}", flush=True)
        assert err <= PREFILL_TOL and worst <= PREFILL_TOL
        ids, _ = dev.generate(prompt, gen)
        ref = g["ids"].tolist()
        first = next((i for i, (a, b) in enumerate(zip(ids, ref)) if a != b),
                     None)
        print(f"{name}: {len(ids)} ids, first difference at {first}",
              flush=True)
        assert ids == ref
    finally:
        dev.close()


def test_llama7b_widths_two_layers_vs_oracle(gpu):
    """dim 4096, 32 MHA heads of 128, ffn 11008, two layers, non-unit norm
    weights: a 100-token prompt in chunks on the step kernels and three
    decode steps within rel-L2 1e-5 of the oracle (hidden state and K/V
    rows), the batched prefill within 2e-3, and 8 greedy ids identical."""
    O.orc().orc_set_threads(16)
    model = W.build("llama7b_2l", 1, 4, norm_seed=13)
    c = model.config
    prompt = gpu.synth_tokens(7, c.vocab_size, 100)
    om = O.oracle_model(model)
    dev = model.to_device()
    try:
        dev.set_path(1)
        cache = gpu.KVCache(c)
        h = dev.prefill(cache, prompt)
        ho = om.prefill(prompt)
        assert rel_l2(h, ho) <= TOL
        for token in (5, 17, 31000):
            hd, ho = dev.decode(cache, token), om.decode(token)
            assert rel_l2(hd, ho) <= TOL
        pos = len(prompt) + 2
        for layer in range(c.layers):
            for kvh in (0, 13, 31):
                for p in (0, 50, pos):
                    k, v = cache.key_value(layer, kvh, p)
                    rk, rv = om.kv_row(layer, kvh, p)
                    assert rel_l2(k, rk) <= TOL and rel_l2(v, rv) <= TOL
        dev.set_path(0)
        cache = gpu.KVCache(c)
        h = dev.prefill(cache, prompt)
        om.reset()
        ho = om.prefill(prompt)
        err = rel_l2(h, ho)
        print(f"7B widths: batched prefill hidden rel-L2 {err:.2e}", flush=True)
        assert err <= PREFILL_TOL
        for layer in range(c.layers):
            for kvh in (0, 31):
                for p in (0, 99):
                    k, v = cache.key_value(layer, kvh, p)
                    rk, rv = om.kv_row(layer, kvh, p)
                    assert rel_l2(k, rk) <= PREFILL_TOL and rel_l2(v, rv) <= PREFILL_TOL
        ids, _ = dev.generate(prompt, 8)
        ref, _, _ = om.generate(prompt, 8)
        assert ids == ref
    finally:
        dev.set_path(0)
        dev.close()


def test_llama7b_widths_token_kernel_vs_oracle(gpu):
    """The cooperative kernel for wide multi-head shapes (dim 4096, 32 heads
    of 128, ffn 11008, INT4) forced on, against the oracle at rel-L2 1e-5:
    a 12-token prefill through it, then, after a 100-token step-kernel
    prefill, three single-token decodes (hidden state and the new K/V rows
    at several heads and both layers) and 8 greedy ids."""
    O.orc().orc_set_threads(16)
    model = W.build("llama7b_2l", 1, 4, norm_seed=13)
    c = model.config
    om = O.oracle_model(model)
    dev = model.to_device()
    try:
        short = gpu.synth_tokens(11, c.vocab_size, 12)
        dev.set_path(gpu.PATH_TOKEN)
        cache = gpu.KVCache(c)
        h = dev.prefill(cache, short)
        ho = om.prefill(short)
        assert rel_l2(h, ho) <= TOL
        for layer in range(c.layers):
            for kvh in (0, 7, 31):
                for p in (0, 11):
                    k, v = cache.key_value(layer, kvh, p)
                    rk, rv = om.kv_row(layer, kvh, p)
                    assert rel_l2(k, rk) <= TOL and rel_l2(v, rv) <= TOL

        prompt = gpu.synth_tokens(7, c.vocab_size, 100)
        dev.set_path(gpu.PATH_STEPS)
        cache = gpu.KVCache(c)
        dev.prefill(cache, prompt)
        om.reset()
        om.prefill(prompt)
        dev.set_path(gpu.PATH_TOKEN)
        for i, token in enumerate((5, 17, 31000)):
            hd, ho = dev.decode(cache, token), om.decode(token)
            err = rel_l2(hd, ho)
            print(f"token kernel decode {i}: rel-L2 {err:.2e}", flush=True)
            assert err <= TOL
            p = len(prompt) + i
            for layer in range(c.layers):
                for kvh in (0, 13, 31):
                    k, v = cache.key_value(layer, kvh, p)
                    rk, rv = om.kv_row(layer, kvh, p)
                    assert rel_l2(k, rk) <= TOL and rel_l2(v, rv) <= TOL
        ids, _ = dev.generate(prompt, 8)
        om.reset()
        ref, _, _ = om.generate(prompt, 8)
        assert ids == ref
    finally:
        dev.set_path(gpu.PATH_AUTO)
        dev.close()


@pytest.mark.parametrize("case", ["twin-up-next", "twin-down-lower-wg", "nan-top"])
def test_llama7b_widths_screened_argmax(gpu, case):
    """The wide kernel's screened classifier argmax (dim 4096) on rows whose
    INT8 screening copy equals the argmax row's with an fp32 logit about
    0.1 higher (the twin one row later) or lower (the twin 700 rows
    earlier), and on a NaN weight in the argmax row: the greedy ids equal
    the oracle's on the same weights."""
    O.orc().orc_set_threads(16)
    model = W.build("llama7b_2l", 1, 4, norm_seed=13)
    c = model.config
    prompt = gpu.synth_tokens(7, c.vocab_size, 20)
    om = O.oracle_model(model)
    hidden = np.asarray(om.prefill(prompt), np.float64)
    top = int(np.argmax(om.logits(hidden)))
    x = hidden / np.sqrt(np.mean(hidden * hidden) + 1e-5) * model.final_norm
    head = model.lm_head.copy()
    if case == "nan-top":
        assert top != 0  # a NaN at row 0 would be the scan's answer
        head[top, 5] = np.nan
    else:
        up = case == "twin-up-next"
        other = (top + (1 if up else -700)) % c.vocab_size
        head[other] = screen_twin(head[top], x, up)
    dev = model.to_device()
    try:
        dev.set_globals(model.embeddings, model.final_norm, head)
        dev.set_path(gpu.PATH_TOKEN)
        ids, _ = dev.generate(prompt, 4)
        changed = dataclasses.replace(model, lm_head=head)  # layer norms kept
        ref, _, _ = O.oracle_model(changed).generate(prompt, 4)
        assert ids == ref, (ids, ref, top)
        if case == "nan-top":
            assert ids[0] != top
        elif case == "twin-up-next":
            assert ids[0] == (top + 1) % c.vocab_size
        else:
            assert ids[0] == top
    finally:
        dev.set_path(gpu.PATH_AUTO)
        dev.close()
