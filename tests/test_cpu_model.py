"""The oracle's token loop on the CPU, pinned against the reference.

* tiny synthetic model (INT8 and INT4): greedy ids, every decode step's
  hidden state, the final-step logits and the KV cache, bit for bit, against
  vectors the reference wrote (tests/golden/tiny_*.npz), with unit norm
  weights and with seeded non-unit ones (tests/golden/tiny_norms_*.npz);
* TinyLlama-shape INT4 (5-token prompt, 16 tokens): greedy ids against the
  reference's (tests/golden/tinyllama_int4.json);
* the reference's llama2.c fixture (tests/fixtures/tiny-llama2.bin, copied
  to tests/golden/): prompt [1, 0, 3] generates [4, 5] in INT8 and INT4
  (src/loader_selftest.cpp, file lines 81-116);
* the hand fixtures of src/selftest.cpp:85-151 (rmsnorm, RoPE at position
  1, residual), first-index argmax ties (src/generate.cpp:24-30) and
  ModelConfig::validate (src/attention.cpp:15-27).
"""
from __future__ import annotations

import ctypes as C
import json
import math
import os

import numpy as np
import pytest

import llama2c
import nutllm_amd as nut
import oracle
from nutllm_amd import workloads as W

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
INT8, INT4 = 0, 1


def digest(model):
    import hashlib
    h = hashlib.sha256()
    h.update(model.embeddings.tobytes())
    h.update(model.lm_head.tobytes())
    for mats in model.layers:
        for name in oracle.PROJECTIONS:
            h.update(mats[name][0].tobytes())
            h.update(mats[name][1].tobytes())
    return h.hexdigest()


@pytest.mark.parametrize("qtype,tag", [(INT8, "int8"), (INT4, "int4")])
def test_tiny_model_matches_reference(qtype, tag):
    g = np.load(os.path.join(GOLDEN, f"tiny_{tag}.npz"))
    model = W.build("tiny", qtype, 0)
    # synthetic weights + product quantiser == what the reference quantised
    assert digest(model) == str(g["digest"])
    om = oracle.oracle_model(model)
    ids, _, _ = om.generate(g["prompt"], 16)
    assert ids == g["ids"].tolist()
    om.reset()
    for i, token in enumerate(g["tokens"]):
        h = om.decode(int(token))
        assert np.array_equal(h, g["hidden"][i]), f"step {i}"
    assert np.array_equal(om.keys, g["keys"])
    assert np.array_equal(om.values, g["values"])
    logits = om.logits(g["hidden"][len(g["prompt"]) - 1])
    assert np.array_equal(logits, g["logits"])


@pytest.mark.parametrize("qtype,tag", [(INT8, "int8"), (INT4, "int4")])
def test_tiny_model_with_norms_matches_reference(qtype, tag):
    """Seeded non-unit attention, ffn and final norms (the three norms of
    src/quant_model.cpp:182-190 and src/generate.cpp:197-198): the oracle's
    greedy ids, every decode step's hidden state, the KV cache and the
    final-step logits equal the reference's bit for bit
    (tests/golden/tiny_norms_*.npz)."""
    g = np.load(os.path.join(GOLDEN, f"tiny_norms_{tag}.npz"))
    model = W.build("tiny", qtype, 0, norm_seed=int(g["norm_seed"]))
    assert digest(model) == str(g["digest"])
    om = oracle.oracle_model(model)
    ids, _, _ = om.generate(g["prompt"], 16)
    assert ids == g["ids"].tolist()
    om.reset()
    for i, token in enumerate(g["tokens"]):
        h = om.decode(int(token))
        assert np.array_equal(h, g["hidden"][i]), f"step {i}"
    assert np.array_equal(om.keys, g["keys"])
    assert np.array_equal(om.values, g["values"])
    logits = om.logits(g["hidden"][len(g["prompt"]) - 1])
    assert np.array_equal(logits, g["logits"])


def test_norm_fixtures_tell_the_norms_apart():
    """The non-unit-norm fixture pins the wiring: with the attention and ffn
    norms swapped, or the final norm left out, the oracle's output differs
    from the reference's."""
    g = np.load(os.path.join(GOLDEN, "tiny_norms_int8.npz"))
    model = W.build("tiny", INT8, 0, norm_seed=int(g["norm_seed"]))
    swapped = W.build("tiny", INT8, 0, norm_seed=int(g["norm_seed"]))
    swapped.norms = [(f, a) for a, f in model.norms]
    om = oracle.oracle_model(swapped)
    h = [om.decode(int(t)) for t in g["tokens"][:3]]
    assert not np.array_equal(h[-1], g["hidden"][2])
    unit_final = W.build("tiny", INT8, 0, norm_seed=int(g["norm_seed"]))
    unit_final.final_norm = np.ones_like(model.final_norm)
    om = oracle.oracle_model(unit_final)
    logits = om.logits(g["hidden"][len(g["prompt"]) - 1])
    assert not np.allclose(logits, g["logits"], rtol=1e-3, atol=0)


def test_tiny_prefill_equals_decode_loop():
    model = W.build("tiny", INT8, 0)
    prompt = W.synth_tokens(1, model.config.vocab_size, 5)
    om = oracle.oracle_model(model)
    h = om.prefill(prompt)
    om.reset()
    for t in prompt:
        h2 = om.decode(int(t))
    assert np.array_equal(h, h2)


def test_tinyllama_int4_greedy_ids_match_reference():
    with open(os.path.join(GOLDEN, "tinyllama_int4.json")) as f:
        g = json.load(f)
    model, prompt, gen = W.build_run("tinyllama_int4")
    assert prompt.tolist() == g["prompt"]
    assert digest(model) == g["digest"]
    om = oracle.oracle_model(model)
    before = oracle.orc().orc_get_threads()
    oracle.orc().orc_set_threads(min(8, os.cpu_count() or 1))
    try:
        ids, _, _ = om.generate(prompt, gen)
    finally:
        oracle.orc().orc_set_threads(before)
    assert ids == g["ids"]


def _llama2c_oracle(path, qtype):
    cfg, w, shared = llama2c.load(path)
    layers, norms = [], []
    for l in range(cfg["layers"]):
        mats = {}
        for name in oracle.PROJECTIONS:
            m = np.ascontiguousarray(w[name][l])
            st, data, scales = oracle.quantize(m, qtype)
            assert st == 0
            mats[name] = (data, scales, m.shape[0], m.shape[1])
        layers.append(mats)
        norms.append((np.ascontiguousarray(w["attention_norm"][l]),
                      np.ascontiguousarray(w["ffn_norm"][l])))
    return oracle.OracleModel(cfg, qtype,
                              np.ascontiguousarray(w["embeddings"]),
                              np.ascontiguousarray(w["final_norm"]),
                              np.ascontiguousarray(w["classifier"]), layers,
                              norms), shared


@pytest.mark.parametrize("qtype", [INT8, INT4])
def test_llama2c_fixture_says_hi(qtype):
    om, shared = _llama2c_oracle(os.path.join(GOLDEN, "tiny-llama2.bin"),
                                 qtype)
    assert not shared
    ids, _, _ = om.generate([1, 0, 3], 8)
    assert ids == [4, 5]


def test_llama2c_shared_fixture_ties_classifier():
    cfg, w, shared = llama2c.load(os.path.join(GOLDEN,
                                               "tiny-llama2-shared.bin"))
    assert shared and w["classifier"] is w["embeddings"]
    assert cfg["eos_token"] == 1


# ------------------------------------------------------- hand fixtures --

def test_rmsnorm_fixture():
    x = np.array([3.0, 4.0], np.float32)
    w = np.array([1.0, 2.0], np.float32)
    out = np.empty(2, np.float32)
    assert oracle.orc().orc_rmsnorm(oracle.ptr(x), oracle.ptr(w),
                                    oracle.ptr(out), 2, 0.0) == 0
    inv = 1.0 / math.sqrt(12.5)
    assert abs(out[0] - 3 * inv) < 1e-6 and abs(out[1] - 8 * inv) < 1e-6


def test_rope_fixture_position_one():
    q = np.array([1.0, 0.0], np.float32)
    k = np.array([0.0, 1.0], np.float32)
    oracle.orc().orc_rotate(oracle.ptr(q), 2, 1)
    oracle.orc().orc_rotate(oracle.ptr(k), 2, 1)
    c, s = math.cos(1.0), math.sin(1.0)
    assert max(abs(q[0] - c), abs(q[1] - s), abs(k[0] + s),
               abs(k[1] - c)) < 1e-6


def test_rope_position_zero_is_identity():
    v = np.random.default_rng(3).standard_normal(64).astype(np.float32)
    r = v.copy()
    oracle.orc().orc_rotate(oracle.ptr(r), 64, 0)
    assert np.array_equal(r, v)


def test_silu_closed_form():
    for x in (-20.0, -1.5, 0.0, 0.25, 3.0, 40.0):
        want = x / (1.0 + math.exp(-x))
        got = oracle.orc().orc_silu(x)
        assert abs(got - want) <= 1e-6 * max(1.0, abs(want))


def test_argmax_first_index_on_ties():
    def am(v):
        a = np.array(v, np.float32)
        return oracle.orc().orc_argmax(oracle.ptr(a), a.size)
    assert am([1, 3, 3, 2]) == 1
    assert am([-np.inf, -1, -1]) == 1
    assert am([0.5] * 7) == 0
    assert am([1, 2, 9, 9, 9]) == 2


CONFIG_CASES = [
    (dict(W.SHAPES["tiny"]), True),
    (dict(W.SHAPES["tinyllama"]), True),
    (dict(W.SHAPES["llama7b"]), True),
    (dict(W.SHAPES["tiny"], kv_heads=0), True),     # 0 means heads
    (dict(W.SHAPES["tiny"], kv_heads=3), False),    # 4 % 3 != 0
    (dict(W.SHAPES["tiny"], kv_heads=8), False),    # more kv than q heads
    (dict(W.SHAPES["tiny"], head_dim=15, dim=60), False),  # odd head_dim
    (dict(W.SHAPES["tiny"], dim=65), False),        # heads * hd != dim
    (dict(W.SHAPES["tiny"], eos_token=256), False),  # eos >= vocab
    (dict(W.SHAPES["tiny"], layers=0), False),
    (dict(W.SHAPES["tiny"], max_seq=0), False),
]


@pytest.mark.parametrize("cfg,valid", CONFIG_CASES)
def test_config_validation(cfg, valid):
    oc = oracle.OrcConfig(**cfg)
    assert bool(oracle.orc().orc_config_valid(C.byref(oc))) == valid
    pc = nut.Config(**cfg)
    assert bool(nut.lib().nut_config_valid(C.byref(pc))) == valid
