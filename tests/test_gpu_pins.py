"""GPU parity of inputs the headline path must not ignore.

* Non-unit attention, ffn and final norm weights (seeded N(1, 0.25^2))
  through the cooperative token kernel (fused and split attention, INT4 and
  INT8), the step kernels and the classifier: a swapped norm offset or an
  ignored final norm changes the hidden state by far more than rel-L2 1e-5
  (src/quant_model.cpp:182-190, src/generate.cpp:197-199).
* First-index argmax on exact logit ties (src/generate.cpp:24-30: the
  reference's std::max_element): identical classifier rows in the same
  wave's row pair, across waves and across workgroups, through the token
  kernel and the step path's classifier + pick.
* The token kernel's screened classifier (an INT8 block-32 copy with
  error bounds, fp32 logits only for the rows the bounds cannot rule out)
  returns the fp32 argmax when two rows' INT8 copies are identical but
  their fp32 logits differ by far more than fp32 rounding: the larger one
  wins in either index order; rows with a NaN or infinite weight behave
  as in the plain fp32 pass.
* QuantizedModelWeights::storage_bytes (src/quant_model.cpp:140-156) equal
  to the value the reference computed for the same model.
* The token kernel's exchange tags across a restart of their 32-bit range.
* The token kernel's bounded waits: a word that is never published ends
  the launch with the error flag instead of a hang.
"""
import dataclasses
import json
import os
import time

import numpy as np
import pytest

import oracle as O
from nutllm_amd import workloads as W
from screening import screen_twin

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
TOL = 1e-5
NORM_SEED = 11


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def check_kv(cache, om, c, positions, tol=TOL):
    for layer in range(c.layers):
        for kvh in range(c.kv_heads):
            for p in positions:
                k, v = cache.key_value(layer, kvh, p)
                rk, rv = om.kv_row(layer, kvh, p)
                assert rel_l2(k, rk) <= tol and rel_l2(v, rv) <= tol, (layer, kvh, p)


@pytest.mark.parametrize("qtype", [0, 1], ids=["int8", "int4"])
def test_nonunit_norms_token_kernel_fused(gpu, qtype):
    """Token kernel within its fused attention pass: the kernel's prefill
    loop over a 5-token prompt, two decode steps (hidden state and every
    layer's new K/V rows), then 12 greedy ids (final norm + classifier in
    the kernel), against the oracle with the same norm weights."""
    O.orc().orc_set_threads(16)
    model = W.build("tinyllama", qtype, 3, 64, norm_seed=NORM_SEED)
    c = model.config
    assert not np.allclose(model.final_norm, 1.0)
    prompt = gpu.synth_tokens(3, c.vocab_size, 5)
    dev = model.to_device()
    om = O.oracle_model(model)
    try:
        dev.set_path(2)
        cache = gpu.KVCache(c)
        h = dev.prefill(cache, prompt)
        err = rel_l2(h, om.prefill(prompt))
        print(f"qtype {qtype}: prefill hidden rel-L2 {err:.2e}", flush=True)
        assert err <= TOL
        for step, token in enumerate((11, 29999)):
            assert rel_l2(dev.decode(cache, token), om.decode(token)) <= TOL
            check_kv(cache, om, c, [len(prompt) + step])
        ids, _ = dev.generate(prompt, 12)
        ref, _, _ = om.generate(prompt, 12)
        assert ids == ref
    finally:
        dev.set_path(0)
        dev.close()


@pytest.mark.parametrize("qtype", [0, 1], ids=["int8", "int4"])
def test_token_kernel_fused_attention_past_32_positions(gpu, qtype):
    """The fused attention near the end of its pass (48 positions INT4, 44
    INT8): a 30-token prompt through the kernel's prefill loop, decode steps
    at positions 30..43 (hidden state and every layer's new K/V rows), then
    12 greedy ids from position 30, against the oracle with non-unit norm
    weights."""
    O.orc().orc_set_threads(16)
    model = W.build("tinyllama", qtype, 3, 64, norm_seed=NORM_SEED)
    c = model.config
    prompt = gpu.synth_tokens(5, c.vocab_size, 30)
    dev = model.to_device()
    om = O.oracle_model(model)
    try:
        dev.set_path(2)
        cache = gpu.KVCache(c)
        assert rel_l2(dev.prefill(cache, prompt), om.prefill(prompt)) <= TOL
        for step in range(14):
            token = 7 + 991 * step
            err = rel_l2(dev.decode(cache, token), om.decode(token))
            print(f"qtype {qtype} position {len(prompt) + step}: hidden rel-L2 {err:.2e}",
                  flush=True)
            assert err <= TOL
            check_kv(cache, om, c, [len(prompt) + step])
        ids, _ = dev.generate(prompt, 12)
        ref, _, _ = om.generate(prompt, 12)
        assert ids == ref
    finally:
        dev.set_path(0)
        dev.close()


def test_nonunit_norms_token_kernel_split(gpu):
    """Token kernel past its fused pass (split attention over the grid):
    from a 120-token step-kernel prefill, three token-kernel decode steps
    (hidden state, new K/V rows of every layer), then the greedy ids of
    generate() (batched prefill, split-attention decode loop with the final
    norm in the classifier phase)."""
    O.orc().orc_set_threads(16)
    model = W.build("tinyllama", 1, 3, 256, norm_seed=NORM_SEED)
    c = model.config
    prompt = gpu.synth_tokens(41, c.vocab_size, 120)
    dev = model.to_device()
    om = O.oracle_model(model)
    try:
        dev.set_path(1)
        cache = gpu.KVCache(c)
        hd = dev.prefill(cache, prompt)
        ho = om.prefill(prompt)
        assert rel_l2(hd, ho) <= TOL
        dev.set_path(2)
        ref = []
        for step in range(3):
            token = int(np.argmax(om.logits(ho)))
            if token == c.eos_token:
                break
            ref.append(token)
            ho, hd = om.decode(token), dev.decode(cache, token)
            err = rel_l2(hd, ho)
            print(f"split step {step}: hidden rel-L2 {err:.2e}", flush=True)
            assert err <= TOL
            check_kv(cache, om, c, [len(prompt) + step])
        ids, _ = dev.generate(prompt, len(ref))
        assert ids == ref
    finally:
        dev.set_path(0)
        dev.close()


def test_nonunit_norms_step_kernels_and_logits(gpu):
    """The step kernels (RMSNorm folded into the Q/K/V and gate/up row
    dots) and the classifier kernel with a non-unit final norm: prefill
    hidden state, every layer's K/V rows, the logits, and the greedy ids
    of the graph-replayed step loop."""
    O.orc().orc_set_threads(16)
    model = W.build("tinyllama", 1, 3, 64, norm_seed=NORM_SEED)
    c = model.config
    prompt = gpu.synth_tokens(5, c.vocab_size, 7)
    dev = model.to_device()
    om = O.oracle_model(model)
    try:
        dev.set_path(1)
        cache = gpu.KVCache(c)
        h = dev.prefill(cache, prompt)
        ho = om.prefill(prompt)
        assert rel_l2(h, ho) <= TOL
        check_kv(cache, om, c, [0, len(prompt) - 1])
        err = rel_l2(dev.logits(ho), om.logits(ho))
        print(f"logits rel-L2 {err:.2e}", flush=True)
        assert err <= TOL
        ids, _ = dev.generate(prompt, 10)
        ref, _, _ = om.generate(prompt, 10)
        assert ids == ref
    finally:
        dev.set_path(0)
        dev.close()


@pytest.fixture(scope="module")
def tie_model(gpu):
    O.orc().orc_set_threads(16)
    model = W.build("tinyllama", 1, 3, 64)
    prompt = gpu.synth_tokens(3, model.config.vocab_size, 5)
    om = O.oracle_model(model)
    top = int(np.argmax(om.logits(om.prefill(prompt))))
    dev = model.to_device()
    yield model, prompt, top, dev
    dev.close()


@pytest.mark.parametrize("offset", [-1, 1, -3, -700, 700],
                         ids=["prev", "next", "same-wg", "lower-wg", "higher-wg"])
@pytest.mark.parametrize("path", [1, 2], ids=["steps", "token"])
def test_argmax_first_index_on_device_ties(gpu, tie_model, path, offset):
    """Classifier row `top` (the argmax after the prompt) copied to row
    top + offset gives two bit-identical logits; the first generated id is
    the lower of the two rows, as std::max_element returns, and the rest of
    the greedy run equals the oracle's on the same weights."""
    model, prompt, top, dev = tie_model
    other = (top + offset) % model.config.vocab_size
    head = model.lm_head.copy()
    head[other] = head[top]
    dev.set_globals(model.embeddings, model.final_norm, head)
    try:
        dev.set_path(path)
        ids, _ = dev.generate(prompt, 4)
        assert ids[0] == min(top, other), (ids, top, other)
        tied = dataclasses.replace(model, lm_head=head)
        ref, _, _ = O.oracle_model(tied).generate(prompt, 4)
        assert ids == ref
    finally:
        dev.set_path(0)
        dev.set_globals(model.embeddings, model.final_norm, model.lm_head)


@pytest.mark.parametrize("offset,up", [(1, True), (700, True), (-1, False), (-700, False)],
                         ids=["next-up", "higher-wg-up", "prev-down", "lower-wg-down"])
@pytest.mark.parametrize("path", [1, 2], ids=["steps", "token"])
def test_argmax_screen_near_ties(gpu, tie_model, path, offset, up):
    """Row top + offset becomes a twin of the argmax row `top` with the same
    INT8 screening copy and an fp32 logit larger (up) or smaller, far above
    fp32 rounding: the first id is the larger logit's row, which a screen
    that broke ties of the copy's logits by index would miss (the twin has
    the higher index when larger, the lower when smaller), and the greedy
    run equals the oracle's on the same weights."""
    model, prompt, top, dev = tie_model
    om = O.oracle_model(model)
    hidden = np.asarray(om.prefill(prompt), np.float64)
    x = hidden / np.sqrt(np.mean(hidden * hidden) + 1e-5) * model.final_norm
    other = (top + offset) % model.config.vocab_size
    head = model.lm_head.copy()
    head[other] = screen_twin(head[top], x, up)
    gap = float(x @ (head[other].astype(np.float64) - head[top]))
    assert (gap > 5e-5) if up else (gap < -5e-5), gap
    want = other if up else top
    dev.set_globals(model.embeddings, model.final_norm, head)
    try:
        dev.set_path(path)
        ids, _ = dev.generate(prompt, 4)
        assert ids[0] == want, (ids, top, other, gap)
        twin = dataclasses.replace(model, lm_head=head)
        ref, _, _ = O.oracle_model(twin).generate(prompt, 4)
        assert ids == ref
    finally:
        dev.set_path(0)
        dev.set_globals(model.embeddings, model.final_norm, model.lm_head)


@pytest.mark.parametrize("poison", ["nan-top", "inf-other"])
@pytest.mark.parametrize("path", [1, 2], ids=["steps", "token"])
def test_argmax_nonfinite_classifier_rows(gpu, tie_model, path, poison):
    """A NaN weight in the argmax row makes its logit NaN, which never wins
    the first-max scan (src/generate.cpp:24-30): the next row does. A +inf
    weight against a positive x element makes another row's logit +inf,
    which wins. The screened argmax keeps every row with a non-finite block
    as a candidate, so both paths give the oracle's ids."""
    model, prompt, top, dev = tie_model
    om = O.oracle_model(model)
    hidden = np.asarray(om.prefill(prompt), np.float64)
    x = hidden / np.sqrt(np.mean(hidden * hidden) + 1e-5) * model.final_norm
    head = model.lm_head.copy()
    if poison == "nan-top":
        assert top != 0  # a NaN at row 0 would be the scan's answer
        head[top, 7] = np.nan
    else:
        other = (top + 321) % model.config.vocab_size
        head[other, int(np.argmax(x))] = np.inf
    dev.set_globals(model.embeddings, model.final_norm, head)
    try:
        dev.set_path(path)
        ids, _ = dev.generate(prompt, 4)
        bad = dataclasses.replace(model, lm_head=head)
        ref, _, _ = O.oracle_model(bad).generate(prompt, 4)
        assert ids == ref, (ids, ref, top)
        if poison == "nan-top":
            assert ids[0] != top
        else:
            assert ids[0] == other
    finally:
        dev.set_path(0)
        dev.set_globals(model.embeddings, model.final_norm, model.lm_head)


def test_storage_bytes_match_reference(gpu):
    """nut_model_storage_bytes equals QuantizedModelWeights::storage_bytes
    that the reference computed for the same models (golden fixtures)."""
    with open(os.path.join(GOLDEN, "tinyllama_int4.json")) as f:
        golden = json.load(f)
    model, _, _ = W.build_run("tinyllama_int4")
    dev = model.to_device()
    try:
        assert dev.storage_bytes() == golden["storage_bytes"]
    finally:
        dev.close()
    for qtype, tag in ((0, "int8"), (1, "int4")):
        g = np.load(os.path.join(GOLDEN, f"tiny_{tag}.npz"))
        dev = W.build("tiny", qtype, 0).to_device()
        try:
            assert dev.storage_bytes() == int(g["storage_bytes"])
        finally:
            dev.close()


def test_token_kernel_tags_across_restart(gpu):
    """Launch counter preset next to the end of the tag range: generate
    calls with fused and split attention, 1-token runs (only the argmax
    exchange) and per-token decodes cross the restart (the exchange buffer
    is zeroed, the counter starts again); every run gives the oracle's
    greedy ids and hidden states."""
    O.orc().orc_set_threads(16)
    model = W.build("tinyllama", 1, 3, 256)
    c = model.config
    short = gpu.synth_tokens(3, c.vocab_size, 5)
    long = gpu.synth_tokens(41, c.vocab_size, 60)
    om = O.oracle_model(model)
    ref_short, _, _ = om.generate(short, 6)
    ref_long, _, _ = om.generate(long, 4)
    ref_one, _, _ = om.generate(long, 1)
    om.reset()
    ref_h = om.prefill(short)
    ref_h2 = om.decode(ref_short[0])
    dev = model.to_device()
    try:
        dev.set_path(2)
        dev.set_launch_count(4091)
        for round_ in range(3):
            assert dev.generate(short, 6)[0] == ref_short, round_
            assert dev.generate(long, 4)[0] == ref_long, round_
            assert dev.generate(long, 1)[0] == ref_one, round_
            cache = gpu.KVCache(c)
            assert rel_l2(dev.prefill(cache, short), ref_h) <= TOL
            assert rel_l2(dev.decode(cache, ref_short[0]), ref_h2) <= TOL
    finally:
        dev.set_path(0)
        dev.close()


def test_token_kernel_bounded_waits_end_the_launch(gpu):
    """A wait that never completes (nut_model_inject_fault: workgroup 0
    leaves its words of the first step's h after W2 unpublished) runs into
    its spin limit and raises the error flag; every later wait gives up once
    it sees the flag, the generate loop leaves at its next argmax exchange,
    the launch ends, and the call fails with DeviceError, once: the next
    call (its prompt on the step kernels, then a token-kernel launch) gives
    the oracle's greedy ids."""
    O.orc().orc_set_threads(16)
    model = W.build("tinyllama", 1, 3, 256)
    c = model.config
    prompt = gpu.synth_tokens(3, c.vocab_size, 5)
    ref, _, _ = O.oracle_model(model).generate(prompt, 4)
    dev = model.to_device()
    try:
        assert dev.generate(prompt, 4)[0] == ref
        dev.inject_fault(1)
        t0 = time.time()
        with pytest.raises(gpu.DeviceError, match="timed out"):
            dev.generate(prompt, 4)
        print(f"faulted generate ended after {time.time() - t0:.2f} s", flush=True)
        dev.inject_fault(0)
        assert dev.generate(prompt, 4)[0] == ref
    finally:
        dev.inject_fault(0)
        dev.close()
