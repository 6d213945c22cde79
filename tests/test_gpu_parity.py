"""GPU parity: the HIP path through the C ABI against the CPU oracle.

Bars (from the path's contract): quantisation bit-exact; matvec, attention,
logits and hidden states within rel-L2 1e-5 (fp32 arithmetic); greedy token
ids identical for the first 16 generated tokens.
"""
import json
import os

import numpy as np
import pytest

import llama2c
import oracle as O
from nutllm_amd import workloads as W

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")

TOL = 1e-5  # rel-L2, fp32 paths


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


@pytest.mark.parametrize("qtype", [0, 1], ids=["int8", "int4"])
@pytest.mark.parametrize("shape", W.MATVEC_SHAPES,
                         ids=[f"{r}x{c}" for r, c in W.MATVEC_SHAPES])
def test_matvec_shapes(gpu, qtype, shape):
    rows, cols = shape
    i = W.MATVEC_SHAPES.index(shape)
    w = gpu.synth_normal(W.MATVEC_SEED, 100 + i, rows * cols).reshape(rows, cols)
    x = gpu.synth_normal(W.MATVEC_SEED, 200 + i, cols, sigma=1.0)
    data, scales = gpu.quantize(w, qtype)
    y = gpu.matvec_quantized(data, scales, rows, cols, qtype, x)
    ref = O.matvec_q(data, scales, rows, cols, qtype, x)
    assert rel_l2(y, ref) <= TOL


@pytest.mark.parametrize("qtype", [0, 1], ids=["int8", "int4"])
@pytest.mark.parametrize("shape,block", [((64, 172), 32), ((5, 37), 32),
                                         ((7, 33), 32), ((9, 40), 16),
                                         ((3, 50), 48), ((1, 1), 32)])
def test_matvec_straddling_blocks(gpu, qtype, shape, block):
    """Blocks along the flattened index straddle rows (src/quant.cpp:289-317)."""
    rows, cols = shape
    rng = np.random.default_rng(rows * 1000 + cols)
    w = rng.uniform(-1, 1, shape).astype(np.float32)
    x = rng.standard_normal(cols).astype(np.float32)
    data, scales = gpu.quantize(w, qtype, block)
    y = gpu.matvec_quantized(data, scales, rows, cols, qtype, x, block)
    ref = O.matvec_q(data, scales, rows, cols, qtype, x, block)
    assert rel_l2(y, ref) <= TOL


@pytest.mark.parametrize("qtype", [0, 1], ids=["int8", "int4"])
def test_matvec_unit_vectors_give_dequantised_columns(gpu, qtype):
    """x = e_k returns column k of the dequantised matrix exactly."""
    rows, cols = 96, 128
    w = gpu.synth_normal(7, 1, rows * cols).reshape(rows, cols)
    data, scales = gpu.quantize(w, qtype)
    deq = O.dequantize(data, scales, rows, cols, qtype)
    for k in (0, 1, 31, 32, 77, 127):
        x = np.zeros(cols, np.float32)
        x[k] = 1.0
        y = gpu.matvec_quantized(data, scales, rows, cols, qtype, x)
        np.testing.assert_array_equal(y, deq[:, k])


def test_matvec_zero_matrix(gpu):
    w = np.zeros((64, 64), np.float32)
    x = np.ones(64, np.float32)
    for qtype in (0, 1):
        data, scales = gpu.quantize(w, qtype)
        assert (scales == 1).all()  # 2^-24 for an all-zero block
        y = gpu.matvec_quantized(data, scales, 64, 64, qtype, x)
        np.testing.assert_array_equal(y, np.zeros(64, np.float32))


@pytest.mark.parametrize("shape", [(32000, 2048), (4096, 4096), (256, 64),
                                   (7, 9)])
def test_matvec_f32_classifier(gpu, shape):
    rows, cols = shape
    w = gpu.synth_normal(5, 1, rows * cols).reshape(rows, cols)
    x = gpu.synth_normal(5, 2, cols, sigma=1.0)
    y = gpu.matvec_f32(w, x)
    ref = np.empty(rows, np.float32)
    O.orc().orc_matvec_f32(O.ptr(w), rows, cols, O.ptr(x), O.ptr(ref))
    assert rel_l2(y, ref) <= TOL


# 768^3 and 224 x 640 x 96 run the k-split kernel (32 x 32 tiles, k over
# eight waves), 256 x 320 x 256 (k not a multiple of 128) the tiled kernel
# with 32 x 32 tiles, 1024 x 256 x 1024 64 x 64 tiles (256 of them), the
# odd shapes the generic kernel
@pytest.mark.parametrize("mkn", [(768, 768, 768), (224, 640, 96), (256, 320, 256),
                                 (1024, 256, 1024), (7, 9, 8), (65, 33, 130)])
def test_matmul_f32(gpu, mkn):
    m, k, n = mkn
    a = gpu.synth_normal(2, 300, m * k, sigma=1.0).reshape(m, k)
    b = gpu.synth_normal(2, 301, k * n, sigma=1.0).reshape(k, n)
    c = gpu.matmul_f32(a, b)
    ref = np.empty((m, n), np.float32)
    O.orc().orc_matmul(O.ptr(a), O.ptr(b), O.ptr(ref), m, k, n)
    assert rel_l2(c, ref) <= TOL
    # every kernel adds in a fixed order (the k-split one its eight partial
    # tiles in wave order): a second call gives the same bits
    assert np.array_equal(gpu.matmul_f32(a, b), c)


@pytest.fixture(scope="module")
def tiny(gpu):
    model, prompt, gen = W.build_run("tiny_int8")
    return model, prompt, gen, model.to_device()


def test_tiny_decode_hidden_and_cache(gpu, tiny):
    model, prompt, _, dev = tiny
    om = O.oracle_model(model)
    cache = gpu.KVCache(model.config)
    for t, tok in enumerate(prompt):
        h = dev.decode(cache, tok)
        ref = om.decode(tok)
        assert rel_l2(h, ref) <= TOL, f"token {t}"
    assert cache.length() == len(prompt)
    c = model.config
    for layer in range(c.layers):
        for head in range(c.kv_heads):
            for pos in range(len(prompt)):
                k, v = cache.key_value(layer, head, pos)
                rk, rv = om.kv_row(layer, head, pos)
                assert rel_l2(k, rk) <= TOL and rel_l2(v, rv) <= TOL


def test_tiny_prefill_equals_decode_loop(gpu, tiny):
    model, prompt, _, dev = tiny
    cache = gpu.KVCache(model.config)
    h = dev.prefill(cache, prompt)
    om = O.oracle_model(model)
    ref = om.prefill(prompt)
    assert rel_l2(h, ref) <= TOL
    assert cache.length() == len(prompt)


def test_tiny_logits(gpu, tiny):
    model, prompt, _, dev = tiny
    om = O.oracle_model(model)
    h = om.prefill(prompt)
    assert rel_l2(dev.logits(h), om.logits(h)) <= TOL


def test_tiny_greedy_tokens(gpu, tiny):
    model, prompt, gen, dev = tiny
    ids, stats = dev.generate(prompt, gen)
    om = O.oracle_model(model)
    ref, _, _ = om.generate(prompt, gen)
    assert ids == ref
    assert stats.prefill_tokens == len(prompt)
    assert stats.generated_tokens == len(ids)


def test_tiny_generation_to_full_cache(gpu, tiny):
    """The loop stops when the cache is full (src/generate.cpp:195-196)."""
    model, prompt, _, dev = tiny
    ids, _ = dev.generate(prompt, 1000)
    om = O.oracle_model(model)
    ref, _, _ = om.generate(prompt, 1000)
    assert ids == ref
    assert len(ids) <= model.config.max_seq - len(prompt)


def test_decode_errors(gpu, tiny):
    model, prompt, _, dev = tiny
    cache = gpu.KVCache(model.config)
    with pytest.raises(gpu.OutOfRange, match="token out of range"):
        dev.decode(cache, model.config.vocab_size)
    with pytest.raises(gpu.OutOfRange):
        dev.decode(cache, -1)
    cache.set_length(model.config.max_seq)
    with pytest.raises(gpu.LengthError, match="context is full"):
        dev.decode(cache, 0)
    with pytest.raises(gpu.InvalidArgument, match="invalid prompt"):
        dev.prefill(cache, np.zeros(0, np.int32))
    other = W.make_config("tiny", max_seq=32)
    with pytest.raises(gpu.InvalidArgument, match="cache configuration mismatch"):
        dev.decode(gpu.KVCache(other), 0)


def test_tinyllama_int4_greedy_16(gpu):
    """Headline shape: 16 greedy ids identical to the oracle's and to the
    ids the reference generated (tests/golden/tinyllama_int4.json)."""
    O.orc().orc_set_threads(16)
    model, prompt, gen = W.build_run("tinyllama_int4")
    dev = model.to_device()
    ids, _ = dev.generate(prompt, gen)
    om = O.oracle_model(model)
    ref, _, _ = om.generate(prompt, gen)
    assert ids == ref
    with open(os.path.join(GOLDEN, "tinyllama_int4.json")) as f:
        golden = json.load(f)
    assert golden["prompt"] == prompt.tolist()
    assert ids == golden["ids"]
    assert len(ids) == 16 or 1 in ref
    # hidden state after the prompt
    cache = gpu.KVCache(model.config)
    h = dev.prefill(cache, prompt)
    om.reset()
    assert rel_l2(h, om.prefill(prompt)) <= TOL
    dev.close()


@pytest.fixture(scope="module")
def tinyllama_int4(gpu):
    O.orc().orc_set_threads(16)
    model, prompt, gen = W.build_run("tinyllama_int4")
    dev = model.to_device()
    yield model, prompt, gen, dev
    dev.close()


@pytest.mark.parametrize("path", [1, 2], ids=["steps", "token"])
def test_tinyllama_int4_paths_greedy(gpu, tinyllama_int4, path):
    """Step kernels and the cooperative token kernel both reproduce the
    oracle's 16 greedy ids and its post-prompt hidden state."""
    model, prompt, gen, dev = tinyllama_int4
    dev.set_path(path)
    ids, stats = dev.generate(prompt, gen)
    om = O.oracle_model(model)
    ref, _, _ = om.generate(prompt, gen)
    assert ids == ref
    cache = gpu.KVCache(model.config)
    h = dev.prefill(cache, prompt)
    om.reset()
    assert rel_l2(h, om.prefill(prompt)) <= TOL
    # one more decode step on the same cache, and its K/V rows
    h2 = dev.decode(cache, ref[0])
    assert rel_l2(h2, om.decode(ref[0])) <= TOL
    pos = len(prompt)
    for layer in (0, model.config.layers - 1):
        for head in range(model.config.kv_heads):
            k, v = cache.key_value(layer, head, pos)
            rk, rv = om.kv_row(layer, head, pos)
            assert rel_l2(k, rk) <= TOL and rel_l2(v, rv) <= TOL
    dev.set_path(0)


def test_tinyllama_int8_token_kernel_short_context(gpu):
    """The INT8 token kernel within its fused attention pass (44 positions):
    a 5-token prompt decoded token by token by the kernel's prefill loop,
    then 16 greedy ids, against the oracle; hidden states and K/V rows
    within rel-L2 1e-5."""
    O.orc().orc_set_threads(16)
    model = W.build("tinyllama", 0, 3, 64)
    c = model.config
    prompt = gpu.synth_tokens(3, c.vocab_size, 5)
    dev = model.to_device()
    om = O.oracle_model(model)
    try:
        dev.set_path(2)
        cache = gpu.KVCache(c)
        h = dev.prefill(cache, prompt)
        assert rel_l2(h, om.prefill(prompt)) <= TOL
        h2 = dev.decode(cache, 11)
        assert rel_l2(h2, om.decode(11)) <= TOL
        for layer in (0, c.layers - 1):
            for kvh in range(c.kv_heads):
                k, v = cache.key_value(layer, kvh, len(prompt))
                rk, rv = om.kv_row(layer, kvh, len(prompt))
                assert rel_l2(k, rk) <= TOL and rel_l2(v, rv) <= TOL
        ids, _ = dev.generate(prompt, 16)
        ref, _, _ = om.generate(prompt, 16)
        assert ids == ref
    finally:
        dev.set_path(0)
        dev.close()


@pytest.mark.parametrize("scale", [300.0, 1e-30], ids=["outliers", "tiny_dims"])
def test_token_kernel_wide_range_activations(gpu, scale):
    """Every 257th embedding dimension scaled by 300 (outlier features, as in
    trained models) or by 1e-30 (elements far below their block's maximum):
    the token kernel's integer digit dots, which keep x to 2^-23.7 of each
    32-block's maximum, still hold the fp32 bar on the post-prompt and
    next-token hidden states and on the new K/V rows."""
    O.orc().orc_set_threads(16)
    model, prompt, _ = W.build_run("tinyllama_int4")
    model.embeddings[:, ::257] *= np.float32(scale)
    dev = model.to_device()
    dev.set_path(2)
    om = O.oracle_model(model)
    cache = gpu.KVCache(model.config)
    h = dev.prefill(cache, prompt)
    assert rel_l2(h, om.prefill(prompt)) <= TOL
    token = int(prompt[0])
    h2 = dev.decode(cache, token)
    assert rel_l2(h2, om.decode(token)) <= TOL
    pos = len(prompt)
    for layer in (0, model.config.layers - 1):
        for head in range(model.config.kv_heads):
            k, v = cache.key_value(layer, head, pos)
            rk, rv = om.kv_row(layer, head, pos)
            assert rel_l2(k, rk) <= TOL and rel_l2(v, rv) <= TOL
    dev.close()


@pytest.mark.parametrize("qtype", [0, 1], ids=["int8", "int4"])
def test_token_kernel_split_attention(gpu, qtype):
    """Contexts beyond the token kernel's fused attention pass (48 positions
    INT4, 44 INT8): attention is split over the grid (each workgroup one KV
    head over a run of positions, each context value merged over the runs
    by one workgroup). From a 300-token prefill on the step kernels, each
    token-kernel decode step's hidden state and new K/V rows within rel-L2
    1e-5 of the oracle; then generate() (batched prefill, split-attention
    decode loop) gives the oracle's greedy ids."""
    O.orc().orc_set_threads(16)
    model = W.build("tinyllama", qtype, 3, 512)
    c = model.config
    prompt = gpu.synth_tokens(23, c.vocab_size, 300)
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
        for step in range(6):
            token = int(np.argmax(om.logits(ho)))
            if token == c.eos_token:
                break
            ref.append(token)
            ho, hd = om.decode(token), dev.decode(cache, token)
            err = rel_l2(hd, ho)
            print(f"qtype {qtype} step {step}: hidden rel-L2 {err:.2e}", flush=True)
            assert err <= TOL
            pos = len(prompt) + step
            for layer in (0, c.layers - 1):
                for kvh in range(c.kv_heads):
                    k, v = cache.key_value(layer, kvh, pos)
                    rk, rv = om.kv_row(layer, kvh, pos)
                    assert rel_l2(k, rk) <= TOL and rel_l2(v, rv) <= TOL
        dev.set_path(0)
        ids, _ = dev.generate(prompt, len(ref))
        assert ids == ref
    finally:
        dev.set_path(0)
        dev.close()


def test_token_kernel_split_attention_max_context(gpu):
    """The split attention at its limit: max_seq 4096, the last decode step
    at 4096 positions (64 per run, every run full). Two caches filled by the
    same batched prefill of 4090 tokens (deterministic, so identical); the
    token kernel on one and the step kernels (checked against the oracle up
    to 1100 positions) on the other agree on each of six decode steps'
    hidden state and new K/V rows within rel-L2 1e-5."""
    model = W.build("tinyllama", 1, 3, 4096)
    c = model.config
    prompt = gpu.synth_tokens(29, c.vocab_size, 4090)
    tokens = [int(t) for t in gpu.synth_tokens(31, c.vocab_size, 6)]
    dev = model.to_device()
    try:
        dev.set_path(0)
        cache_t, cache_s = gpu.KVCache(c), gpu.KVCache(c)
        h_t = dev.prefill(cache_t, prompt)
        h_s = dev.prefill(cache_s, prompt)
        assert np.array_equal(h_t, h_s)
        for step, token in enumerate(tokens):
            dev.set_path(2)
            h_t = dev.decode(cache_t, token)
            dev.set_path(1)
            h_s = dev.decode(cache_s, token)
            err = rel_l2(h_t, h_s)
            print(f"position {len(prompt) + step}: hidden rel-L2 {err:.2e}", flush=True)
            assert err <= TOL
            pos = len(prompt) + step
            for layer in (0, c.layers - 1):
                for kvh in range(c.kv_heads):
                    kt, vt = cache_t.key_value(layer, kvh, pos)
                    ks, vs = cache_s.key_value(layer, kvh, pos)
                    assert rel_l2(kt, ks) <= TOL and rel_l2(vt, vs) <= TOL
    finally:
        dev.set_path(0)
        dev.close()


def test_token_kernel_rejects_unsupported_shape(gpu, tiny):
    model, prompt, _, dev = tiny
    dev.set_path(2)
    with pytest.raises(gpu.InvalidArgument, match="token kernel"):
        dev.generate(prompt, 4)
    dev.set_path(0)


@pytest.mark.parametrize("qtype", [0, 1], ids=["int8", "int4"])
def test_llama2c_fixture_says_hi(gpu, qtype):
    """The reference's llama2.c fixture (all-zero projections): prompt
    [1, 0, 3] generates [4, 5] then eos (src/loader_selftest.cpp, file lines
    81-116), through the device model and the product quantiser."""
    cfg, w, _ = llama2c.load(os.path.join(GOLDEN, "tiny-llama2.bin"))
    dev = gpu.DeviceModel(gpu.Config(**cfg), qtype)
    dev.set_globals(np.ascontiguousarray(w["embeddings"]),
                    np.ascontiguousarray(w["final_norm"]),
                    np.ascontiguousarray(w["classifier"]))
    for l in range(cfg["layers"]):
        mats = {}
        for name in O.PROJECTIONS:
            m = np.ascontiguousarray(w[name][l])
            data, scales = gpu.quantize(m, qtype)
            mats[name] = (data, scales, m.shape[0], m.shape[1])
        dev.set_layer(l, mats, np.ascontiguousarray(w["attention_norm"][l]),
                      np.ascontiguousarray(w["ffn_norm"][l]))
    ids, stats = dev.generate(np.array([1, 0, 3], np.int32), 8)
    assert ids == [4, 5]
    assert stats.prefill_tokens == 3 and stats.generated_tokens == 2
    dev.close()


@pytest.mark.parametrize("norms", [False, True], ids=["unit_norms", "seeded_norms"])
@pytest.mark.parametrize("qtype,tag", [(0, "int8"), (1, "int4")])
def test_tiny_matches_reference_golden(gpu, qtype, tag, norms):
    """Greedy ids equal the reference's; every decode step's hidden state
    and the final-step logits within rel-L2 1e-5 of the reference's
    (tests/golden/tiny_*.npz; tiny_norms_*.npz with seeded non-unit
    attention, ffn and final norms)."""
    g = np.load(os.path.join(GOLDEN, f"tiny_{'norms_' if norms else ''}{tag}.npz"))
    model = W.build("tiny", qtype, 0, norm_seed=int(g["norm_seed"]) if norms else None)
    dev = model.to_device()
    ids, _ = dev.generate(g["prompt"], 16)
    assert ids == g["ids"].tolist()
    cache = gpu.KVCache(model.config)
    for i, token in enumerate(g["tokens"]):
        h = dev.decode(cache, int(token))
        assert rel_l2(h, g["hidden"][i]) <= TOL, f"step {i}"
    logits = dev.logits(g["hidden"][len(g["prompt"]) - 1])
    assert rel_l2(logits, g["logits"]) <= TOL
    dev.close()


@pytest.mark.parametrize("prompt_len", [2, 5, 6, 15, 29])
def test_tinyllama_int4_prefill_step_chunk(gpu, tinyllama_int4, prompt_len):
    """Prompts below the GEMM threshold (30 tokens) run as one chunk of
    consecutive tokens through the step kernels (each launch covers every
    token of the chunk; the arithmetic per token is the decode step's; from
    6 tokens the row launches take four rows per wave). Hidden state and
    K/V rows within rel-L2 1e-5 of the oracle's per-token prefill."""
    model, _, _, dev = tinyllama_int4
    prompt = gpu.synth_tokens(17, model.config.vocab_size, prompt_len)
    cache = gpu.KVCache(model.config)
    dev.set_path(0)
    h = dev.prefill(cache, prompt)
    om = O.oracle_model(model)
    assert rel_l2(h, om.prefill(prompt)) <= TOL
    for layer in (0, model.config.layers - 1):
        for kvh in range(model.config.kv_heads):
            for p in sorted({0, prompt_len // 2, prompt_len - 1}):
                k, v = cache.key_value(layer, kvh, p)
                rk, rv = om.kv_row(layer, kvh, p)
                assert rel_l2(k, rk) <= TOL and rel_l2(v, rv) <= TOL
    # the next decode step continues from the chunked prefill
    assert rel_l2(dev.decode(cache, 7), om.decode(7)) <= TOL


PREFILL_TOL = 2e-3  # rel-L2, batched (GEMM) prefill


@pytest.mark.parametrize("prompt_len", [30, 40, 64, 130, 300])
def test_tinyllama_int4_prefill_gemm(gpu, tinyllama_int4, prompt_len):
    """Prompts of 30+ tokens run as a batch (MFMA GEMMs, causal attention).
    Hidden state and K/V rows within rel-L2 2e-3 of the fp32 step arithmetic
    (oracle for 30 and 40 tokens, the device step kernels for 64, 130 and
    300: one whole 64-query attention tile with no padding, then three and
    five tiles), and the greedy ids that follow the prefill identical to the
    oracle's. 30 tokens is the shortest batched prompt (34 padding rows in
    its tile)."""
    model, _, _, dev = tinyllama_int4
    prompt = gpu.synth_tokens(11, model.config.vocab_size, prompt_len)
    cache = gpu.KVCache(model.config)
    h = dev.prefill(cache, prompt)
    if prompt_len <= 40:
        om = O.oracle_model(model)
        ref = om.prefill(prompt)
        kv_ref = lambda l, kvh, p: om.kv_row(l, kvh, p)  # noqa: E731
    else:
        dev.set_path(1)
        ref_cache = gpu.KVCache(model.config)
        ref = dev.prefill(ref_cache, prompt)
        dev.set_path(0)
        kv_ref = lambda l, kvh, p: ref_cache.key_value(l, kvh, p)  # noqa: E731
    err = rel_l2(h, ref)
    print(f"prefill {prompt_len} tokens: hidden rel-L2 {err:.2e}", flush=True)
    assert err <= PREFILL_TOL
    for layer in (0, model.config.layers - 1):
        for kvh in range(model.config.kv_heads):
            for p in (0, prompt_len // 2, prompt_len - 1):
                k, v = cache.key_value(layer, kvh, p)
                rk, rv = kv_ref(layer, kvh, p)
                assert rel_l2(k, rk) <= PREFILL_TOL and rel_l2(v, rv) <= PREFILL_TOL
    if prompt_len <= 40:
        ids, _ = dev.generate(prompt, 8)
        ref_ids, _, _ = om.generate(prompt, 8)
        assert ids == ref_ids


@pytest.mark.parametrize("qtype", [0, 1], ids=["int8", "int4"])
def test_prefill_gemm_fills_the_cache(gpu, qtype):
    """A batched prefill of exactly max_seq tokens (max_seq 192: three full
    64-query attention tiles, the attention's K/V limb rows used to the
    last): hidden state and the first and last positions' K/V rows within
    rel-L2 2e-3 of the step kernels, and the next decode step then fails
    with the reference's full-cache error."""
    model = W.build("tinyllama", qtype, 5, 192)
    c = model.config
    prompt = gpu.synth_tokens(29, c.vocab_size, c.max_seq)
    dev = model.to_device()
    try:
        cache = gpu.KVCache(c)
        h = dev.prefill(cache, prompt)
        dev.set_path(1)
        ref_cache = gpu.KVCache(c)
        ref = dev.prefill(ref_cache, prompt)
        dev.set_path(0)
        err = rel_l2(h, ref)
        print(f"prefill of max_seq tokens: hidden rel-L2 {err:.2e}", flush=True)
        assert err <= PREFILL_TOL
        for layer in (0, c.layers - 1):
            for kvh in range(c.kv_heads):
                for p in (0, c.max_seq - 1):
                    k, v = cache.key_value(layer, kvh, p)
                    rk, rv = ref_cache.key_value(layer, kvh, p)
                    assert rel_l2(k, rk) <= PREFILL_TOL and rel_l2(v, rv) <= PREFILL_TOL
        with pytest.raises(gpu.LengthError, match="context is full"):
            dev.decode(cache, 0)
    finally:
        dev.close()


@pytest.mark.parametrize("shape,qtype", [("step_mha128", 1), ("step_gqa4", 0)],
                         ids=["mha128-int4", "gqa4-int8"])
def test_prefill_gemm_other_heads(gpu, shape, qtype):
    """Batched prefill of 200 tokens at head_dim 128 with one query head
    per KV head, and at head_dim 64 with four, non-unit norm weights:
    hidden state and K/V rows within rel-L2 2e-3 of the oracle."""
    O.orc().orc_set_threads(16)
    model = W.build(shape, qtype, 6)
    c = model.config
    rng = np.random.default_rng(9)
    norms = [tuple((1.0 + 0.25 * rng.standard_normal(c.dim)).astype(np.float32)
                   for _ in range(2)) for _ in range(c.layers)]
    dev = gpu.DeviceModel(c, qtype)
    dev.set_globals(model.embeddings, model.final_norm, model.lm_head)
    for i, mats in enumerate(model.layers):
        dev.set_layer(i, mats, norms[i][0], norms[i][1])
    cfg = {n: getattr(c, n) for n, _ in O.OrcConfig._fields_}
    om = O.OracleModel(cfg, qtype, model.embeddings, model.final_norm,
                       model.lm_head, model.layers, norms)
    prompt = gpu.synth_tokens(23, c.vocab_size, 200)
    try:
        cache = gpu.KVCache(c)
        h = dev.prefill(cache, prompt)
        err = rel_l2(h, om.prefill(prompt))
        print(f"{shape}: prefill hidden rel-L2 {err:.2e}", flush=True)
        assert err <= PREFILL_TOL
        for layer in range(c.layers):
            for kvh in range(c.kv_heads):
                for p in (0, 99, 199):
                    k, v = cache.key_value(layer, kvh, p)
                    rk, rv = om.kv_row(layer, kvh, p)
                    assert rel_l2(k, rk) <= PREFILL_TOL and rel_l2(v, rv) <= PREFILL_TOL
    finally:
        dev.close()


def test_tinyllama_int4_graph_replays_match_eager(gpu, tinyllama_int4):
    """A 60-token prompt is past the token kernel's fused attention, so
    generation replays a captured graph of one greedy iteration per token.
    Two graph runs, with eager step-kernel work between them, give the ids
    of the eager path and of the oracle."""
    model, _, _, dev = tinyllama_int4
    prompt = gpu.synth_tokens(13, model.config.vocab_size, 60)
    om = O.oracle_model(model)
    ref, _, _ = om.generate(prompt, 8)
    dev.set_path(0)
    first, _ = dev.generate(prompt, 8)
    dev.set_path(1)
    eager, _ = dev.generate(prompt, 8)
    dev.set_path(0)
    second, _ = dev.generate(prompt, 8)
    assert eager == ref
    assert first == ref and second == ref


STEP_SHAPES = [("step_mha128", 1), ("step_gqa4", 0), ("step_gqa2", 1)]


@pytest.mark.parametrize("shape,qtype", STEP_SHAPES,
                         ids=["mha128-int4", "gqa4-int8", "gqa2-int4"])
def test_step_kernels_long_context(gpu, shape, qtype):
    """Step kernels against the oracle at a 1100-token context: RMSNorm
    folded into the Q/K/V and gate/up matvecs (non-unit norm weights), and
    attention split over 35 chunks of 32 positions whose splits are merged
    by the last workgroup of each KV head. Hidden state after the prefill
    (74 chunks of up to 15 consecutive tokens), K/V rows and each decode
    step of the greedy continuation (rel-L2 1e-5); 8 greedy ids identical."""
    O.orc().orc_set_threads(16)
    model = W.build(shape, qtype, 5)
    c = model.config
    rng = np.random.default_rng(7)
    norms = [tuple((1.0 + 0.25 * rng.standard_normal(c.dim)).astype(np.float32)
                   for _ in range(2)) for _ in range(c.layers)]
    dev = gpu.DeviceModel(c, qtype)
    dev.set_globals(model.embeddings, model.final_norm, model.lm_head)
    for i, mats in enumerate(model.layers):
        dev.set_layer(i, mats, norms[i][0], norms[i][1])
    cfg = {n: getattr(c, n) for n, _ in O.OrcConfig._fields_}
    om = O.OracleModel(cfg, qtype, model.embeddings, model.final_norm,
                       model.lm_head, model.layers, norms)
    prompt = gpu.synth_tokens(21, c.vocab_size, 1100)
    dev.set_path(1)
    try:
        cache = gpu.KVCache(c)
        h = dev.prefill(cache, prompt)
        om.reset()
        om_h = om.prefill(prompt)
        err = rel_l2(h, om_h)
        print(f"{shape}: prefill hidden rel-L2 {err:.2e}", flush=True)
        assert err <= TOL
        for layer in range(c.layers):
            for kvh in range(c.kv_heads):
                for p in (0, 550, 1099):
                    k, v = cache.key_value(layer, kvh, p)
                    rk, rv = om.kv_row(layer, kvh, p)
                    assert rel_l2(k, rk) <= TOL and rel_l2(v, rv) <= TOL
        # greedy continuation on both caches (src/generate.cpp:194-207):
        # every decode step's hidden state, then the device's own loop
        ref, ho, hd = [], om_h, h
        for _ in range(8):
            token = int(np.argmax(om.logits(ho)))
            if token == c.eos_token:
                break
            ref.append(token)
            ho, hd = om.decode(token), dev.decode(cache, token)
            assert rel_l2(hd, ho) <= TOL
        ids, _ = dev.generate(prompt, 8)
        assert ids == ref
    finally:
        dev.set_path(0)
        dev.close()
