"""Write the golden vectors under tests/golden/ from the reference itself.

The expected outputs come from oracle/_ref/libnutref.so: the reference's
own sources (src/quant.cpp, src/quant_model.cpp, src/generate.cpp, ...)
compiled in place by `make -C oracle ref`. Inputs are seeded (numpy
default_rng, or the shared synthetic generator of nutllm_amd.workloads), so
every fixture can be regenerated:

    make -C oracle ref && python tests/golden/make_golden.py

Files written:
  quant.npz       quantiser cases: crafted fp16-scale blocks (ties,
                  subnormal boundary, clamp, zero block, lround ties of the
                  codes), row-straddling blocks, random matrices; bytes,
                  scale bits, storage_bytes, error bounds, and the matvec
                  output of each (matvec_quantized_threaded)
  quant_errors.json  inputs the reference rejects, with the exception kind
  tiny_int8.npz, tiny_int4.npz
                  the tiny synthetic model quantised by the reference:
                  greedy ids (16), per-step hidden states, final-step
                  logits, KV cache contents
  tiny_norms_int8.npz, tiny_norms_int4.npz
                  the same with seeded non-unit attention, ffn and final
                  norm weights
  tinyllama_int4.json  greedy ids of the TinyLlama-shape INT4 run
                  (5-token prompt, 16 tokens) and its storage_bytes
  fp32_*.npz      the fp32 model path (ModelWeights): prefill_tokens rows
                  for a 6-token prompt, then 4 decode_token hidden states
                  and the KV cache, for the tiny shape (untied and tied)
                  and a dim-256 / head_dim-64 shape
  sampled.json    greedy-free runs: generate_tokens_cached with temperature /
                  top-p / seed (choose_token's sampling branch) on the tiny
                  INT8 and TinyLlama INT4 models
  tinyllama_int8_2k.npz, llama7b_int4.npz
                  the long-prompt runs (TinyLlama-shape INT8, 2048-token
                  prompt, 128 tokens; Llama-2-7B-shape INT4, 512-token
                  prompt, 128 tokens): greedy ids, the hidden state after
                  the prompt, sampled K/V cache rows, storage_bytes

Also copied verbatim (data files the reference's tests hold):
  tiny-llama2.bin, tiny-llama2-shared.bin   (tests/fixtures/)
"""
from __future__ import annotations

import hashlib
import json
import os
import shutil
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402
from nutllm_amd import INT4, INT8, workloads as W  # noqa: E402

REFERENCE = "/root/reference"


def ref_quantize(w, qtype, block_size=32):
    w = np.ascontiguousarray(w, np.float32)
    rows, cols = w.shape
    n = rows * cols
    data = np.zeros(n if qtype == INT8 else (n + 1) // 2, np.uint8)
    scales = np.zeros((n + block_size - 1) // block_size, np.uint16)
    storage = oracle.C.c_size_t()
    bounds = np.zeros(n, np.float32)
    st = oracle.ref().ref_quantize(
        oracle.ptr(w), rows, cols, qtype, block_size, oracle.ptr(data),
        oracle.ptr(scales), oracle.C.byref(storage), oracle.ptr(bounds))
    return st, data, scales, storage.value, bounds.reshape(rows, cols)


def ref_matvec(w, qtype, x, threads=1, block_size=32):
    w = np.ascontiguousarray(w, np.float32)
    rows, cols = w.shape
    y = np.zeros(rows, np.float32)
    oracle.check(oracle.ref().ref_matvec_q(
        oracle.ptr(w), rows, cols, qtype, block_size,
        oracle.ptr(np.ascontiguousarray(x, np.float32)), oracle.ptr(y),
        threads), "ref_matvec_q")
    return y


def half_value(bits):
    return float(np.uint16(bits).view(np.float16))


def crafted_scale_row(qtype, rng):
    """One row of 32-blocks; block j's max |w| is limit * e_j for a crafted
    scale e_j, the other weights uniform in (-max, max)."""
    limit = 7 if qtype == INT4 else 127
    es = []
    # exact fp16 values and midpoints between neighbours (lround ties),
    # normal range
    for bits in (0x0400, 0x0401, 0x3C00, 0x3C01, 0x3BFF, 0x2E66, 0x5640,
                 0x7BFE):
        lo, hi = half_value(bits), half_value(bits + 1)
        es += [lo, (lo + hi) / 2]
    # subnormal range: exact, midpoints, the clamp to 1 and to 1023
    for m in (1, 2, 3, 100, 511, 1022):
        es += [m * 2.0 ** -24, (m + 0.5) * 2.0 ** -24]
    es += [0.3 * 2.0 ** -24, 0.5 * 2.0 ** -24, 1023.25 * 2.0 ** -24,
           1023.5 * 2.0 ** -24, 1023.75 * 2.0 ** -24, 2.0 ** -14 * 0.99999]
    # the largest scales
    es += [65504.0 / 2, 65504.0]
    blocks = []
    for e in es:
        mx = np.float32(e) * np.float32(limit)
        b = rng.uniform(-1.0, 1.0, 32).astype(np.float32) * mx
        b[rng.integers(32)] = mx if rng.integers(2) else -mx
        blocks.append(b)
    # a block whose codes land on lround ties: w = (k + 1/2) * stored
    s = half_value(0x3C00)  # 1.0: exact scale for max = limit
    b = np.array([(k % limit) + 0.5 for k in range(31)] + [limit],
                 np.float32) * np.float32(s)
    b[::2] *= -1
    blocks.append(b)
    blocks.append(np.zeros(32, np.float32))  # zero block: scale 2^-24
    return np.concatenate(blocks)[None, :]


def quant_cases():
    rng = np.random.default_rng(20240601)
    cases = []
    for qtype in (INT8, INT4):
        cases.append((f"crafted_{qtype}", crafted_scale_row(qtype, rng), qtype))
        # the reference's own packing KAT (src/quant_selftest.cpp:92-101)
        cases.append((f"kat_{qtype}",
                      np.array([[-7.0, -1.0, 2.0, 7.0]], np.float32), qtype))
        # blocks straddling rows (cols % 32 != 0), odd element count
        cases.append((f"straddle_{qtype}",
                      rng.standard_normal((5, 37)).astype(np.float32), qtype))
        # the tiny model's W2 shape (64 x 172)
        cases.append((f"w2_{qtype}",
                      (rng.standard_normal((64, 172)) * 0.02).astype(np.float32),
                      qtype))
        # fast layout with wide dynamic range per block
        w = rng.standard_normal((16, 256)).astype(np.float32)
        w *= np.exp2(rng.integers(-20, 8, size=(16, 256))).astype(np.float32)
        cases.append((f"range_{qtype}", w, qtype))
    return cases


def write_quant():
    out = {}
    names = []
    rng = np.random.default_rng(7)
    for name, w, qtype in quant_cases():
        st, data, scales, storage, bounds = ref_quantize(w, qtype)
        assert st == 0, (name, st)
        x = rng.standard_normal(w.shape[1]).astype(np.float32)
        y = ref_matvec(w, qtype, x, threads=1)
        y3 = ref_matvec(w, qtype, x, threads=3)
        assert np.array_equal(y, y3), name  # thread-count invariance
        out[f"{name}/w"] = w
        out[f"{name}/qtype"] = np.int32(qtype)
        out[f"{name}/data"] = data
        out[f"{name}/scales"] = scales
        out[f"{name}/storage"] = np.int64(storage)
        out[f"{name}/bounds"] = bounds
        out[f"{name}/x"] = x
        out[f"{name}/y"] = y
        names.append(name)
    out["names"] = np.array(names)
    np.savez_compressed(os.path.join(HERE, "quant.npz"), **out)


def write_quant_errors():
    cases = [
        ("nan", [[float("nan")] + [1.0] * 31], INT8),
        ("inf", [[float("inf")] + [1.0] * 31], INT4),
        ("scale_above_fp16_int8", [[65504.0 * 127 * 1.01] + [0.0] * 31], INT8),
        ("scale_above_fp16_int4", [[65504.0 * 7 * 1.01] + [0.0] * 31], INT4),
    ]
    out = []
    for name, w, qtype in cases:
        st, *_ = ref_quantize(np.array(w, np.float32), qtype)
        out.append({"name": name, "w0": repr(w[0][0]), "qtype": qtype,
                    "status": st})
    with open(os.path.join(HERE, "quant_errors.json"), "w") as f:
        json.dump(out, f, indent=1)


def weight_digest(model):
    h = hashlib.sha256()
    h.update(model.embeddings.tobytes())
    h.update(model.lm_head.tobytes())
    for mats in model.layers:
        for name in oracle.PROJECTIONS:
            h.update(mats[name][0].tobytes())
            h.update(mats[name][1].tobytes())
    return h.hexdigest()


def write_tiny(qtype, tag):
    model = W.build("tiny", qtype, 0, keep_fp32=True)
    c = model.config
    cfg = {n: getattr(c, n) for n, _ in oracle.OrcConfig._fields_}
    ref = oracle.RefModel(cfg, qtype, model.embeddings, model.final_norm,
                          model.lm_head, model.fp32_layers)
    prompt = W.synth_tokens(1, c.vocab_size, 5)
    ids, _, _ = ref.generate(prompt, 16)
    tokens = np.concatenate([prompt, np.array(ids[:-1], np.int32)])
    kv = oracle.orc().orc_kv_elements(oracle.C.byref(oracle.OrcConfig(**cfg)))
    hidden, keys, values = ref.decode_trace(tokens, kv_elements=kv)
    logits = ref.logits(hidden[len(prompt) - 1])
    storage = ref.storage_bytes()
    ref.close()
    np.savez_compressed(
        os.path.join(HERE, f"tiny_{tag}.npz"), prompt=prompt,
        ids=np.array(ids, np.int32), tokens=tokens, hidden=hidden,
        logits=logits, keys=keys, values=values,
        digest=np.array(weight_digest(model)),
        storage_bytes=np.int64(storage))


NORM_SEED = 9


def write_tiny_norms(qtype, tag):
    """As write_tiny, with seeded non-unit norm weights (attention and ffn
    norm of both layers, final norm: N(1, 0.25^2), workloads.seeded_norms):
    the three norms of src/quant_model.cpp:182-190 and
    src/generate.cpp:197-198 each enter the reference's output."""
    model = W.build("tiny", qtype, 0, keep_fp32=True, norm_seed=NORM_SEED)
    c = model.config
    cfg = {n: getattr(c, n) for n, _ in oracle.OrcConfig._fields_}
    ref = oracle.RefModel(cfg, qtype, model.embeddings, model.final_norm,
                          model.lm_head, model.fp32_layers, norms=model.norms)
    prompt = W.synth_tokens(1, c.vocab_size, 5)
    ids, _, _ = ref.generate(prompt, 16)
    tokens = np.concatenate([prompt, np.array(ids[:-1], np.int32)])
    kv = oracle.orc().orc_kv_elements(oracle.C.byref(oracle.OrcConfig(**cfg)))
    hidden, keys, values = ref.decode_trace(tokens, kv_elements=kv)
    logits = ref.logits(hidden[len(prompt) - 1])
    ref.close()
    np.savez_compressed(
        os.path.join(HERE, f"tiny_norms_{tag}.npz"), prompt=prompt,
        ids=np.array(ids, np.int32), tokens=tokens, hidden=hidden,
        logits=logits, keys=keys, values=values, norm_seed=np.int64(NORM_SEED),
        digest=np.array(weight_digest(model)))


def write_tinyllama():
    model, prompt, gen = W.build_run("tinyllama_int4")
    c = model.config
    cfg = {n: getattr(c, n) for n, _ in oracle.OrcConfig._fields_}
    layers = (model.layer_fp32(l) for l in range(c.layers))
    ref = oracle.RefModel(cfg, INT4, model.embeddings, model.final_norm,
                          model.lm_head, layers)
    ids, _, _ = ref.generate(prompt, gen, threads=8)
    storage = ref.storage_bytes()
    ref.close()
    with open(os.path.join(HERE, "tinyllama_int4.json"), "w") as f:
        json.dump({"run": "tinyllama_int4", "prompt": prompt.tolist(),
                   "ids": ids, "digest": weight_digest(model),
                   "storage_bytes": storage}, f, indent=1)


SAMPLING = [(0.7, 0.9, 42), (1.0, 1.0, 7), (0.3, 0.5, 1), (2.0, 0.95, 123)]


def write_sampled():
    """The reference's sampled ids for a few (temperature, top_p, seed)."""
    runs = []
    for name, tag in (("tiny_int8", "tiny"), ("tinyllama_int4", "tinyllama")):
        model, prompt, _ = W.build_run(name)
        ref = oracle.RefModel.from_quantized(model)
        for temperature, top_p, seed in SAMPLING:
            ids = ref.generate_sampled(prompt, 16, temperature, top_p, seed,
                                       threads=min(8, os.cpu_count() or 1))
            runs.append({"run": name, "prompt": prompt.tolist(),
                         "temperature": temperature, "top_p": top_p,
                         "seed": seed, "ids": ids})
        ref.close()
    with open(os.path.join(HERE, "sampled.json"), "w") as f:
        json.dump(runs, f, indent=1)


FP32_RUNS = [("tiny", 21, False), ("tiny", 23, True), ("step_gqa2", 22, False)]


def write_fp32():
    for shape, seed, tied in FP32_RUNS:
        model = W.build_fp32(shape, seed, max_seq=64, norm_seed=seed + 100, tied=tied)
        c = model.config
        cfg = (oracle.C.c_size_t * 9)(*[getattr(c, n) for n, _ in oracle.OrcConfig._fields_])
        h = oracle.C.c_void_p()
        oracle.check(oracle.ref().ref_fmodel_create(
            cfg, int(tied), oracle.ptr(model.embeddings), oracle.ptr(model.final_norm),
            None if tied else oracle.ptr(model.lm_head), oracle.C.byref(h)))
        for i, w in enumerate(model.layers):
            oracle.check(oracle.ref().ref_fmodel_add_layer(
                h, *[oracle.ptr(np.ascontiguousarray(w[n])) for n in oracle.PROJECTIONS],
                oracle.ptr(model.norms[i][0]), oracle.ptr(model.norms[i][1])))
        prompt = W.synth_tokens(seed, c.vocab_size, 6)
        tokens = W.synth_tokens(seed + 1, c.vocab_size, 4)
        kv = oracle.orc().orc_kv_elements(oracle.C.byref(oracle.OrcConfig(
            **{n: getattr(c, n) for n, _ in oracle.OrcConfig._fields_})))
        rows = np.zeros((6, c.dim), np.float32)
        hidden = np.zeros((4, c.dim), np.float32)
        keys, values = np.zeros(kv, np.float32), np.zeros(kv, np.float32)
        oracle.check(oracle.ref().ref_fmodel_run(
            h, oracle.ptr(prompt), 6, oracle.ptr(tokens), 4, 1, oracle.ptr(rows),
            oracle.ptr(hidden), oracle.ptr(keys), oracle.ptr(values)), "ref_fmodel_run")
        oracle.ref().ref_fmodel_free(h)
        tag = f"fp32_{shape}{'_tied' if tied else ''}"
        np.savez_compressed(os.path.join(HERE, f"{tag}.npz"), prompt=prompt, tokens=tokens,
                            rows=rows, hidden=hidden, keys=keys, values=values,
                            seed=np.int64(seed), tied=np.int64(tied))


def kv_sample(c, n):
    """(layer, kv head, position) rows kept from a long run's cache."""
    kvh = c.kv_heads or c.heads
    return np.array([(l, h, p) for l in sorted({0, c.layers // 2, c.layers - 1})
                     for h in sorted({0, kvh - 1})
                     for p in sorted({0, n // 2, n - 1})], np.int64)


def write_long(name):
    """A long-prompt run through the reference's own path over the product
    quantiser's storage (bit-identical to QuantizedMatrix::quantize, pinned
    by quant.npz): its greedy generate_tokens_cached ids, and from a
    decode trace of the prompt the last hidden state and sampled K/V rows."""
    model, prompt, gen = W.build_run(name)
    c = model.config
    cfg = {n: getattr(c, n) for n, _ in oracle.OrcConfig._fields_}
    kv = oracle.orc().orc_kv_elements(oracle.C.byref(oracle.OrcConfig(**cfg)))
    ref = oracle.RefModel.from_quantized(model)
    threads = min(8, os.cpu_count() or 1)
    hidden, keys, values = ref.decode_trace(prompt, threads, kv_elements=kv)
    ids, pre, dec = ref.generate(prompt, gen, threads=threads)
    storage = ref.storage_bytes()
    ref.close()
    rows = kv_sample(c, len(prompt))
    kvh = c.kv_heads or c.heads
    offs = [((l * kvh + h) * c.max_seq + p) * c.head_dim for l, h, p in rows]
    k_rows = np.stack([keys[o:o + c.head_dim] for o in offs])
    v_rows = np.stack([values[o:o + c.head_dim] for o in offs])
    np.savez_compressed(
        os.path.join(HERE, f"{name}.npz"), prompt=prompt,
        ids=np.array(ids, np.int32), hidden=hidden[-1], kv_index=rows,
        keys=k_rows, values=v_rows, digest=np.array(weight_digest(model)),
        storage_bytes=np.int64(storage))
    print(f"{name}: {len(ids)} ids, prefill {pre:.1f} s, decode {dec:.1f} s "
          f"({threads} threads)", flush=True)


def copy_fixtures():
    for name in ("tiny-llama2.bin", "tiny-llama2-shared.bin"):
        shutil.copyfile(os.path.join(REFERENCE, "tests", "fixtures", name),
                        os.path.join(HERE, name))


def main():
    if not oracle.ref_available():
        sys.exit("oracle/_ref/libnutref.so is not built: make -C oracle ref")
    if "--only-sampled" in sys.argv:
        write_sampled()
        return
    if "--only-fp32" in sys.argv:
        write_fp32()
        return
    if "--only-norms" in sys.argv:
        write_tiny_norms(INT8, "int8")
        write_tiny_norms(INT4, "int4")
        return
    if "--only-long" in sys.argv:
        for name in ("tinyllama_int8_2k", "llama7b_int4"):
            write_long(name)
        return
    write_quant()
    write_quant_errors()
    write_tiny(INT8, "int8")
    write_tiny(INT4, "int4")
    write_tiny_norms(INT8, "int8")
    write_tiny_norms(INT4, "int4")
    copy_fixtures()
    write_fp32()
    if "--skip-tinyllama" not in sys.argv:
        write_tinyllama()
        write_sampled()
    if "--long" in sys.argv:
        for name in ("tinyllama_int8_2k", "llama7b_int4"):
            write_long(name)


if __name__ == "__main__":
    main()
