"""Synthetic workloads: the decoder shapes and seeded random-init weights.

The reference loads checkpoints; these configurations replace them with
seeded N(0, 0.02) fp32 weights (norm weights 1.0, the reference's default,
src/attention.cpp:37-38), quantised by the product quantiser:

  tiny       dim 64, 2 layers, 4/2 heads (hd 16), ffn 172, vocab 256,
             max_seq 64, INT8, weights seed 0, prompt seed 1 (5 ids)
  tinyllama  dim 2048, 22 layers, 32/4 heads (hd 64), ffn 5632, vocab 32000,
             INT4 (or INT8), seed 3
  llama7b    dim 4096, 32 layers, 32/32 heads (hd 128), ffn 11008,
             vocab 32000, INT4, seed 4

Streams of nut_synth_normal: embeddings 1, classifier 2, projection p of
layer l: 16 + 8 l + p (p in query, key, value, output, gate, up, down).
eos_token is 1, as the llama2.c adapter sets (src/llama2.cpp:222-223).

``build(..., norm_seed=s)`` replaces the unit norm weights with seeded
N(1, 0.25^2) vectors (attention and ffn norm of every layer, and the final
norm), so that tests see every norm weight enter the computation.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

from . import (INT4, INT8, PROJECTIONS, Config, DeviceModel, projection_shapes,
               quantize, synth_normal, synth_tokens)

SIGMA = 0.02
STREAM_EMBED, STREAM_CLASSIFIER = 1, 2


def stream_of(layer, projection):
    return 16 + 8 * layer + PROJECTIONS.index(projection)


SHAPES = {
    "tiny": dict(layers=2, heads=4, dim=64, head_dim=16, ffn_dim=172,
                 vocab_size=256, max_seq=64, eos_token=1, kv_heads=2),
    "tinyllama": dict(layers=22, heads=32, dim=2048, head_dim=64,
                      ffn_dim=5632, vocab_size=32000, max_seq=2048,
                      eos_token=1, kv_heads=4),
    "llama7b": dict(layers=32, heads=32, dim=4096, head_dim=128,
                    ffn_dim=11008, vocab_size=32000, max_seq=640,
                    eos_token=1, kv_heads=32),
    # the Llama-2-7B widths with two layers, for oracle parity at full width
    "llama7b_2l": dict(layers=2, heads=32, dim=4096, head_dim=128,
                       ffn_dim=11008, vocab_size=32000, max_seq=640,
                       eos_token=1, kv_heads=32),
    # small shapes for the step-kernel parity tests: head_dim 128 with one
    # query head per KV head, head_dim 64 with four and with two
    "step_mha128": dict(layers=2, heads=2, dim=256, head_dim=128, ffn_dim=512,
                        vocab_size=512, max_seq=1200, eos_token=1, kv_heads=2),
    "step_gqa4": dict(layers=2, heads=8, dim=512, head_dim=64, ffn_dim=768,
                      vocab_size=512, max_seq=1200, eos_token=1, kv_heads=2),
    "step_gqa2": dict(layers=2, heads=4, dim=256, head_dim=64, ffn_dim=512,
                      vocab_size=512, max_seq=1200, eos_token=1, kv_heads=2),
}

# The named runs: shape, quant type, weight seed, prompt seed, prompt
# length, generated tokens, max_seq override.
RUNS = {
    "tiny_int8": ("tiny", INT8, 0, 1, 5, 16, None),
    "tinyllama_int4": ("tinyllama", INT4, 3, 3, 5, 16, None),
    "tinyllama_int8_2k": ("tinyllama", INT8, 3, 3, 2048, 128, 2176),
    "llama7b_int4": ("llama7b", INT4, 4, 4, 512, 128, None),
}

# Standalone matvec shapes (out x in), weights seed 2.
MATVEC_SHAPES = [(2048, 2048), (256, 2048), (5632, 2048), (2048, 5632),
                 (4096, 4096)]
MATVEC_SEED = 2


def make_config(shape, max_seq=None):
    d = dict(SHAPES[shape])
    if max_seq is not None:
        d["max_seq"] = max_seq
    return Config(**d)


@dataclass
class SynthModel:
    """Host copy of a synthetic QuantizedModelWeights."""

    config: Config
    qtype: int
    seed: int
    embeddings: np.ndarray
    final_norm: np.ndarray
    lm_head: np.ndarray
    layers: list = field(default_factory=list)  # name -> (data, scales, r, c)
    # per layer (attention_norm, ffn_norm); None means all ones
    norms: list | None = None

    def layer_fp32(self, layer):
        """The layer's fp32 projections, regenerated from the seed."""
        out = {}
        for name, (rows, cols) in projection_shapes(self.config).items():
            out[name] = synth_normal(self.seed, stream_of(layer, name),
                                     rows * cols, SIGMA).reshape(rows, cols)
        return out

    def layer_norms(self, layer):
        """(attention_norm, ffn_norm) of a layer."""
        if self.norms is not None:
            return self.norms[layer]
        ones = np.ones(self.config.dim, np.float32)
        return ones, ones

    def to_device(self):
        m = DeviceModel(self.config, self.qtype)
        m.set_globals(self.embeddings, self.final_norm, self.lm_head)
        for i, mats in enumerate(self.layers):
            m.set_layer(i, mats, *self.layer_norms(i))
        return m

    def weight_bytes_per_token(self, screened=False):
        """Bytes of weights one decode token streams: packed weights + fp16
        scales of every projection, the classifier, the 2L+1 norm vectors
        and one embedding row. The classifier is the fp32 matrix, or with
        `screened` what the token kernels' screened argmax reads instead:
        its INT8 block-32 copy, codes and fp16 scales (the few fp32 rows it
        recomputes are not counted)."""
        c = self.config
        linear = sum(d.nbytes + s.nbytes for mats in self.layers
                     for (d, s, *_rest) in mats.values())
        classifier = (c.vocab_size * (c.dim + c.dim // 16) if screened
                      else c.vocab_size * c.dim * 4)
        return (linear + classifier +
                (2 * c.layers + 1) * c.dim * 4 + c.dim * 4)


def seeded_norms(seed, dim, layers):
    """Per-layer (attention, ffn) norm weights and a final norm, N(1, 0.25^2)
    from numpy's default_rng(seed)."""
    rng = np.random.default_rng(seed)
    draw = lambda: (1.0 + 0.25 * rng.standard_normal(dim)).astype(np.float32)  # noqa: E731
    per_layer = [(draw(), draw()) for _ in range(layers)]
    return per_layer, draw()


def build(shape, qtype, seed, max_seq=None, keep_fp32=False, norm_seed=None):
    """Generate and quantise a synthetic model (host arrays); norm_seed
    draws non-unit norm weights (seeded_norms)."""
    cfg = make_config(shape, max_seq)
    n = cfg.vocab_size * cfg.dim
    emb = synth_normal(seed, STREAM_EMBED, n, SIGMA).reshape(cfg.vocab_size,
                                                            cfg.dim)
    head = synth_normal(seed, STREAM_CLASSIFIER, n, SIGMA).reshape(
        cfg.vocab_size, cfg.dim)
    model = SynthModel(cfg, qtype, seed, emb, np.ones(cfg.dim, np.float32),
                       head)
    if norm_seed is not None:
        model.norms, model.final_norm = seeded_norms(norm_seed, cfg.dim,
                                                     cfg.layers)
    fp32 = []
    for layer in range(cfg.layers):
        weights = model.layer_fp32(layer)
        mats = {}
        for name, w in weights.items():
            data, scales = quantize(w, qtype)
            mats[name] = (data, scales, w.shape[0], w.shape[1])
        model.layers.append(mats)
        if keep_fp32:
            fp32.append(weights)
    if keep_fp32:
        model.fp32_layers = fp32
    return model


def build_run(name, keep_fp32=False):
    shape, qtype, seed, prompt_seed, prompt_len, gen, max_seq = RUNS[name]
    model = build(shape, qtype, seed, max_seq, keep_fp32)
    prompt = synth_tokens(prompt_seed, model.config.vocab_size, prompt_len)
    return model, prompt, gen


# fp32 model path (ModelWeights, decode_token / prefill_tokens): the same
# streams as the quantised models, each projection drawn as its reference
# [in x out] Matrix.
FP32_SHAPES = {"query": lambda c: (c.dim, c.dim), "key": lambda c: (c.dim, c.kv_dim),
               "value": lambda c: (c.dim, c.kv_dim), "output": lambda c: (c.dim, c.dim),
               "gate": lambda c: (c.dim, c.ffn_dim), "up": lambda c: (c.dim, c.ffn_dim),
               "down": lambda c: (c.ffn_dim, c.dim)}


@dataclass
class SynthFModel:
    """Host copy of a synthetic fp32 ModelWeights ([in x out] projections)."""

    config: Config
    seed: int
    tied: bool
    embeddings: np.ndarray
    final_norm: np.ndarray
    lm_head: np.ndarray
    layers: list
    norms: list

    def to_device(self):
        from . import DeviceFModel
        m = DeviceFModel(self.config, self.tied)
        m.set_globals(self.embeddings, self.final_norm,
                      None if self.tied else self.lm_head)
        for i, w in enumerate(self.layers):
            m.set_layer(i, w, *self.norms[i])
        return m


def build_fp32(shape, seed, max_seq=None, norm_seed=None, tied=False):
    cfg = make_config(shape, max_seq)
    n = cfg.vocab_size * cfg.dim
    emb = synth_normal(seed, STREAM_EMBED, n, SIGMA).reshape(cfg.vocab_size, cfg.dim)
    head = emb if tied else synth_normal(seed, STREAM_CLASSIFIER, n, SIGMA).reshape(
        cfg.vocab_size, cfg.dim)
    layers = []
    for layer in range(cfg.layers):
        w = {}
        for name in PROJECTIONS:
            rows, cols = FP32_SHAPES[name](cfg)
            w[name] = synth_normal(seed, stream_of(layer, name), rows * cols,
                                   SIGMA).reshape(rows, cols)
        layers.append(w)
    if norm_seed is None:
        ones = np.ones(cfg.dim, np.float32)
        norms, final = [(ones, ones)] * cfg.layers, ones
    else:
        norms, final = seeded_norms(norm_seed, cfg.dim, cfg.layers)
    return SynthFModel(cfg, seed, tied, emb, final, head, layers, norms)

