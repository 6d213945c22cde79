"""Reader of llama2.c checkpoints for the tests (src/llama2.cpp:199-296).

Header: seven int32 (dim, ffn_dim, layers, heads, kv_heads, vocab, max_seq);
a negative vocab means an unshared classifier follows the weights. Then
fp32 arrays in this order: embeddings [vocab][dim], attention norms
[L][dim], Wq [L][dim][dim], Wk and Wv [L][kv_dim][dim], Wo [L][dim][dim],
ffn norms [L][dim], W1 (gate) [L][ffn][dim], W2 (down) [L][dim][ffn],
W3 (up) [L][ffn][dim], final norm [dim], RoPE tables [max_seq][head_dim]
(unused), classifier [vocab][dim] when unshared. eos_token is 1
(src/llama2.cpp:222-223).
"""
from __future__ import annotations

import numpy as np


def load(path):
    header = np.fromfile(path, np.int32, 7)
    dim, ffn, layers, heads, kv_heads, vocab_raw, max_seq = map(int, header)
    shared = vocab_raw > 0
    vocab = abs(vocab_raw)
    head_dim = dim // heads
    kv_dim = kv_heads * head_dim
    flat = np.fromfile(path, np.float32, offset=28)
    pos = 0

    def take(*shape):
        nonlocal pos
        n = int(np.prod(shape))
        out = flat[pos:pos + n].reshape(shape)
        pos += n
        return out

    w = {"embeddings": take(vocab, dim),
         "attention_norm": take(layers, dim),
         "query": take(layers, dim, dim),
         "key": take(layers, kv_dim, dim),
         "value": take(layers, kv_dim, dim),
         "output": take(layers, dim, dim),
         "ffn_norm": take(layers, dim),
         "gate": take(layers, ffn, dim),
         "down": take(layers, dim, ffn),
         "up": take(layers, ffn, dim),
         "final_norm": take(dim)}
    take(max_seq, head_dim)
    w["classifier"] = w["embeddings"] if shared else take(vocab, dim)
    assert pos == flat.size, "size does not match the configuration"
    config = dict(layers=layers, heads=heads, dim=dim, head_dim=head_dim,
                  ffn_dim=ffn, vocab_size=vocab, max_seq=max_seq,
                  eos_token=1, kv_heads=kv_heads)
    return config, w, shared


def write(path, config, w, shared=False):
    """Write a llama2.c checkpoint (the layout load() reads) from a config
    dict and a weights dict keyed as load() returns them; the RoPE tables
    are written as zeros (the loaders skip them)."""
    c = config
    head_dim = c["dim"] // c["heads"]
    vocab = c["vocab_size"] if shared else -c["vocab_size"]
    header = np.array([c["dim"], c["ffn_dim"], c["layers"], c["heads"],
                       c["kv_heads"], vocab, c["max_seq"]], np.int32)
    parts = [w["embeddings"], w["attention_norm"], w["query"], w["key"],
             w["value"], w["output"], w["ffn_norm"], w["gate"], w["down"],
             w["up"], w["final_norm"],
             np.zeros((c["max_seq"], head_dim), np.float32)]
    if not shared:
        parts.append(w["classifier"])
    with open(path, "wb") as f:
        f.write(header.tobytes())
        for p in parts:
            f.write(np.ascontiguousarray(p, np.float32).tobytes())
