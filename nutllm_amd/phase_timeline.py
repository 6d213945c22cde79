"""Per-phase timeline of the cooperative token kernel.

    python3 -m nutllm_amd.phase_timeline [workload]

Runs one greedy generate of the workload (default ``tinyllama_int4``) to
warm up, then a second one with every workgroup stamping the 100 MHz
real-time clock at 4 marks per iteration and 13 per layer
(``record_timeline(2)``), and prints
medians over workgroups, layers and the steady iterations (the first two
and the last are left out):

- each compute segment of a layer (A: rmsnorm + Q/K/V rows + RoPE; B:
  attention, then the Wo rows; C: rmsnorm + gate/up rows; D: W2 rows), and
  the weight-DMA issue after each publish;
- each exchange: from the last workgroup's publish to the median
  workgroup holding the input (``ready``), and the publish skew (last
  publish minus median publish).

Columns 0-3 of ``timeline()`` are the iteration start, the classifier's
input staged (after the h exchange and the final rmsnorm), the classifier
pass done and the token known (after the argmax exchange); mark k of layer
l is column 4 + 13 l + k: 0 A input
ready, 1 A published, 2 DMA issued, 3 B input ready, 4 attention done,
5 B published, 6 DMA issued, 7 C input ready, 8 C published, 9 DMA
issued, 10 D input ready, 11 D published, 12 next DMA issued.

Wide multi-head shapes run the kernel of wide.hip, whose marks are: 0 A
input ready, 1 q/k/v published, 2 partial scores published (V and Wo
rows issued), 3 context published, 4 Wo input ready, 5 Wo published,
6 C input ready (gate/up rows issued before the wait), 7 C published,
8 D input ready (W2 rows issued before the wait), 9 D published, 10 and
12 layer end (the next layer's q/k/v rows are issued before its wait);
the printout is then the median of each segment between consecutive
marks.
"""
import sys

import numpy as np

from . import workloads

MARKS = 13
HEAD = 4  # iteration start, classifier input, classifier pass, token known
SEGMENTS = [("A rows", 0, 1), ("A dma issue", 1, 2), ("B attention", 3, 4),
            ("B Wo rows", 4, 5), ("B dma issue", 5, 6), ("C rows", 7, 8),
            ("C dma issue", 8, 9), ("D rows", 10, 11), ("D dma issue", 11, 12)]
# (name, publish mark, ready mark, the ready mark's layer offset)
EXCHANGES = [("q/k/v", 1, 3, 0), ("h after Wo", 5, 7, 0), ("act", 8, 10, 0),
             ("h after W2", 11, 0, 1)]


def summarise(t, layers):
    """t: [workgroups, iterations, 4 + 13 layers] in microseconds."""
    its = range(2, t.shape[1] - 1)
    col = lambda l, k: HEAD + MARKS * l + k
    out = {}
    for name, a, b in SEGMENTS:
        d = [t[:, it, col(l, b)] - t[:, it, col(l, a)] for it in its for l in range(layers)]
        out[name] = float(np.median(np.concatenate(d)))
    for name, p, r, shift in EXCHANGES:
        ready, skew = [], []
        for it in its:
            for l in range(layers - shift):
                pub = t[:, it, col(l, p)]
                ready.append(np.median(t[:, it, col(l + shift, r)]) - pub.max())
                skew.append(pub.max() - np.median(pub))
        out["exchange " + name] = float(np.mean(ready))
        out["skew " + name] = float(np.mean(skew))
    lay = [np.median(t[:, it, col(l + 1, 0)] - t[:, it, col(l, 0)])
           for it in its for l in range(layers - 1)]
    out["layer"] = float(np.median(lay))
    classifier_parts(t, its, out)
    return out


def classifier_parts(t, its, out):
    """The iteration's head: the h exchange and final rmsnorm into the
    classifier, its pass (median workgroup), the spread of the pass's end
    (last minus median workgroup), the argmax exchange (last workgroup's
    pass end to the median workgroup knowing the token), and all of it up
    to layer 0's staged input."""
    med = lambda a, b: float(np.median([np.median(t[:, it, b] - t[:, it, a])  # noqa: E731
                                        for it in its]))
    out["classifier input (h exchange)"] = med(0, 1)
    out["classifier pass"] = med(1, 2)
    out["skew classifier pass"] = float(np.mean([t[:, it, 2].max() - np.median(t[:, it, 2])
                                                 for it in its]))
    out["argmax exchange"] = float(np.mean([np.median(t[:, it, 3]) - t[:, it, 2].max()
                                            for it in its]))
    out["classifier + argmax"] = med(0, HEAD)


WIDE_SEGMENTS = [("A issue + h exchange", -1, 0), ("A rows", 0, 1),
                 ("V/Wo issue + partial scores", 1, 2),
                 ("score exchange + softmax + context", 2, 3),
                 ("context exchange", 3, 4), ("Wo rows", 4, 5),
                 ("gate/up issue + h exchange", 5, 6), ("gate/up rows", 6, 7),
                 ("W2 issue + act exchange", 7, 8), ("W2 rows", 8, 9),
                 ("layer end", 9, 12)]


def summarise_wide(t, layers):
    """The wide kernel's segments: mark -1 is the previous layer's end."""
    its = range(2, t.shape[1] - 1)
    col = lambda l, k: HEAD + MARKS * l + k
    out = {}
    for name, a, b in WIDE_SEGMENTS:
        d = []
        for it in its:
            for l in range(1 if a < 0 else 0, layers):
                start = t[:, it, col(l - 1, 12)] if a < 0 else t[:, it, col(l, a)]
                d.append(t[:, it, col(l, b)] - start)
        out[name] = float(np.median(np.concatenate(d)))
    lay = [np.median(t[:, it, col(l + 1, 0)] - t[:, it, col(l, 0)])
           for it in its for l in range(layers - 1)]
    out["layer"] = float(np.median(lay))
    classifier_parts(t, its, out)
    return out


def main(argv):
    name = argv[1] if len(argv) > 1 else "tinyllama_int4"
    model, prompt, gen = workloads.build_run(name)
    dev = model.to_device()
    try:
        dev.generate(prompt, gen)
        dev.record_timeline(2)
        ids, _ = dev.generate(prompt, gen)
        n = len(ids)
        t = dev.timeline(n)
        ms = dev.last_decode_ms()
    finally:
        # the model's graph, stream and buffers go before the HIP runtime's
        # own exit handlers run
        dev.close()
    print(f"{name}: {n} tokens, {ms * 1e3 / n:.1f} us per token (HIP events)")
    c = model.config
    wide = c.kv_heads in (0, c.heads) and c.head_dim == 128
    summary = summarise_wide if wide else summarise
    for key, v in summary(t, c.layers).items():
        print(f"  {key:24s} {v:6.2f} us")


if __name__ == "__main__":
    main(sys.argv)
