"""nutllm_amd.phase_timeline.summarise on a synthetic timeline whose marks
sit at known offsets: every segment, exchange and skew comes back exactly."""
import numpy as np

from nutllm_amd import phase_timeline as pt

# offset of each of the 13 marks within a layer, microseconds
OFFS = [0.0, 1.0, 1.5, 3.0, 5.0, 5.5, 6.0, 8.5, 10.5, 10.75, 13.0, 14.0, 14.5]
LAYER = 17.0
CLASSIFY = 40.0


# the iteration's head: classifier input staged, pass done, token known
HEAD_OFFS = [0.0, 2.5, 30.0, 38.0]


def synthetic(wgs=8, iters=6, layers=3):
    t = np.zeros((wgs, iters, 4 + 13 * layers))
    for it in range(iters):
        start = it * (CLASSIFY + layers * LAYER)
        for w in range(wgs):
            for k, o in enumerate(HEAD_OFFS):
                t[w, it, k] = start + o
            for l in range(layers):
                for k, o in enumerate(OFFS):
                    t[w, it, 4 + 13 * l + k] = start + CLASSIFY + l * LAYER + o
            # one late publisher per publish mark: +0.4 us
            if w == wgs - 1:
                for l in range(layers):
                    for k in (1, 5, 8, 11):
                        t[w, it, 4 + 13 * l + k] += 0.4
    return t


def test_summarise_segments_and_exchanges():
    out = pt.summarise(synthetic(), 3)
    assert out["A rows"] == OFFS[1] - OFFS[0]
    assert out["B attention"] == OFFS[4] - OFFS[3]
    assert out["C rows"] == OFFS[8] - OFFS[7]
    assert out["D dma issue"] == OFFS[12] - OFFS[11]
    # ready (median workgroup) minus the last publish, which is 0.4 late
    assert np.isclose(out["exchange q/k/v"], OFFS[3] - OFFS[1] - 0.4)
    assert np.isclose(out["exchange act"], OFFS[10] - OFFS[8] - 0.4)
    assert np.isclose(out["exchange h after W2"], LAYER - OFFS[11] - 0.4)
    assert np.isclose(out["skew h after Wo"], 0.4)
    assert out["layer"] == LAYER
    assert out["classifier + argmax"] == CLASSIFY
    assert out["classifier input (h exchange)"] == HEAD_OFFS[1]
    assert out["classifier pass"] == HEAD_OFFS[2] - HEAD_OFFS[1]
    assert out["argmax exchange"] == HEAD_OFFS[3] - HEAD_OFFS[2]
    assert out["skew classifier pass"] == 0.0
