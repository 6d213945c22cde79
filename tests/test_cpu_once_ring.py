"""The ring of write-once exchange slices of the cooperative token kernels.

persistent.hip and wide.hip publish every exchange of a (token, layer) step
into write-once words of a slice of a ring (persistent.hpp: kOnceRing,
once_slice); a producer sets its words of step u back to unset at the start
of phase C of step u + 2 (before its take of that step's h after Wo), and
that take retires those stores. This test
replays the kernels' per-workgroup phase order as a happens-before graph
(program order inside a workgroup; an edge from each publish to every take
that reads it) and checks, for every word, that

1. every consumer's take of step u happens before the producer re-arms it;
2. the re-arm is retired before any consumer's first poll of the slice's
   next use (step u + kOnceRing);
3. the producer re-arms before it publishes into the slice again;
4. the ring's size does not depend on the number of tokens.

It is run for the fused and split attention of persistent.hip and for
wide.hip, for the generate loop (classifier first in every iteration) and
for the prefill loop, and shows that a ring of two slices would not do
with this placement, and that a re-arm one take too early is caught.
"""
import itertools
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

WGS = 8            # modelled workgroups
GROUPS = 2         # q/k/v exchanged inside a group (persistent.hip)


def group(w):
    return w // (WGS // GROUPS)


def phases(kind, classify, it, l):
    """Events of one workgroup in step (it, l), in program order:
    ("take", X) reads every producer's words of exchange X (X in the
    group for "qkv"), ("pub", X) publishes its own, ("rearm",) sets its
    words of the previous step back to unset; the classifier's argmax
    exchange ("arg") uses tagged words outside the ring."""
    ev = []
    if l == 0 and classify and it > 0:
        ev += [("take", "dn", -1), ("pub", "arg", 0), ("take", "arg", 0)]
    elif l > 0:
        ev += [("take", "dn", -1)]
    if kind == "fused":
        ev += [("pub", "qkv", 0), ("take", "qkv", 0), ("pub", "wo", 0), ("take", "wo", 0)]
    elif kind == "split":
        ev += [("pub", "qkv", 0), ("take", "qkv", 0), ("pub", "part", 0), ("take", "part", 0),
               ("pub", "ctx", 0), ("take", "ctx", 0), ("pub", "wo", 0), ("take", "wo", 0)]
    else:  # wide: partial scores (tagged), context, h after Wo
        ev += [("pub", "score", 0), ("take", "score", 0), ("pub", "ctx", 0),
               ("take", "ctx", 0), ("pub", "wo", 0), ("take", "wo", 0)]
    ev += [("pub", "act", 0), ("take", "act", 0), ("pub", "dn", 0)]
    # the re-arm of step u - LAG's words, right before the take REARM_BEFORE
    ev.insert(ev.index(("take", REARM_BEFORE, 0)), ("rearm",))
    return ev


# The kernels: at the start of phase C of step u + 2, before its take of
# the h after Wo, the words of step u (LAG 2) go back to unset.
REARM_BEFORE, LAG = "wo", 2


RING_EXCHANGES = {"fused": ("qkv", "wo", "act", "dn"),
                  "split": ("qkv", "ctx", "wo", "act", "dn"),
                  "wide": ("ctx", "wo", "act", "dn")}


def consumers(x, producer):
    """Workgroups that read `producer`'s words of exchange x: q/k/v, split
    attention's partials and the wide kernel's partial scores stay inside
    a group of workgroups (a KV head's, a head's); the rest are read by
    every workgroup."""
    if x in ("qkv", "part", "score"):
        return [w for w in range(WGS) if group(w) == group(producer)]
    return list(range(WGS))


def build(kind, classify, iters, layers):
    """Nodes (w, u, k, 0) for event k of workgroup w in step u; a take has
    a second node (w, u, k, 1): its first poll is (.., 0), its completion
    (every polled word set, then s_waitcnt vmcnt(0) and a barrier) is
    (.., 1), and the publishes it reads lead there."""
    steps = iters * layers
    events = {}
    succ = {}

    def edge(a, b):
        succ.setdefault(a, set()).add(b)

    for w in range(WGS):
        prev = None
        for u in range(steps):
            it, l = divmod(u, layers)
            ev = phases(kind, classify, it, l)
            events[u] = ev
            for k, e in enumerate(ev):
                node = (w, u, k, 0)
                if prev is not None:
                    edge(prev, node)
                prev = node
                if e[0] == "take":
                    edge(node, (w, u, k, 1))
                    prev = (w, u, k, 1)
    # publish -> take edges; ("take", "dn", -1) reads the previous step
    for u in range(steps):
        for k, e in enumerate(events[u]):
            if e[0] != "take":
                continue
            x, back = e[1], e[2]
            src = u + back
            if src < 0:
                continue
            kp = next(i for i, f in enumerate(events[src]) if f[0] == "pub" and f[1] == x)
            for q in range(WGS):
                for p in range(WGS):
                    if q in consumers(x, p):
                        edge((p, src, kp, 0), (q, u, k, 1))
    return events, succ


def reach(succ, a, b, memo):
    key = (a, b)
    if key in memo:
        return memo[key]
    seen, stack = {a}, [a]
    found = False
    while stack:
        n = stack.pop()
        if n == b:
            found = True
            break
        for m in succ.get(n, ()):
            if m not in seen and m[1] <= b[1]:
                seen.add(m)
                stack.append(m)
    memo[key] = found
    return found


def violations(kind, classify, ring, iters=3, layers=3):
    events, succ = build(kind, classify, iters, layers)
    steps = iters * layers
    memo = {}
    bad = []
    for u in range(steps):
        for x in RING_EXCHANGES[kind]:
            for p in range(WGS):
                # where step u's words of x are read, re-armed and retired
                takes = [(k, e) for uu in (u, u + 1) if uu < steps
                         for k, e in enumerate(events[uu])
                         if e[0] == "take" and e[1] == x and uu + e[2] == u]
                ur = u + LAG  # the step that re-arms step u's words
                if ur >= steps:
                    continue
                kr = next(i for i, e in enumerate(events[ur]) if e[0] == "rearm")
                # the next take retires the stores (its closing s_waitcnt)
                kret = next(i for i in range(kr + 1, len(events[ur]))
                            if events[ur][i][0] == "take")
                # 1: every read of the words completes before the re-arm
                for q in consumers(x, p):
                    for k, e in takes:
                        uu = u if e[2] == 0 else u + 1
                        if not reach(succ, (q, uu, k, 1), (p, ur, kr, 0), memo):
                            bad.append(("read after re-arm", kind, x, u, p, q))
                # 2: the re-arm is retired (the next take completes) before
                # the first poll of the slice's next use
                retired = (p, ur, kret, 1)
                nxt = u + ring
                if nxt >= steps:
                    continue
                # 3: the producer re-arms before it publishes into the slice
                # again (program order)
                for k, e in enumerate(events[nxt]):
                    if e[0] == "pub" and e[1] == x and (ur > nxt or (ur == nxt and kr > k)):
                        bad.append(("re-arm after the next publish", kind, x, u, p, p))
                for q in consumers(x, p):
                    for k, e in enumerate(events[nxt]):
                        if e[0] == "take" and e[1] == x and e[2] == 0:
                            if not reach(succ, retired, (q, nxt, k, 0), memo):
                                bad.append(("poll before re-arm retired", kind, x, u, p, q))
                    if nxt + 1 < steps:
                        for k, e in enumerate(events[nxt + 1]):
                            if e[0] == "take" and e[1] == x and e[2] == -1:
                                if not reach(succ, retired, (q, nxt + 1, k, 0), memo):
                                    bad.append(("poll before re-arm retired", kind, x, u, p,
                                                q))
    return bad


def ring_size():
    src = open(os.path.join(ROOT, "nutllm_amd", "csrc", "persistent.hpp")).read()
    m = re.search(r"constexpr int kOnceRing = (\d+);", src)
    assert m
    return int(m.group(1))


@pytest.mark.parametrize("kind,classify", list(itertools.product(
    ["fused", "split", "wide"], [True, False])))
def test_ring_protocol_holds(kind, classify):
    ring = ring_size()
    assert violations(kind, classify, ring) == []


def with_placement(before, lag, fn):
    global REARM_BEFORE, LAG
    saved = REARM_BEFORE, LAG
    REARM_BEFORE, LAG = before, lag
    try:
        return fn()
    finally:
        REARM_BEFORE, LAG = saved


@pytest.mark.parametrize("kind", ["fused", "split", "wide"])
def test_a_ring_of_two_is_too_small_for_this_placement(kind):
    """With the re-arm two steps back, two slices would put the re-arm after
    the producer's own new words in the slice (and polls before it)."""
    bad = violations(kind, True, 2)
    assert any(b[0] == "re-arm after the next publish" for b in bad)


def test_the_one_step_placement_needs_three_in_the_prefill_loop():
    """Re-arming one step back at the start of phase D (before the take of
    act) works with three slices, and not with two in the prefill loop
    (nothing orders a consumer's first poll of step u + 2 after the re-arm
    when layer 0 takes no exchange)."""
    assert with_placement("act", 1, lambda: violations("fused", False, 3)) == []
    bad = with_placement("act", 1, lambda: violations("fused", False, 2))
    assert bad and all(b[0] == "poll before re-arm retired" for b in bad)
    assert with_placement("act", 1, lambda: violations("fused", True, 2)) == []


def test_rearm_one_take_too_early_is_caught():
    """Re-arming the previous step's words before the h after Wo of this
    step has been taken lets a slow consumer still be reading them."""
    bad = with_placement("wo", 1, lambda: violations("fused", True, 4))
    assert any(b[0] == "read after re-arm" for b in bad)


def test_ring_memory_is_independent_of_tokens():
    """token_once_floats(shape, wide) has no iteration count: the ring is
    kOnceRing step slices of token_once_stride words."""
    src = open(os.path.join(ROOT, "nutllm_amd", "csrc", "persistent.hpp")).read()
    m = re.search(r"inline size_t token_once_floats\(([^)]*)\)\s*\{\s*return ([^;]*);", src)
    assert m, "token_once_floats"
    assert "n_iter" not in m.group(1) and "layers" not in m.group(1)
    assert m.group(2).strip() == "kOnceRing * token_once_stride(s, wide)"
    call = open(os.path.join(ROOT, "nutllm_amd", "csrc", "model.cpp")).read()
    assert "token_once_floats(s, wide)" in call
