"""Ordering audit of the K/V cache rows the cooperative token kernels read.

The token kernels (nutllm_amd/csrc/persistent.hip, wide.hip) store each new
K/V row to the cache in phase A of every layer and stage earlier rows back
from the cache for attention. The reference reads exactly what
KVCache::store wrote (src/quant_model.cpp:45-108, src/kvcache.cpp:173-235);
on the device a row can be read by a workgroup on another XCD than its
writer's, in the same launch. This test replays the launch schedules of the
GPU tests and the bench workloads from the kernels' indexing (which
workgroup stores which dims of which row, which rows each workgroup stages
at each position), with workgroup b on XCD b % 8 (round-robin dispatch), and
classifies every staged row:

- written by an earlier launch: ordered by the kernel boundary (the end of
  a kernel releases, the start of the next acquires, at agent scope);
- written earlier in the same launch by the reading workgroup itself
  (the wide kernel's rule): program order on one CU;
- written earlier in the same launch by other workgroups: the writer's
  stores are agent-scope (sc1) and retired by its s_waitcnt vmcnt(0) before
  its next publish, every workgroup takes the writer's h-after-W2 words
  (an all-gather) in every layer before the next iteration reaches the
  staging, so the staging is ordered after the stores only if its load is
  itself agent-coherent (sc1 in the DMA's cache policy, read here from the
  source);
- flagged: anything else (a row of the current position, which must come
  from the exchange, or a row no launch wrote yet).
"""
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "nutllm_amd", "csrc")

GRID, XCDS = 256, 8
SC1, NT = 16, 2


def xcd(b):
    return b % XCDS


# ------------------------------------------------ token kernel indexing --
# TinyLlama shapes: 32 query heads over 4 KV heads of 64 dims.
HEADS, KVH, HD = 32, 4, 64
GROUP = HEADS // KVH
GQ, GR = GROUP * HD, GROUP * HD + 2 * HD  # q rows of a group; + its k, v rows
WGS_G = GRID // KVH
GR_WG = GR // WGS_G  # rows per workgroup in phase A (10)
SPLITS, PMAX = GRID // KVH, 64
FUSED_POSITIONS = {"int4": 48, "int8": 44}


def token_group(b, long):
    """(KV head group, index in the group) of workgroup b
    (persistent.hip: grp, gj)."""
    if long:
        return b // WGS_G, b % WGS_G
    return (b & 7) >> 1, ((b >> 3) << 1) | (b & 1)


def token_writes(b, long):
    """[(kv_head, which, dim)] the K (which 1) and V (which 2) dims workgroup
    b stores in phase A of every layer (persistent.hip: qkv_row, the
    store_coherent pair)."""
    g, gj = token_group(b, long)
    out = []
    for pair in range(GR_WG // 2):
        lr = gj * GR_WG + 2 * pair
        which = 0 if lr < GQ else 1 if lr < GQ + HD else 2
        d = lr % HD
        if which > 0:
            out += [(g, which, d), (g, which, d + 1)]
    return out


def token_reads(b, long, pos):
    """(kv_head, first row, end row) workgroup b stages from the cache at
    decode position pos: the group's KV head, rows [0, pos) in the fused
    attention; KV head b / SPLITS, rows [ap0, min(ap1, pos)) of its run
    with split attention (row pos itself comes from the q/k/v exchange)."""
    if not long:
        g, _ = token_group(b, long)
        return (g, 0, pos)
    n = pos + 1
    per = -(-n // SPLITS)
    ap0 = min(n, (b % SPLITS) * per)
    ap1 = min(n, ap0 + per)
    return (b // SPLITS, ap0, max(ap0, min(ap1, pos)))


# ------------------------------------------------- wide kernel indexing --
# Llama-2-7B shape: 32 heads (MHA) of 128 dims, 8 workgroups per head.
W_HEADS, W_HD = 32, 128
W_GW = GRID // W_HEADS
W_SLICE = W_HD // W_GW


def wide_writes(b):
    """The wide kernel's workgroup b stores dims [SLICE part, +SLICE) of
    head b % HEADS's K and V rows (wide.hip: head, part)."""
    head, part = b % W_HEADS, b // W_HEADS
    return [(head, which, W_SLICE * part + d) for which in (1, 2) for d in range(W_SLICE)]


def wide_reads(b, pos):
    """...and reads the same dims of rows [0, pos) (row pos from its own
    registers)."""
    head, part = b % W_HEADS, b // W_HEADS
    return (head, 0, pos), [(head, which, W_SLICE * part + d)
                            for which in (1, 2) for d in range(W_SLICE)]


# ---------------------------------------------------------------- policy --

def _constant(src, name):
    m = re.search(r"constexpr int " + name + r" = (\d+);", src)
    assert m, name
    return int(m.group(1))


def staging_policies():
    """Cache policy of each K/V staging DMA in persistent.hip, evaluated
    from the constants of token_device.hpp: {"fused": p, "long": p}."""
    dev = open(os.path.join(CSRC, "token_device.hpp")).read()
    consts = {n: _constant(dev, n) for n in ("kStreamPolicy", "kAgentCoherent")}
    src = open(os.path.join(CSRC, "persistent.hip")).read()
    found = {}
    for m in re.finditer(r"dma_padded_rows<([^>]*)>\((kst|vst), (kc|vc) \+ (\w+)", src):
        expr, _, _, base = m.groups()
        value = 0
        for term in expr.split("|"):
            term = term.strip()
            value |= consts[term] if term in consts else int(term)
        kind = "long" if base == "row0" else "fused"
        found.setdefault(kind, set()).add(value)
    assert set(found) == {"fused", "long"}, found
    return {k: v.pop() if len(v) == 1 else min(v) for k, v in found.items()}


# ----------------------------------------------------------------- audit --

def audit(launches, policies, kernel="token"):
    """Replay `launches` [(start, n_iter, long)] on one cache; rows before
    the first launch's start were written by an earlier launch (prefill).
    Returns counts per category and the flagged reads."""
    written_launch = {}  # (kv_head, row) -> launch index of the last write
    written_iter = {}
    writers = {}  # (kv_head, which, dim) -> workgroup
    for b in range(GRID):
        for key in (wide_writes(b) if kernel == "wide" else token_writes(b, False)):
            writers.setdefault(("wide", key) if kernel == "wide" else ("fused", key), b)
        if kernel == "token":
            for key in token_writes(b, True):
                writers.setdefault(("long", key), b)
    counts = {"earlier launch": 0, "same workgroup": 0, "other workgroup, coherent": 0,
              "cross-XCD": 0, "flagged": 0}
    flagged = []
    first_start = launches[0][0]
    heads = W_HEADS if kernel == "wide" else KVH
    row_writers = {}  # (mode, reader dims) -> the workgroups that store them
    for h in range(heads):
        for row in range(first_start):
            written_launch[(h, row)] = -1
    for li, (start, n_iter, long) in enumerate(launches):
        mode = "wide" if kernel == "wide" else ("long" if long else "fused")
        policy = policies.get(mode, 0)
        for it in range(n_iter):
            pos = start + it
            for b in range(GRID):
                if kernel == "wide":
                    (h, r0, r1), dims = wide_reads(b, pos)
                else:
                    h, r0, r1 = token_reads(b, long, pos)
                    dims = [(h, w, d) for w in (1, 2) for d in range(HD)]
                for row in range(r0, r1):
                    if row >= pos:
                        flagged.append((li, it, b, h, row, "row of the current position"))
                        counts["flagged"] += 1
                        continue
                    wl = written_launch.get((h, row))
                    if wl is None:
                        flagged.append((li, it, b, h, row, "row never written"))
                        counts["flagged"] += 1
                    elif wl < li:
                        counts["earlier launch"] += 1
                    else:
                        assert written_iter[(h, row)] < it
                        dk = (mode, tuple(dims))
                        if dk not in row_writers:
                            row_writers[dk] = {writers[(mode, key)] for key in dims}
                        wbs = row_writers[dk]
                        if wbs == {b}:
                            counts["same workgroup"] += 1
                        elif policy & SC1:
                            counts["other workgroup, coherent"] += 1
                            if any(xcd(w) != xcd(b) for w in wbs):
                                counts["cross-XCD"] += 1
                        else:
                            flagged.append((li, it, b, h, row,
                                            f"written in this launch by workgroups "
                                            f"{sorted(wbs)[:4]}... (XCDs "
                                            f"{sorted({xcd(w) for w in wbs})}), read by "
                                            f"{b} (XCD {xcd(b)}) without sc1"))
                            counts["flagged"] += 1
            for h in range(heads):
                written_launch[(h, pos)] = li
                written_iter[(h, pos)] = it
    return counts, flagged


def test_every_kv_dim_has_one_writer():
    """Each dim of each K and V row is stored by exactly one workgroup per
    layer, in both attention variants and in the wide kernel."""
    for long in (False, True):
        seen = {}
        for b in range(GRID):
            for key in token_writes(b, long):
                assert key not in seen, (long, key)
                seen[key] = b
        assert len(seen) == KVH * 2 * HD
    seen = {}
    for b in range(GRID):
        for key in wide_writes(b):
            assert key not in seen
            seen[key] = b
    assert len(seen) == W_HEADS * 2 * W_HD


def test_staging_policies_are_agent_coherent():
    p = staging_policies()
    assert p["fused"] & SC1 and p["long"] & SC1, p
    assert p["long"] & NT, p


# Launch schedules: (first cached row count, [(start, n_iter, long)]).
def split_attention_test(qtype):
    """test_token_kernel_split_attention: a 300-token step-kernel prefill,
    six one-token token-kernel decodes, then generate() after a batched
    prefill of the same prompt (a 6-iteration launch)."""
    fused = FUSED_POSITIONS[qtype]
    decodes = [(300 + s, 1, 300 + s + 1 > fused) for s in range(6)]
    return [decodes, [(300, 6, True)]]


WORKLOADS = {
    "split attention test int8": split_attention_test("int8"),
    "split attention test int4": split_attention_test("int4"),
    "split attention at max context": [[(4090 + s, 1, True) for s in range(6)]],
    "token-kernel prefill (path 2), 5 tokens + generate 16": [[(0, 5, False)], [(5, 16, False)]],
    "bench tinyllama_int4 (5 + 16)": [[(5, 16, False)]],
    "bench tinyllama_int8_2k (2048 + 128)": [[(2048, 128, True)]],
}


@pytest.mark.parametrize("name", list(WORKLOADS))
def test_token_kernel_kv_reads_are_ordered(name):
    policies = staging_policies()
    total = {}
    for launches in WORKLOADS[name]:
        # each list is one cache: rows before its first launch came from a
        # prefill launch
        counts, flagged = audit(launches, policies)
        assert not flagged, flagged[:5]
        for k, v in counts.items():
            total[k] = total.get(k, 0) + v
    print(f"{name}: {total}")
    assert total["flagged"] == 0


def test_generate_loops_read_rows_other_xcds_wrote():
    """The generate loops stage rows that workgroups on other XCDs stored
    earlier in the same launch, which is why the staging loads carry sc1;
    the one-token decode launches read earlier launches' rows only."""
    policies = staging_policies()
    counts, _ = audit(WORKLOADS["bench tinyllama_int8_2k (2048 + 128)"][0], policies)
    assert counts["cross-XCD"] > 0 and counts["other workgroup, coherent"] > 0
    counts, _ = audit(WORKLOADS["bench tinyllama_int4 (5 + 16)"][0], policies)
    assert counts["cross-XCD"] > 0
    counts, _ = audit(WORKLOADS["split attention test int8"][0], policies)
    assert counts["other workgroup, coherent"] == 0 and counts["earlier launch"] > 0


def test_audit_flags_a_non_coherent_staging():
    """The audit itself: the same schedules with the staging policy of the
    build before the fix (nt only, or the default policy) are flagged."""
    counts, flagged = audit([(2048, 8, True)], {"fused": 0, "long": NT})
    assert counts["flagged"] > 0 and "without sc1" in flagged[0][-1]
    counts, flagged = audit([(5, 4, False)], {"fused": 0, "long": NT})
    assert counts["flagged"] > 0


def test_audit_flags_current_row_and_unwritten_rows():
    """A read of the current position's row from the cache, or of a row no
    launch wrote, is flagged (the schedule model is not vacuous)."""
    orig = token_reads

    def reads_through_pos(b, long, pos):
        h, r0, r1 = orig(b, long, pos)
        return (h, r0, max(r1, min(pos + 1, r0 + PMAX)) if long else pos + 1)
    globals()["token_reads"] = reads_through_pos
    try:
        counts, flagged = audit([(10, 2, False)], {"fused": SC1, "long": SC1 | NT})
    finally:
        globals()["token_reads"] = orig
    assert any(f[-1] == "row of the current position" for f in flagged)


def test_wide_kernel_reads_only_its_own_rows():
    """The wide kernel (Llama-2-7B shape, 512 + 128): each workgroup reads
    only the dims of the rows it stored itself, so in-launch rows are
    ordered by program order on one CU; rows of the prefill by the kernel
    boundary."""
    counts, flagged = audit([(512, 128, False)], {"wide": 0}, kernel="wide")
    assert not flagged
    assert counts["other workgroup, coherent"] == 0
    assert counts["same workgroup"] > 0 and counts["earlier launch"] > 0
