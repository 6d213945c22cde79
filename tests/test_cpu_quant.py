"""Quantiser, fp16 scale helpers and quantised matvec on the CPU.

Pins the oracle (oracle/nut_oracle.c) and the product's host quantiser
(libnutllm_hip.so, nut_quantize) against:
  * golden vectors written by the reference itself (tests/golden/quant.npz,
    from src/quant.cpp compiled in place; see tests/golden/make_golden.py);
  * the reference's own known answers: the INT4 packing KAT [-7,-1,2,7] ->
    f9 72 (src/quant_selftest.cpp:92-101), the storage formula
    (src/quant_selftest.cpp:155-159), the all-zero block scale 2^-24
    (src/quant.cpp:171-173);
  * an independent library: numpy's fp16 conversion, exhaustively, with the
    reference's documented departures from round-to-nearest-even (lround
    ties away from zero, the subnormal clamp to 1..1023,
    src/quant.cpp:23-46).
"""
from __future__ import annotations

import ctypes as C
import json
import os

import numpy as np
import pytest

import nutllm_amd as nut
import oracle

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
INT8, INT4 = 0, 1


@pytest.fixture(scope="module")
def golden():
    return np.load(os.path.join(GOLDEN, "quant.npz"))


def case_names(g):
    return [str(n) for n in g["names"]]


def orc_half(value):
    bits = C.c_uint16()
    status = oracle.orc().orc_float_to_half(C.c_float(value), C.byref(bits))
    return status, bits.value


# --------------------------------------------------------------- fp16 --

def test_half_to_float_exhaustive():
    """Every finite non-negative half decodes as numpy's float16 does."""
    bits = np.arange(0, 0x7C00, dtype=np.uint16)
    expect = bits.view(np.float16).astype(np.float32)
    orc = np.array([oracle.orc().orc_half_to_float(int(b)) for b in bits],
                   np.float32)
    prod = np.array([nut.half_to_float(int(b)) for b in bits], np.float32)
    assert np.array_equal(orc, expect)
    assert np.array_equal(prod, expect)


def _expected_half(v):
    """fp16 bits the reference stores for a positive finite v <= 65504:
    round to nearest, ties upward (std::lround), and below 2^-14 the
    mantissa lround(v * 2^24) clamped to 1..1023."""
    v = np.float32(v)
    if v < np.float32(2.0 ** -14):
        return int(min(1023, max(1, np.floor(np.float64(v) * 2.0 ** 24 + 0.5))))
    h = np.float16(v)  # round to nearest even: differs only at ties
    hb = int(h.view(np.uint16))
    lo = np.float32(h)
    if lo > v:
        hb -= 1
        lo = np.float32(np.uint16(hb).view(np.float16))
    hi = np.float32(np.uint16(hb + 1).view(np.float16))
    # nearest, ties to the larger neighbour
    return hb + 1 if (np.float64(v) - lo) >= (np.float64(hi) - v) else hb


def test_float_to_half_exact_values_round_trip():
    for bits in range(1, 0x7C00):
        v = float(np.uint16(bits).view(np.float16))
        st, got = orc_half(v)
        assert st == 0 and got == bits, (hex(bits), hex(got))
        assert nut.float_to_half(v) == bits


def test_float_to_half_ties_round_up():
    """Midpoints between neighbouring halves go to the upper neighbour
    (numpy would pick the even one), except the 1023.5 * 2^-24 midpoint
    below 2^-14, which the subnormal clamp holds at 0x03FF."""
    for bits in range(1, 0x7BFF):
        lo = np.float64(np.uint16(bits).view(np.float16))
        hi = np.float64(np.uint16(bits + 1).view(np.float16))
        mid = np.float32((lo + hi) / 2)
        assert np.float64(mid) == (lo + hi) / 2  # representable tie
        st, got = orc_half(float(mid))
        want = 0x03FF if bits == 0x03FF else bits + 1
        assert st == 0 and got == want, (hex(bits), hex(got))
        assert nut.float_to_half(float(mid)) == want


def test_float_to_half_random_against_numpy():
    rng = np.random.default_rng(99)
    exps = rng.uniform(-30, 15.99, 40000)
    vals = np.exp2(exps).astype(np.float32)
    vals = vals[vals <= np.float32(65504.0)]
    for v in vals:
        want = _expected_half(v)
        st, got = orc_half(float(v))
        assert st == 0 and got == want, (float(v), hex(got), hex(want))
    # the product helper on a subsample
    for v in vals[:5000]:
        assert nut.float_to_half(float(v)) == _expected_half(v)


def test_float_to_half_subnormal_clamp():
    # below half the smallest subnormal: clamped up to 1 (numpy gives 0)
    for v in (2.0 ** -40, 2.0 ** -26, 0.49 * 2.0 ** -24):
        assert orc_half(v) == (0, 1)
        assert nut.float_to_half(v) == 1
    # just below 2^-14: clamped to 0x03FF (numpy rounds up to 0x0400)
    v = float(np.nextafter(np.float32(2.0 ** -14), np.float32(0)))
    assert orc_half(v) == (0, 0x03FF)
    assert nut.float_to_half(v) == 0x03FF


@pytest.mark.parametrize("value,status", [
    (0.0, 1), (-1.0, 1), (float("inf"), 1), (float("nan"), 1),
    (65504.5, 4), (1e9, 4)])
def test_float_to_half_errors(value, status):
    """invalid_argument for non-positive / non-finite scales, range_error
    above fp16 (src/quant.cpp:24-27)."""
    assert orc_half(value)[0] == status
    err = nut.InvalidArgument if status == 1 else nut.RangeError
    with pytest.raises(err):
        nut.float_to_half(value)


# ---------------------------------------------------------- quantiser --

def test_int4_packing_kat():
    """[-7, -1, 2, 7] -> bytes f9 72, scale 1.0 (src/quant_selftest.cpp:92)."""
    w = np.array([[-7.0, -1.0, 2.0, 7.0]], np.float32)
    st, data, scales = oracle.quantize(w, INT4)
    assert st == 0
    assert data.tolist() == [0xF9, 0x72]
    assert scales.tolist() == [0x3C00]
    pdata, pscales = nut.quantize(w, INT4)
    assert pdata.tolist() == [0xF9, 0x72] and pscales.tolist() == [0x3C00]


def test_zero_block_scale_is_min_subnormal():
    w = np.zeros((2, 64), np.float32)
    for qt in (INT8, INT4):
        st, data, scales = oracle.quantize(w, qt)
        assert st == 0 and set(scales.tolist()) == {0x0001}
        assert not data.any()
        pdata, pscales = nut.quantize(w, qt)
        assert set(pscales.tolist()) == {0x0001} and not pdata.any()


@pytest.mark.parametrize("rows,cols", [(1, 1), (3, 7), (5, 37), (64, 172),
                                       (2048, 2048), (4096, 11008)])
def test_storage_formula(rows, cols):
    n = rows * cols
    blocks = -(-n // 32)
    for qt, data in ((INT8, n), (INT4, -(-n // 2))):
        want = data + 2 * blocks
        assert oracle.orc().orc_storage_bytes(rows, cols, qt, 32) == want
        assert nut.lib().nut_quant_storage_bytes(rows, cols, qt, 32) == want


@pytest.mark.parametrize("impl", ["oracle", "product"])
def test_quantize_matches_reference(golden, impl):
    for name in case_names(golden):
        w = golden[f"{name}/w"]
        qt = int(golden[f"{name}/qtype"])
        if impl == "oracle":
            st, data, scales = oracle.quantize(w, qt)
            assert st == 0, name
        else:
            data, scales = nut.quantize(w, qt)
        assert np.array_equal(data, golden[f"{name}/data"]), name
        assert np.array_equal(scales, golden[f"{name}/scales"]), name
        rows, cols = w.shape
        assert oracle.orc().orc_storage_bytes(rows, cols, qt, 32) == \
            int(golden[f"{name}/storage"]), name


def test_crafted_scales_cover_ties_and_clamps(golden):
    """The crafted rows hold fp16 ties, subnormal ties and both clamps; the
    reference's scale bits agree with the closed form above."""
    for qt, limit in ((INT8, 127), (INT4, 7)):
        w = golden[f"crafted_{qt}/w"].reshape(-1, 32)
        scales = golden[f"crafted_{qt}/scales"]
        for block, bits in zip(w[:-1], scales[:-1]):
            exact = np.float32(np.abs(block).max()) / np.float32(limit)
            assert bits == _expected_half(exact), (float(exact), hex(bits))
        assert scales[-1] == 0x0001  # zero block


def test_error_bound_matches_reference(golden):
    for name in case_names(golden):
        w = golden[f"{name}/w"]
        qt = int(golden[f"{name}/qtype"])
        rows, cols = w.shape
        q = oracle.qmat(golden[f"{name}/data"], golden[f"{name}/scales"],
                        rows, cols, qt)
        bounds = golden[f"{name}/bounds"]
        deq = oracle.dequantize(golden[f"{name}/data"],
                                golden[f"{name}/scales"], rows, cols, qt)
        # a sample of elements through the oracle's error_bound
        idx = np.random.default_rng(1).integers(0, rows * cols, 64)
        for i in idx:
            r, c = divmod(int(i), cols)
            got = oracle.orc().orc_error_bound(C.byref(q), r, c)
            assert np.float32(got) == bounds[r, c], (name, r, c)
        assert np.all(np.abs(deq - w) <= bounds), name


def test_quantize_errors_match_reference():
    with open(os.path.join(GOLDEN, "quant_errors.json")) as f:
        cases = json.load(f)
    for case in cases:
        w = np.zeros((1, 32), np.float32)
        w[0, 0] = np.float32(float(case["w0"]))
        w[0, 1:] = 1.0 if case["name"] in ("nan", "inf") else 0.0
        st, _, _ = oracle.quantize(w, case["qtype"])
        assert st == case["status"], case
        err = nut.InvalidArgument if case["status"] == 1 else nut.RangeError
        with pytest.raises(err):
            nut.quantize(w, case["qtype"])


def test_quantize_rejects_zero_block_size():
    w = np.ones((2, 32), np.float32)
    assert oracle.quantize(w, INT8, block_size=0)[0] == 1
    with pytest.raises(nut.InvalidArgument):
        nut.quantize(w, INT8, block_size=0)


# -------------------------------------------------------------- matvec --

def test_matvec_matches_reference(golden):
    """AVX2 block path (fast layout) and double scalar path (straddling
    blocks) reproduce the reference bit for bit."""
    for name in case_names(golden):
        w = golden[f"{name}/w"]
        qt = int(golden[f"{name}/qtype"])
        rows, cols = w.shape
        y = oracle.matvec_q(golden[f"{name}/data"], golden[f"{name}/scales"],
                            rows, cols, qt, golden[f"{name}/x"])
        assert np.array_equal(y, golden[f"{name}/y"]), name


def test_matvec_unit_vectors_give_columns(golden):
    for name in ("range_0", "range_1", "w2_1", "straddle_0"):
        w = golden[f"{name}/w"]
        qt = int(golden[f"{name}/qtype"])
        rows, cols = w.shape
        data, scales = golden[f"{name}/data"], golden[f"{name}/scales"]
        deq = oracle.dequantize(data, scales, rows, cols, qt)
        for k in (0, 1, cols // 2, cols - 1):
            x = np.zeros(cols, np.float32)
            x[k] = 1.0
            y = oracle.matvec_q(data, scales, rows, cols, qt, x)
            assert np.array_equal(y, deq[:, k]), (name, k)


def test_matvec_fp64_brute_force(golden):
    for name in case_names(golden):
        w = golden[f"{name}/w"]
        qt = int(golden[f"{name}/qtype"])
        rows, cols = w.shape
        data, scales = golden[f"{name}/data"], golden[f"{name}/scales"]
        x = golden[f"{name}/x"]
        deq = oracle.dequantize(data, scales, rows, cols, qt).astype(np.float64)
        exact = deq @ x.astype(np.float64)
        y = oracle.matvec_q(data, scales, rows, cols, qt, x)
        scale = np.abs(deq) @ np.abs(x.astype(np.float64)) + 1e-30
        assert np.all(np.abs(y - exact) <= 1e-5 * scale), name


def test_matvec_thread_count_invariant(golden):
    name = "w2_0"
    w = golden[f"{name}/w"]
    rows, cols = w.shape
    args = (golden[f"{name}/data"], golden[f"{name}/scales"], rows, cols, 0,
            golden[f"{name}/x"])
    before = oracle.orc().orc_get_threads()
    try:
        oracle.orc().orc_set_threads(1)
        y1 = oracle.matvec_q(*args)
        oracle.orc().orc_set_threads(5)
        y5 = oracle.matvec_q(*args)
    finally:
        oracle.orc().orc_set_threads(before)
    assert np.array_equal(y1, y5)


def test_matvec_zero_matrix():
    w = np.zeros((8, 64), np.float32)
    st, data, scales = oracle.quantize(w, INT4)
    y = oracle.matvec_q(data, scales, 8, 64, INT4,
                        np.arange(64, dtype=np.float32))
    assert not y.any()
