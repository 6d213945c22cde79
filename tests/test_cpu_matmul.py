"""The oracle's fp32 GEMM (orc_matmul) on the CPU.

matmul_threaded (src/threading.cpp:163-181) runs the AVX2 register-blocked
kernel of src/matmul.cpp:123-214: every C element accumulates A[i][k] B[k][j]
over k = 0 .. K-1 in order with one fused multiply-add per step, starting
from zero. orc_matmul is pinned by:
  * the reference itself, compiled in place (oracle/_ref, when built):
    bit for bit, on a ragged shape and on the 768^3 workload;
  * what the mathematics fixes: identity and permutation matrices give exact
    copies, and a float64 product bounds the rounding;
  * a planted ordering mistake (summing k in reverse) that these checks
    catch.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle as O


def orc_matmul(a, b):
    m, k = a.shape
    n = b.shape[1]
    c = np.empty((m, n), np.float32)
    O.check(O.orc().orc_matmul(O.ptr(a), O.ptr(b), O.ptr(c), m, k, n),
            "orc_matmul")
    return c


def rand(rng, *shape):
    return rng.standard_normal(shape).astype(np.float32)


def test_identity_and_permutation_are_exact():
    rng = np.random.default_rng(11)
    a = rand(rng, 37, 53)
    eye = np.eye(53, dtype=np.float32)
    assert np.array_equal(orc_matmul(a, eye), a)
    perm = np.eye(53, dtype=np.float32)[rng.permutation(53)]
    assert np.array_equal(orc_matmul(a, perm), a @ perm)


def test_close_to_float64_product():
    rng = np.random.default_rng(12)
    a, b = rand(rng, 41, 67), rand(rng, 67, 29)
    exact = a.astype(np.float64) @ b.astype(np.float64)
    got = orc_matmul(a, b).astype(np.float64)
    # sequential fp32 fma over 67 terms: error well under 67 ulp of |a||b|
    bound = 67 * np.finfo(np.float32).eps * (np.abs(a) @ np.abs(b))
    assert np.all(np.abs(got - exact) <= bound)


def sequential_fma(a, b):
    """C[i][j] = fma(a[i][k], b[k][j], C[i][j]) for k in order, in float32.
    numpy has no fused multiply-add: each step adds in float64, where the
    product of two floats is exact, and rounds to float32; that double
    rounding can differ from one fused rounding only in rare ties."""
    c = np.zeros((a.shape[0], b.shape[1]), np.float32)
    for k in range(a.shape[1]):
        c = (c.astype(np.float64) + np.outer(a[:, k].astype(np.float64),
                                             b[k].astype(np.float64))
             ).astype(np.float32)
    return c


def test_order_is_sequential_fma():
    rng = np.random.default_rng(13)
    a, b = rand(rng, 9, 40), rand(rng, 40, 7)
    assert np.array_equal(orc_matmul(a, b), sequential_fma(a, b))
    # a planted mistake: k summed in reverse order differs somewhere
    planted = sequential_fma(a[:, ::-1].copy(), b[::-1].copy())
    assert not np.array_equal(planted, sequential_fma(a, b))


@pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built")
@pytest.mark.parametrize("mkn", [(20, 33, 48), (768, 768, 768)],
                         ids=["ragged", "768cubed"])
def test_bit_exact_with_reference(mkn):
    m, k, n = mkn
    rng = np.random.default_rng(14)
    a, b = rand(rng, m, k), rand(rng, k, n)
    ref = np.empty((m, n), np.float32)
    O.check(O.ref().ref_matmul(O.ptr(a), O.ptr(b), O.ptr(ref), m, k, n, 4),
            "ref_matmul")
    O.orc().orc_set_threads(4)
    assert np.array_equal(orc_matmul(a, b), ref)
