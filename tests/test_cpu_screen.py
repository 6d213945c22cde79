"""CPU checks of the screened classifier argmax's error bound.

The token kernels find the greedy argmax through an INT8 block-32 copy of
the fp32 classifier: per block, s = the smallest fp16 at or above
max|w| / 127 (and 2^-14), q = rint(w / s); x goes in as per-block integer
digits X = rint(x 7e6 / max|x_b|) with scale xsc_b = max|x_b| / 7e6. A
row's screened logit a = sum_b s_b xsc_b (q . X)_b then differs from the
fp32 logit by at most kappa(n) T with T = sum_b s_b ||x_b||_1 and
kappa(n) = 1.01 (0.5 (1 + 2^-10) + 127 gamma_n + 0.0025)
(screen_kappa in nutllm_amd/csrc/token_device.hpp). Here, in float64 and
with float32 sums in several orders, on random rows and on rows built so
that every rounding error of the copy points the same way:

* the copy's part is at most T / 2 and comes within a few percent of it
  on the built rows (so a factor much below one half would fail);
* the whole difference to float32 logits summed in any of three orders
  stays under kappa(n) T.
"""
import numpy as np
import pytest

from screening import screen_scales

LIMB_RANGE = 7.0e6


def kappa(n):
    gamma = n * 2.0 ** -24 / (1.0 - n * 2.0 ** -24)
    return 1.01 * (0.5 * (1.0 + 1.0 / 1024) + 127.0 * gamma + 0.0025)


def screened(row, x):
    """(a, T, the copy's exact part sum_k x_k (w_k - s q_k)) in float64."""
    n = row.size
    s = np.repeat(screen_scales(row), 32)
    q = np.clip(np.rint(row.astype(np.float64) / s), -127, 127)
    xb = x.astype(np.float64).reshape(-1, 32)
    mx = np.max(np.abs(xb), axis=1)
    xsc = np.where(mx > 0, mx / LIMB_RANGE, 0.0)
    digits = np.where(mx[:, None] > 0, np.rint(xb * (LIMB_RANGE / np.where(mx > 0, mx, 1.0))[:, None]), 0.0)
    xhat = (digits * xsc[:, None]).reshape(n)
    a = float(np.sum(s * q * xhat))
    t = float(np.sum(screen_scales(row) * np.sum(np.abs(xb), axis=1)))
    copy_part = float(np.sum(x.astype(np.float64) * (row.astype(np.float64) - s * q)))
    return a, t, copy_part


def fp32_logits(row, x):
    """The fp32 logit summed three ways: in order, reversed, and as 64
    lanes of strided partial sums reduced pairwise."""
    p = (row.astype(np.float32) * x.astype(np.float32)).astype(np.float32)
    out = []
    for order in (p, p[::-1]):
        acc = np.float32(0)
        for v in order:
            acc = np.float32(acc + v)
        out.append(float(acc))
    lanes = np.zeros(64, np.float32)
    for k in range(p.size):
        lanes[k % 64] = np.float32(lanes[k % 64] + p[k])
    while lanes.size > 1:
        lanes = (lanes[: lanes.size // 2] + lanes[lanes.size // 2:]).astype(np.float32)
    out.append(float(lanes[0]))
    return out


def aligned_row(rng, n, x):
    """Every weight but each block's largest sits 0.49 of a code step from
    its code, on the side that makes its error push the logit the same way
    as x (the copy's error then nearly reaches T / 2)."""
    s = np.repeat(screen_scales((rng.standard_normal(n) * 0.02).astype(np.float32)), 32)
    q = rng.integers(-100, 100, n).astype(np.float64)
    w = (q + 0.49 * np.sign(x)) * s  # |w| < 127 s keeps s
    w = w.astype(np.float32)
    w.reshape(-1, 32)[:, 0] = (127.0 * s.reshape(-1, 32)[:, 0]).astype(np.float32)
    return w


@pytest.mark.parametrize("n", [2048, 4096])
def test_copy_error_reaches_half_t_and_no_more(n):
    rng = np.random.default_rng(n)
    worst = 0.0
    for trial in range(20):
        x = rng.standard_normal(n).astype(np.float32)
        row = aligned_row(rng, n, x) if trial % 2 else (rng.standard_normal(n) * 0.02).astype(np.float32)
        _, t, copy_part = screened(row, x)
        ratio = abs(copy_part) / t
        assert ratio <= 0.5 * (1 + 2.0 ** -10), ratio
        worst = max(worst, ratio)
    # the built rows come within a few percent of the half
    assert worst > 0.45, worst


@pytest.mark.parametrize("n", [2048, 4096])
@pytest.mark.parametrize("kind", ["normal", "aligned", "outliers"])
def test_bound_covers_fp32_logits(n, kind):
    rng = np.random.default_rng(7 + n)
    for _ in range(4):
        x = rng.standard_normal(n).astype(np.float32)
        if kind == "outliers":
            x[rng.integers(0, n, 8)] *= 300.0
        row = (aligned_row(rng, n, x) if kind == "aligned"
               else (rng.standard_normal(n) * 0.02).astype(np.float32))
        if kind == "outliers":
            row[rng.integers(0, n, 8)] = 3.0
        a, t, _ = screened(row, x)
        e = kappa(n) * t
        for s in fp32_logits(row, x):
            assert abs(s - a) <= e, (kind, s, a, e)

