"""Test helpers for the token kernels' screened classifier argmax: rows
whose INT8 block-32 screening copy (codes rint(w / s), s the smallest fp16
at or above the block's max |w| / 127) equals another row's, with a
different fp32 logit."""
import numpy as np


def screen_scales(row):
    """Block-32 scales of the screening copy: the smallest fp16 at or above
    each block's max |w| / 127, and at least 2^-14."""
    t = np.max(np.abs(row.reshape(-1, 32).astype(np.float64)), axis=1) / 127.0
    h = t.astype(np.float16)
    low = h.astype(np.float64) < t
    h[low] = np.nextafter(h[low], np.float16(np.inf))
    return np.maximum(h.astype(np.float64), 2.0 ** -14)


def screen_twin(row, x, up):
    """A copy of classifier row `row` whose INT8 screening copy (block-32
    codes rint(w / s), s = screen_scales) is identical to the row's: every
    weight but each block's largest moves half way to the edge of its code's
    rounding interval, towards larger logits (up) or smaller ones."""
    row = np.asarray(row, np.float32)
    s = np.repeat(screen_scales(row), 32)
    q = np.rint(row / s)
    big = np.zeros(row.size, bool)
    big[np.argmax(np.abs(row.reshape(-1, 32)), axis=1) + 32 * np.arange(row.size // 32)] = True
    toward = np.where((x > 0) == up, 1.0, -1.0)
    edge = (q + 0.5 * toward) * s
    twin = np.where(big, row, (row + 0.5 * (edge - row)).astype(np.float32)).astype(np.float32)
    keep = np.abs(twin) >= np.repeat(np.max(np.abs(row.reshape(-1, 32)), axis=1), 32)
    twin[keep & ~big] = row[keep & ~big]  # no block maximum changes
    assert np.array_equal(screen_scales(twin), screen_scales(row))
    assert np.array_equal(np.rint(twin / s), q)
    return twin
