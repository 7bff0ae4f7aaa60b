"""The cancelling-column inputs (tests/cancelling.py), on the CPU: every
column made zero is zero in the oracle's dequant with nonzero scales, the
rest of the matrix is untouched outside the edited blocks, and the inputs
tell the two ways of writing a sub-block's sum apart -- an fp32 emulation of
the scale algebra s * sum(q x) - t * sum(x) breaks the 1e-5 componentwise
bound on them, the per-weight form sum(fl(s q - t) x) keeps it."""

from __future__ import annotations

import numpy as np
import pytest

from cancelling import BLOCK, CANCEL_FORMATS, cancel_columns, outlier_x
from conftest import MATVEC_RTOL, matvec_errors
from flatrun_amd import synth
from oracle import gguf_np as G


@pytest.mark.parametrize("q", CANCEL_FORMATS)
def test_columns_zero_with_nonzero_scales(q):
    n, k = 48, 1024
    cols = [0, 37, 100, 255, 300, 511, 512 + 200, 1023]
    raw = synth.make_blocks(q, n, k, seed=7)
    out = cancel_columns(q, raw, n, k, cols)
    w0 = G.DEQUANT[q](raw, (n, k))
    w = G.DEQUANT[q](out, (n, k))
    assert np.all(w[:, cols] == 0)
    bb, be = BLOCK[q]
    touched = sorted({c // be for c in cols})
    untouched = np.ones(k, bool)
    for b in touched:
        untouched[b * be:(b + 1) * be] = False
    assert np.array_equal(w[:, untouched], w0[:, untouched])
    # the cancelling blocks keep nonzero weights elsewhere: the scales are live
    for c in cols:
        b = c // be
        blk = w[:, b * be:(b + 1) * be]
        assert np.count_nonzero(blk) > blk.size // 2, (q, c)


def _q4k_codes(raw, n, k):
    """(codes (n, k) float32, s and t per (row, sub-block)) of Q4_K blocks."""
    a = np.asarray(raw, np.uint8).reshape(-1, 144)
    d = a[:, 0:2].copy().view("<f2").astype(np.float32).reshape(-1)
    dmin = a[:, 2:4].copy().view("<f2").astype(np.float32).reshape(-1)
    sc, m = G.scale_min_k4(a[:, 4:16])
    q = G._nibbles_k(a[:, 16:144]).astype(np.float32).reshape(n, k)
    s = (d[:, None] * sc).reshape(n, k // 32)
    t = (dmin[:, None] * m).reshape(n, k // 32)
    return q, s, t


def test_inputs_separate_scale_algebra_from_per_weight():
    n, k = 64, 4096
    cols = [5, 1000, 3000]
    raw = cancel_columns("Q4_K", synth.make_blocks("Q4_K", n, k, seed=11), n, k, cols)
    x = outlier_x(k, cols, seed=12)
    q, s, t = _q4k_codes(raw, n, k)
    xs = x.reshape(k // 32, 32)
    y_alg = np.zeros(n, np.float32)
    y_pw = np.zeros(n, np.float32)
    w = G.dequant_q4_k(raw, (n, k))
    for b in range(k // 32):
        qx = np.sum(q[:, 32 * b:32 * b + 32] * xs[b], axis=1, dtype=np.float32)
        sx = np.float32(np.sum(xs[b], dtype=np.float32))
        y_alg += s[:, b] * qx - t[:, b] * sx
        y_pw += np.sum(w[:, 32 * b:32 * b + 32] * xs[b], axis=1, dtype=np.float32)
    y64 = G.matmul_f64("Q4_K", x, raw, n, k)
    a64 = G.abs_matmul_f64("Q4_K", x, raw, n, k)
    assert matvec_errors(y_alg, y64, a64)[1] > 10 * MATVEC_RTOL
    assert matvec_errors(y_pw, y64, a64)[1] < MATVEC_RTOL / 10
