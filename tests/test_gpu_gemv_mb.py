"""Q4_K matvec with fp32 products on the matrix cores (frq_gemv_mb.hip):
batch 1 through the tuned entry (FRQ_GEMV_MB), batches of 4 (and 5 .. 8 at
k <= 8192) through frq_dev_gemv, each against the oracle's fp64 matvec at
the 1e-5 contract (componentwise relative to sum_j |w_ij x_j|), on ordinary
data and on exactly cancelling weights under outlier x; a row's bits must not
depend on the other rows of its batch, on its position in it or on the rows
per workgroup.
"""

from __future__ import annotations

import numpy as np
import pytest

from cancelling import cancel_columns, outlier_x
from conftest import assert_matvec_close, bits_equal
from test_gpu_batched import _check_extreme_row
from flatrun_amd import _lib, device, synth
from oracle import gguf_np as G

pytestmark = pytest.mark.gpu


def _check(raw, xs, n, k, y, what):
    xs2 = xs.reshape(-1, k)
    y2 = y.reshape(xs2.shape[0], n)
    y64 = G.matmul_f64("Q4_K", xs2, raw, n, k).reshape(xs2.shape[0], n)
    a64 = G.abs_matmul_f64("Q4_K", xs2, raw, n, k).reshape(xs2.shape[0], n)
    for r in range(xs2.shape[0]):
        assert_matvec_close(y2[r], y64[r], a64[r], what=f"{what} row {r}")


def _tuned(raw, x, n, k, **geom):
    w, xd, yd = device.DeviceBuffer.from_host(raw), device.DeviceBuffer.from_host(x), device.DeviceBuffer(4 * n)
    try:
        cfg = device.gemv_tuned("Q4_K", w, xd, yd, n, k, kernel=_lib.GEMV_MB, **geom)
        device.synchronize()
        return yd.to_host(np.float32), cfg
    finally:
        w.free()
        xd.free()
        yd.free()


def _batched(raw, xs, n, k):
    b = xs.shape[0]
    w, xd, yd = device.DeviceBuffer.from_host(raw), device.DeviceBuffer.from_host(xs), device.DeviceBuffer(4 * n * b)
    try:
        nan = np.full(n * b, np.nan, np.float32)
        _lib.check(_lib.lib().frq_memcpy_h2d(yd.ptr, nan.ctypes.data, nan.nbytes))
        device.gemv("Q4_K", w, xd, yd, n, k, batch=b)
        device.synchronize()
        return yd.to_host(np.float32).reshape(b, n)
    finally:
        w.free()
        xd.free()
        yd.free()


# (n, k): one and several row groups, ragged row counts, odd block counts
# (the last pair half empty), one to three block pairs per wavefront, the
# headline shape and the longest rows the plan takes (48 pairs, 16 waves)
SHAPES = [(1, 256), (5, 256), (13, 13 * 256), (45, 4096), (260, 3584), (4100, 4096), (3584, 18944),
          (1024, 14336), (64, 24576), (3, 33 * 256)]


@pytest.mark.parametrize("n,k", SHAPES)
def test_batch1_against_oracle(frq, n, k):
    raw = synth.make_blocks("Q4_K", n, k, seed=n + k)
    x = synth.make_x(k, seed=k)
    y, cfg = _tuned(raw, x, n, k)
    assert cfg["kernel"] == _lib.GEMV_MB, cfg
    assert cfg["waves_per_wg"] * cfg["unroll"] * 2 >= k // 256, cfg
    _check(raw, x, n, k, y, f"MB {n}x{k} {cfg}")


def test_rows_and_pairs_per_wave(frq):
    """Rows per workgroup change nothing in a row's bits; pairs per wavefront
    (a different split of k over the wavefronts) stay within the contract."""
    n, k = 200, 12 * 512
    raw = synth.make_blocks("Q4_K", n, k, seed=11)
    x = synth.make_x(k, seed=12)
    for nbp in (1, 2, 3):
        ref = None
        for rows in (1, 3, 4, 7, 8, 13, 16):
            y, cfg = _tuned(raw, x, n, k, rows=rows, unroll=nbp)
            assert (cfg["rows"], cfg["unroll"]) == (rows, nbp), cfg
            if ref is None:
                ref = y
                _check(raw, x, n, k, y, f"MB rows {rows} pairs {nbp}")
            else:
                assert bits_equal(y, ref), (rows, nbp)


def test_plan_limits(frq):
    """Rows above 16 per workgroup and more than 16 wavefronts of block pairs
    are refused as unsupported, not launched."""
    n, k = 8, 49 * 512                    # 49 pairs: three per wavefront would need 17 wavefronts
    raw = synth.make_blocks("Q4_K", n, k, seed=1)
    x = synth.make_x(k, seed=2)
    with pytest.raises(RuntimeError, match="no plan"):
        _tuned(raw, x, n, k)
    raw2 = synth.make_blocks("Q4_K", 64, 4096, seed=1)
    with pytest.raises(RuntimeError, match="no plan"):
        _tuned(raw2, synth.make_x(4096, seed=3), 64, 4096, rows=17)
    with pytest.raises(RuntimeError, match="no plan"):
        _tuned(raw2, synth.make_x(4096, seed=3), 64, 4096, unroll=4)


@pytest.mark.parametrize("n,k", [(300, 4096), (3584, 18944), (100, 8192), (77, 14336), (9, 256)])
@pytest.mark.parametrize("seq", [4, 5, 8])
def test_batched_rows_against_oracle(frq, n, k, seq):
    """Batches of four rows (any k the plan takes) and of five to eight
    (k <= 8192) in one launch of this kernel, longer rows' larger batches in
    the small-M element-wise kernel; each row within the contract and with
    the bits it has in another batch of the same size, at another position
    among other rows."""
    raw = synth.make_blocks("Q4_K", n, k, seed=seq * 7 + n)
    xs = synth.make_x(k, seed=seq + 40, batch=seq)
    xs[seq - 1, 3] = 2.0**20
    y = _batched(raw, xs, n, k)
    _check(raw, xs, n, k, y, f"Q4_K {n}x{k} seq {seq}")
    other = synth.make_x(k, seed=seq + 90, batch=seq)
    for r in range(seq):
        moved = other.copy()
        moved[(r + 1) % seq] = xs[r]
        assert bits_equal(y[r], _batched(raw, moved, n, k)[(r + 1) % seq]), r


@pytest.mark.parametrize("n,k", [(512, 4096), (96, 18944), (40, 8192)])
def test_cancelling_weights(frq, n, k):
    """Exactly zero weights under non-zero scales meet x outliers of 2^24,
    -2^20 and 2^28, at batch 1 and in batches of 4 and 8 (8: this kernel
    where k <= 8192, else the element-wise small-M kernel)."""
    cols = sorted({5, 256 + 37, k - 3, 2 * 256 + 129})
    raw = cancel_columns("Q4_K", synth.make_blocks("Q4_K", n, k, seed=n), n, k, cols)
    x = outlier_x(k, cols, seed=3)
    y, _ = _tuned(raw, x, n, k)
    _check(raw, x, n, k, y, f"MB cancelling {n}x{k}")
    for seq in (4, 8):
        xs = np.stack([outlier_x(k, cols, seed=10 + r) for r in range(seq)])
        _check(raw, xs, n, k, _batched(raw, xs, n, k), f"MB cancelling {n}x{k} seq {seq}")


def test_nonfinite_and_tiny_x(frq):
    """x scaled by 2^-140 (subnormal products) and 2^110, and rows with inf
    or NaN, against the exact per-weight result under the batched path's
    criterion (1e-5 of sum_j |w_ij x_j| plus k 2^-150; IEEE classes for
    non-finite x)."""
    n, k = 64, 4096
    raw = synth.make_blocks("Q4_K", n, k, seed=5)
    base = synth.make_x(k, seed=6)
    rows = [base * np.float32(2.0**-140), base * np.float32(2.0**110), base.copy(), base.copy()]
    rows[2][17] = np.inf
    rows[3][100] = np.nan
    xs = np.stack(rows).astype(np.float32)
    y = _batched(raw, xs, n, k)
    W = G.DEQUANT["Q4_K"](raw, (n, k)).astype(np.float64)
    for r in range(4):
        _check_extreme_row(y[r], W, xs[r], f"MB row {r}")
        y1, _ = _tuned(raw, xs[r], n, k)
        assert bits_equal(y1, y[r]), r
