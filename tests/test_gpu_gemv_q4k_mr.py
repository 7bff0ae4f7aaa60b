"""The small-M Q4_K matvec (frq_gemv_mr.hip) against the oracle.

Two to six rows of x on a Q4_K matrix (k <= 24576, 16-byte aligned W and x)
run as launches of two or three rows that read W once each: per weight
w = fma(d*sc, q, -dmin*m), the dequant's fp32 value, then one fp32 FMA per
row of x, so the contract is the single-row matvec's -- 1e-5 of fp64,
normwise and componentwise per row -- on cancelling weights too. Cases: the
benchmark and model shapes at 2 .. 6 rows, ragged row counts (n not a
multiple of the rows per workgroup, one block per row, the largest k),
bits of a row independent of the batch it arrives in and of its position,
x with inf / NaN, rows longer than the kernel takes (their rows take the
GEMM or per-row GEMVs, under the same contract) and a misaligned x (an
argument error).
"""

from __future__ import annotations

import numpy as np
import pytest

from conftest import assert_matvec_close, bits_equal
from flatrun_amd import _lib, device, synth
from oracle import gguf_np as G

pytestmark = pytest.mark.gpu


def run(raw, xs, n, k, x_offset=0):
    """frq_dev_gemv with batch = rows of xs; x placed x_offset bytes into its
    buffer; outputs start as NaN so an unwritten element fails."""
    b = xs.shape[0]
    w = device.DeviceBuffer.from_host(raw)
    xd = device.DeviceBuffer(xs.nbytes + 16)
    yd = device.DeviceBuffer(4 * n * b)
    try:
        host = np.zeros(xs.nbytes + 16, np.uint8)
        host[x_offset:x_offset + xs.nbytes] = xs.reshape(-1).view(np.uint8)
        _lib.check(_lib.lib().frq_memcpy_h2d(xd.ptr, host.ctypes.data, host.nbytes))
        nan = np.full(n * b, np.nan, np.float32)
        _lib.check(_lib.lib().frq_memcpy_h2d(yd.ptr, nan.ctypes.data, nan.nbytes))
        device.gemv("Q4_K", w, xd.ptr + x_offset, yd, n, k, batch=b, w_bytes=raw.nbytes)
        device.synchronize()
        return yd.to_host(np.float32).reshape(b, n)
    finally:
        w.free()
        xd.free()
        yd.free()


def check_rows(raw, xs, n, k, y, what):
    y64 = G.matmul_f64("Q4_K", xs, raw, n, k)
    a64 = G.abs_matmul_f64("Q4_K", xs, raw, n, k)
    for r in range(xs.shape[0]):
        assert_matvec_close(y[r], y64[r], a64[r], what=f"{what} row {r}")


@pytest.mark.parametrize("n,k", [(3584, 18944), (18944, 3584), (4096, 4096), (1536, 8960), (512, 3584)])
@pytest.mark.parametrize("seq", [2, 3, 4, 5, 6])
def test_rows_within_contract(frq, n, k, seq):
    raw = synth.make_blocks("Q4_K", n, k, seed=n + k + seq)
    xs = synth.make_x(k, seed=seq + 11, batch=seq)
    xs[0, 7] = 2.0**24
    xs[seq - 1, k - 5] = -3e-30
    y = run(raw, xs, n, k)
    assert np.all(np.isfinite(y))
    check_rows(raw, xs, n, k, y, f"{n}x{k} seq {seq}")


@pytest.mark.parametrize("n,k", [(1, 256), (7, 256), (17, 512), (300, 24576), (4097, 1024), (4111, 2816)])
def test_ragged_shapes(frq, n, k):
    """Row counts that leave a partial workgroup, a single block per row, and
    the largest k (96 blocks: twelve wavefronts)."""
    for seq in (2, 3):
        raw = synth.make_blocks("Q4_K", n, k, seed=n * 3 + seq)
        xs = synth.make_x(k, seed=n + seq, batch=seq)
        check_rows(raw, xs, n, k, run(raw, xs, n, k), f"{n}x{k} seq {seq}")


def test_row_bits_independent_of_batch(frq):
    """A row's bits depend only on the row: the same x row gives the same
    output in a batch of 2, 3, 4, 5 or 6 (launches of two and of three rows)
    at any position."""
    n, k = 3584, 18944
    raw = synth.make_blocks("Q4_K", n, k, seed=5)
    pool = synth.make_x(k, seed=6, batch=6)
    probe = pool[2].copy()
    ref = None
    for seq in (2, 3, 4, 5, 6):
        for pos in sorted({0, seq - 1, seq // 2}):
            xs = pool[:seq].copy()
            xs[pos] = probe
            got = run(raw, xs, n, k)[pos]
            if ref is None:
                ref = got
                check_rows(raw, probe[None, :], n, k, ref[None, :], "probe row")
            assert bits_equal(got, ref), (seq, pos)


def test_non_finite_x(frq):
    n, k = 1024, 4096
    raw = synth.make_blocks("Q4_K", n, k, seed=7)
    W = G.dequant_q4_k(raw, (n, k)).astype(np.float64)
    xs = synth.make_x(k, seed=8, batch=3)
    xs[0, 100] = np.inf
    xs[1, 2000] = np.nan
    xs[2, 5], xs[2, 6] = np.inf, -np.inf
    y = run(raw, xs, n, k)
    for r in range(3):
        with np.errstate(all="ignore"):
            ref = (W * xs[r].astype(np.float64)[None, :]).sum(axis=1)
        assert np.array_equal(np.isnan(y[r]), np.isnan(ref)), r
        assert np.array_equal(np.isinf(y[r]), np.isinf(ref)), r
        inf = np.isinf(ref)
        assert np.array_equal(np.sign(y[r][inf]), np.sign(ref[inf])), r


def test_longer_rows_take_other_kernels(frq):
    """k past 96 blocks: the small-M kernel declines and the rows run
    elsewhere, within the same contract."""
    n, k = 512, 24832
    for seq in (2, 3):
        raw = synth.make_blocks("Q4_K", n, k, seed=k + seq)
        xs = synth.make_x(k, seed=seq, batch=seq)
        check_rows(raw, xs, n, k, run(raw, xs, n, k), f"{n}x{k} seq {seq}")


def test_misaligned_x_is_refused(frq):
    """x 4 bytes off a 16-byte boundary is an argument error of the device
    entry point, as for one row; nothing is launched."""
    n, k = 512, 4096
    raw = synth.make_blocks("Q4_K", n, k, seed=3)
    with pytest.raises(_lib.FrqError, match="16-byte aligned"):
        run(raw, synth.make_x(k, seed=4, batch=2), n, k, x_offset=4)
