"""The small-M matvec (frq_gemv_mr.hip) against the oracle and the
single-row kernels.

A few rows of x (Q4_K and Q8_0: two to six, Q6_K: two to ten) on a matrix
the kernel takes run as launches of two or three rows that read W once each.
Q4_K forms every weight as w = fma(d*sc, q, -dmin*m), the dequant's fp32
value, then one fp32 FMA per row of x, so the contract is the single-row
matvec's -- 1e-5 of fp64, normwise and componentwise per row -- on cancelling
weights too. Q6_K and Q8_0 run the single-row ring kernels' per-lane sums and
reduction order for each row of x, so every row has the bits of a batch-1
call. Cases: the benchmark and model shapes at every routed row count, ragged
row counts (n not a multiple of the rows per workgroup, one block per row,
the largest k), a row's bits independent of its batch and position, x with
inf / NaN, shapes the kernel refuses (an odd block count, a Q6_K / Q8_0 W
off its 4-byte alignment, rows longer than its lanes: their rows take
per-row GEMVs or the GEMM, under the same contract) and a misaligned x (an
argument error).
"""

from __future__ import annotations

import numpy as np
import pytest

from conftest import assert_matvec_close, bits_equal
from flatrun_amd import _lib, device, synth
from oracle import gguf_np as G

pytestmark = pytest.mark.gpu

ROUTED = {"Q4_K": 6, "Q6_K": 10, "Q8_0": 6}     # rows of x that the small-M kernel takes


def run(q, raw, xs, n, k, x_offset=0, w_offset=0):
    """frq_dev_gemv with batch = rows of xs; x (W) placed x_offset (w_offset)
    bytes into its buffer; outputs start as NaN so an unwritten element
    fails."""
    b = xs.shape[0]
    wd = device.DeviceBuffer(raw.nbytes + 16)
    xd = device.DeviceBuffer(xs.nbytes + 16)
    yd = device.DeviceBuffer(4 * n * b)
    try:
        host_w = np.zeros(raw.nbytes + 16, np.uint8)
        host_w[w_offset:w_offset + raw.nbytes] = raw
        _lib.check(_lib.lib().frq_memcpy_h2d(wd.ptr, host_w.ctypes.data, host_w.nbytes))
        host = np.zeros(xs.nbytes + 16, np.uint8)
        host[x_offset:x_offset + xs.nbytes] = xs.reshape(-1).view(np.uint8)
        _lib.check(_lib.lib().frq_memcpy_h2d(xd.ptr, host.ctypes.data, host.nbytes))
        nan = np.full(n * b, np.nan, np.float32)
        _lib.check(_lib.lib().frq_memcpy_h2d(yd.ptr, nan.ctypes.data, nan.nbytes))
        device.gemv(q, wd.ptr + w_offset, xd.ptr + x_offset, yd, n, k, batch=b, w_bytes=raw.nbytes)
        device.synchronize()
        return yd.to_host(np.float32).reshape(b, n)
    finally:
        wd.free()
        xd.free()
        yd.free()


def check_rows(q, raw, xs, n, k, y, what):
    y64 = G.matmul_f64(q, xs, raw, n, k)
    a64 = G.abs_matmul_f64(q, xs, raw, n, k)
    for r in range(xs.shape[0]):
        assert_matvec_close(y[r], y64[r], a64[r], what=f"{what} row {r}")


def single_rows(q, raw, xs, n, k):
    return np.stack([run(q, raw, xs[r:r + 1].copy(), n, k)[0] for r in range(xs.shape[0])])


SHAPES = [("Q4_K", 3584, 18944), ("Q4_K", 18944, 3584), ("Q4_K", 4096, 4096), ("Q4_K", 1536, 8960),
          ("Q4_K", 512, 3584), ("Q6_K", 4096, 14336), ("Q6_K", 1024, 4096), ("Q6_K", 9504, 3584),
          ("Q8_0", 4864, 896), ("Q8_0", 4096, 4096), ("Q8_0", 896, 4864), ("Q8_0", 1024, 14336)]


@pytest.mark.parametrize("q,n,k", SHAPES)
def test_rows_within_contract(frq, q, n, k):
    """Every routed row count; Q6_K / Q8_0 rows bit-equal to batch-1 calls."""
    top = ROUTED[q]
    raw = synth.make_blocks(q, n, k, seed=n + k)
    xs = synth.make_x(k, seed=k + 1, batch=top)
    xs[0, 7] = 2.0**24
    xs[top - 1, k - 5] = -3e-30
    ref = single_rows(q, raw, xs, n, k) if q != "Q4_K" else None
    for seq in range(2, top + 1):
        y = run(q, raw, xs[:seq].copy(), n, k)
        assert np.all(np.isfinite(y)), seq
        check_rows(q, raw, xs[:seq], n, k, y, f"{q} {n}x{k} seq {seq}")
        if ref is not None:
            assert bits_equal(y, ref[:seq]), (q, n, k, seq)


@pytest.mark.parametrize("q,n,k", [("Q4_K", 1, 256), ("Q4_K", 7, 256), ("Q4_K", 17, 512), ("Q4_K", 300, 24576),
                                   ("Q4_K", 4097, 1024), ("Q4_K", 4111, 2816), ("Q6_K", 1, 512), ("Q6_K", 33, 512),
                                   ("Q6_K", 300, 24576), ("Q6_K", 4097, 1024), ("Q8_0", 1, 64), ("Q8_0", 45, 64),
                                   ("Q8_0", 300, 16384), ("Q8_0", 4113, 1024)])
def test_ragged_shapes(frq, q, n, k):
    """Row counts that leave a partial workgroup, the smallest block count,
    and the largest k (twelve or sixteen wavefronts)."""
    for seq in (2, 3):
        raw = synth.make_blocks(q, n, k, seed=n * 3 + seq)
        xs = synth.make_x(k, seed=n + seq, batch=seq)
        y = run(q, raw, xs, n, k)
        check_rows(q, raw, xs, n, k, y, f"{q} {n}x{k} seq {seq}")
        if q != "Q4_K":
            assert bits_equal(y, single_rows(q, raw, xs, n, k)), (q, n, k, seq)


def test_q4k_row_bits_independent_of_batch(frq):
    """A Q4_K row's bits depend only on the row: the same x row gives the
    same output in a batch of 2, 3, 5 or 6 (launches of two and of three rows
    of this kernel) at any position. (Four rows take the fp32 matrix-core
    kernel, whose rows are position- and content-independent within their
    batch size: test_gpu_gemv_mb.py.)"""
    n, k = 3584, 18944
    raw = synth.make_blocks("Q4_K", n, k, seed=5)
    pool = synth.make_x(k, seed=6, batch=6)
    probe = pool[2].copy()
    ref = None
    for seq in (2, 3, 5, 6):
        for pos in sorted({0, seq - 1, seq // 2}):
            xs = pool[:seq].copy()
            xs[pos] = probe
            got = run("Q4_K", raw, xs, n, k)[pos]
            if ref is None:
                ref = got
                check_rows("Q4_K", raw, probe[None, :], n, k, ref[None, :], "probe row")
            assert bits_equal(got, ref), (seq, pos)


@pytest.mark.parametrize("q", ["Q4_K", "Q6_K", "Q8_0"])
def test_non_finite_x(frq, q):
    n, k = 1024, 4096
    raw = synth.make_blocks(q, n, k, seed=7)
    W = G.DEQUANT[q](raw, (n, k)).astype(np.float64)
    xs = synth.make_x(k, seed=8, batch=3)
    xs[0, 100] = np.inf
    xs[1, 2000] = np.nan
    xs[2, 5], xs[2, 6] = np.inf, -np.inf
    y = run(q, raw, xs, n, k)
    for r in range(3):
        with np.errstate(all="ignore"):
            ref = (W * xs[r].astype(np.float64)[None, :]).sum(axis=1)
        assert np.array_equal(np.isnan(y[r]), np.isnan(ref)), r
        assert np.array_equal(np.isinf(y[r]), np.isinf(ref)), r
        inf = np.isinf(ref)
        assert np.array_equal(np.sign(y[r][inf]), np.sign(ref[inf])), r


@pytest.mark.parametrize("q,n,k,w_offset", [("Q4_K", 512, 24832, 0), ("Q6_K", 512, 768, 0),
                                            ("Q6_K", 512, 4096, 2), ("Q6_K", 64, 25088, 0), ("Q8_0", 512, 96, 0),
                                            ("Q8_0", 512, 4096, 2)])
def test_refused_shapes_take_other_kernels(frq, q, n, k, w_offset):
    """An odd block count, W 2 bytes off a 4-byte boundary (Q6_K, Q8_0), or
    k past the kernel's lanes (Q4_K, Q6_K; the library's Q8_0 rows end
    where the kernel's lanes do): the small-M kernel declines and the rows run
    elsewhere (per-row GEMVs up to three rows, else the GEMM or per-row
    GEMVs), within the same contract."""
    for seq in (2, 3, 5):
        raw = synth.make_blocks(q, n, k, seed=k + seq)
        xs = synth.make_x(k, seed=seq, batch=seq)
        check_rows(q, raw, xs, n, k, run(q, raw, xs, n, k, w_offset=w_offset), f"{q} {n}x{k}+{w_offset} seq {seq}")


def test_misaligned_x_is_refused(frq):
    """x 4 bytes off a 16-byte boundary is an argument error of the device
    entry point, as for one row; nothing is launched."""
    n, k = 512, 4096
    raw = synth.make_blocks("Q4_K", n, k, seed=3)
    with pytest.raises(_lib.FrqError, match="16-byte aligned"):
        run("Q4_K", raw, synth.make_x(k, seed=4, batch=2), n, k, x_offset=4)
