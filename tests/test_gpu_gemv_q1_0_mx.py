"""The matrix-core Q1_0 GEMV (frq_gemv_mx.hip) against the oracle.

The kernel writes x per 32-element group as a 30-bit fixed-point number
(four balanced int8 digits) and forms each group's sum of +-x on the int8
matrix cores; every Q1_0 weight has |w| = |d|, so the truncation stays
within 2^-24 of each group's own sum |w x| and the contract -- 1e-5 of fp64,
normwise and componentwise per row -- holds for any finite x. Cases: every
explicit geometry (blocks per wavefront 1 / 2 / 4 / 8, rows per workgroup
1 / 5 / 16 / chosen) on ragged row counts and the smallest and largest block
counts, outliers next to tiny and subnormal x in one group, fp16 edge scales
(zero, negative, subnormal, largest), x with inf / NaN (summed weight by
weight so they propagate like the fp32 matvec), the geometries it refuses,
and the default path's choice of kernel.
"""

from __future__ import annotations

import numpy as np
import pytest

from conftest import assert_matvec_close
from flatrun_amd import _lib, device, synth
from oracle import gguf_np as G
from q1_0_split import emulate

pytestmark = pytest.mark.gpu

MX = 16                                               # the kernel's work unit in frq_gemv_config.cpl


def run(raw, x, n, k, **geom):
    w = device.DeviceBuffer.from_host(raw)
    xd = device.DeviceBuffer.from_host(x)
    yd = device.DeviceBuffer(4 * n)
    try:
        cfg = device.gemv_tuned("Q1_0", w, xd, yd, n, k, kernel=_lib.GEMV_ROWS, **geom)
        device.synchronize()
        return yd.to_host(np.float32), cfg
    finally:
        w.free()
        xd.free()
        yd.free()


def check(raw, x, n, k, y, what):
    return assert_matvec_close(y, G.matmul_f64("Q1_0", x, raw, n, k), G.abs_matmul_f64("Q1_0", x, raw, n, k),
                               what=what)


@pytest.mark.parametrize("n,k", [(4096, 4096), (33, 4096), (300, 4096), (7, 256), (12, 16384), (17, 1024),
                                 (1, 768), (2048, 2304)])
def test_every_geometry(frq, n, k):
    raw = synth.make_blocks("Q1_0", n, k, seed=n + k)
    x = synth.make_x(k, seed=k)
    x[3], x[k // 2], x[-1] = 2.0**24, -3e-30, 1e-40
    nb = k // 128
    runs = 0
    for L in (1, 2, 4, 8):
        if (nb + L - 1) // L > 16:
            continue
        for tr in (0, 1, 5, 16):
            y, cfg = run(raw, x, n, k, cpl=MX, rows=tr, unroll=L)
            assert cfg["cpl"] == MX and cfg["unroll"] == L and cfg["waves_per_wg"] == (nb + L - 1) // L
            check(raw, x, n, k, y, f"{n}x{k} {cfg}")
            runs += 1
    assert runs >= 4


def test_group_outliers_and_tiny_values(frq):
    """Each group's fixed point is relative to its own largest |x|: a 2^30
    outlier next to tiny and subnormal values in one group, groups of zeros,
    a group of subnormals only, and groups spanning 2^-126 .. 2^100."""
    n, k = 1024, 4096
    raw = synth.make_blocks("Q1_0", n, k, seed=11)
    rng = np.random.default_rng(12)
    x = synth.make_x(k, seed=13)
    x[0] = 2.0**30
    x[1:32] = rng.standard_normal(31).astype(np.float32) * np.float32(1e-6)
    x[5] = 1e-42
    x[32:64] = 0.0
    x[64:96] = (rng.standard_normal(32) * 1e-40).astype(np.float32)
    for gi in range(3, k // 32):
        x[32 * gi:32 * gi + 32] *= np.float32(2.0 ** int(rng.integers(-126, 100)))
    y, cfg = run(raw, x, n, k, cpl=MX)
    assert np.all(np.isfinite(y))
    check(raw, x, n, k, y, "outliers")


def test_edge_scales(frq):
    """fp16 block scales 0, -0, negative, subnormal and 65504."""
    n, k = 2048, 4096
    raw = synth.make_blocks("Q1_0", n, k, seed=21).reshape(n, k // 128, 18).copy()
    edge = np.array([0.0, -0.0, -1.5, 6e-8, 65504.0, -65504.0, 2.0**-14], np.float16)
    raw[:, :7, 0:2] = edge.view(np.uint8).reshape(7, 2)[None, :, :]
    raw[::3, 9, 0:2] = np.array([-2.0**-24], np.float16).view(np.uint8)
    raw = raw.reshape(-1)
    x = synth.make_x(k, seed=22)
    y, _ = run(raw, x, n, k, cpl=MX)
    check(raw, x, n, k, y, "edge scales")


def test_non_finite_x(frq):
    n, k = 1024, 4096
    raw = synth.make_blocks("Q1_0", n, k, seed=3)
    W = G.dequant_q1_0(raw, (n, k)).astype(np.float64)
    for vals in ({200: np.inf}, {1000: np.nan}, {200: np.inf, 3000: -np.inf, 3001: np.inf}):
        x = synth.make_x(k, seed=4)
        for i, v in vals.items():
            x[i] = v
        with np.errstate(all="ignore"):
            ref = (W * x.astype(np.float64)[None, :]).sum(axis=1)
        y, _ = run(raw, x, n, k, cpl=MX)
        assert np.array_equal(np.isnan(y), np.isnan(ref)), vals
        assert np.array_equal(np.isinf(y), np.isinf(ref)), vals
        fin = np.isinf(ref)
        assert np.array_equal(np.sign(y[fin]), np.sign(ref[fin])), vals


def test_refused_geometries(frq):
    raw = synth.make_blocks("Q1_0", 64, 4096, seed=5)
    x = synth.make_x(4096, seed=6)
    # blocks per wavefront other than 1 / 2 / 4 / 8, more than 16 rows, and
    # 32 blocks at one per wavefront (32 > 16 wavefronts)
    for geom in (dict(unroll=3), dict(unroll=16), dict(rows=17), dict(unroll=1)):
        with pytest.raises(RuntimeError):
            run(raw, x, 64, 4096, cpl=MX, **geom)
    raw_odd = synth.make_blocks("Q1_0", 8, 384, seed=7)   # 3 blocks per row: rows not 4-byte aligned
    with pytest.raises(RuntimeError):
        run(raw_odd, synth.make_x(384, seed=8), 8, 384, cpl=MX)
    raw_long = synth.make_blocks("Q1_0", 4, 130 * 128, seed=9)
    with pytest.raises(RuntimeError):
        run(raw_long, synth.make_x(130 * 128, seed=10), 4, 130 * 128, cpl=MX)


@pytest.mark.parametrize("n,k,mx", [(4096, 4096, True), (1024, 1024, True), (6144, 2048, True), (512, 4096, False),
                                    (4096, 8192, False), (14336, 4096, False)])
def test_default_route(frq, n, k, mx):
    """The default path takes the matrix cores where they measured faster
    than the element-wise ring kernel; either way within the contract."""
    raw = synth.make_blocks("Q1_0", n, k, seed=n)
    x = synth.make_x(k, seed=n + 1)
    w = device.DeviceBuffer.from_host(raw)
    xd = device.DeviceBuffer.from_host(x)
    yd = device.DeviceBuffer(4 * n)
    try:
        cfg = device.gemv_tuned("Q1_0", w, xd, yd, n, k, kernel=_lib.GEMV_AUTO)
        device.synchronize()
        y_auto = yd.to_host(np.float32)
        device.gemv("Q1_0", w, xd, yd, n, k)
        device.synchronize()
        y_def = yd.to_host(np.float32)
    finally:
        w.free()
        xd.free()
        yd.free()
    assert (cfg["cpl"] == MX) == mx, cfg
    assert np.array_equal(y_auto.view(np.uint32), y_def.view(np.uint32))
    check(raw, x, n, k, y_def, f"default {n}x{k}")


def test_misaligned_weights_take_the_ring(frq):
    """A weight base 2 bytes off a 4-byte boundary cannot take the aligned
    sign-bit windows: the explicit request is refused, the default path runs
    another kernel with the same contract."""
    n, k = 2048, 4096
    raw = synth.make_blocks("Q1_0", n, k, seed=31)
    x = synth.make_x(k, seed=32)
    buf = device.DeviceBuffer(raw.nbytes + 16)
    host = np.zeros(raw.nbytes + 16, np.uint8)
    host[2:2 + raw.nbytes] = raw
    _lib.check(_lib.lib().frq_memcpy_h2d(buf.ptr, host.ctypes.data, host.nbytes))
    xd = device.DeviceBuffer.from_host(x)
    yd = device.DeviceBuffer(4 * n)
    try:
        with pytest.raises(RuntimeError):
            device.gemv_tuned("Q1_0", buf.ptr + 2, xd, yd, n, k, kernel=_lib.GEMV_ROWS, cpl=MX, w_bytes=raw.nbytes)
        cfg = device.gemv_tuned("Q1_0", buf.ptr + 2, xd, yd, n, k, kernel=_lib.GEMV_AUTO, w_bytes=raw.nbytes)
        device.synchronize()
        assert cfg["cpl"] != MX
        check(raw, x, n, k, yd.to_host(np.float32), "misaligned")
    finally:
        buf.free()
        xd.free()
        yd.free()


@pytest.mark.parametrize("n,k", [(4096, 4096), (300, 4096), (7, 256), (12, 16384), (2048, 2304), (6144, 2048)])
def test_bits_equal_model(frq, n, k):
    """The kernel's bits equal the model of its arithmetic (tests/q1_0_split.py)
    for every blocks-per-wavefront choice: every digit, sign bit and group
    lands where the model puts it, and the sums run in its order."""
    raw = synth.make_blocks("Q1_0", n, k, seed=3 * n + k)
    x = synth.make_x(k, seed=k + 5)
    x[7], x[k // 3] = 2.0**26, -(2.0**-20)
    nb = k // 128
    for L in (1, 2, 4, 8):
        if (nb + L - 1) // L > 16:
            continue
        y, cfg = run(raw, x, n, k, cpl=MX, unroll=L, rows=0 if L != 2 else 5)
        want = emulate(raw, x, n, k, L)
        assert np.array_equal(y.view(np.uint32), want.view(np.uint32)), (L, int(np.sum(y != want)))
