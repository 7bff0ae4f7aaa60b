"""The matrix-core Q4_K GEMV (int8 MFMA; frq_gemv_mx.hip) against the oracle.

Contract: the matvec tolerance (1e-5 normwise and componentwise against the
fp64 oracle) for every finite x. x is carried as a 60-bit fixed-point number
per 32-element sub-block (two levels of four 8-bit digits) relative to the
sub-block's max |x|, exact for every element within 2^36 of that maximum;
a block whose x the split cannot carry exactly (wider range, |x| >= 2^30,
inf, NaN) is computed per weight in fp32. So the cases below put outliers on
exactly-zero weight columns (the case a fixed-point split relative to the
maximum cannot hide), realistic massive activations, ranges past 2^36, and
non-finite x. Bits are independent of the rows per workgroup and of the row
tiles per wavefront for a given K-split (fixed per-row summation order); the
two halves of a K-split row combine in either arrival order to the same bits.
"""

from __future__ import annotations

import numpy as np
import pytest

from conftest import assert_matvec_close, bits_equal
from flatrun_amd import _lib, device, synth
from oracle import gguf_np as G

pytestmark = pytest.mark.gpu


# every forced launch runs each load depth of the kernel: all of a
# wavefront's weight loads issued before its x split ("all": unroll >= its
# blocks), and block j + 1's loads issued before block j's products ("ahead":
# unroll = 1)
_MX = {"kernel": _lib.GEMV_MX, "unroll": 4}


@pytest.fixture(autouse=True, params=["all", "ahead"])
def mx_depth(request):
    _MX["unroll"] = 4 if request.param == "all" else 1
    yield dict(_MX)
    _MX["unroll"] = 4


def run_mx(raw, x, n, k, rows=0, tiles=0, ksplit=0, stream=None):
    """One forced matrix-core launch."""
    w = device.DeviceBuffer.from_host(raw)
    xd = device.DeviceBuffer.from_host(x)
    yd = device.DeviceBuffer(max(4, 4 * n))
    try:
        _lib.check(_lib.lib().frq_memcpy_h2d(yd.ptr, np.full(n, np.nan, np.float32).ctypes.data, 4 * n))
        cfg = device.gemv_tuned("Q4_K", w, xd, yd, n, k, **_MX, rows=rows, cpl=tiles, slices=ksplit,
                                stream=stream)
        device.synchronize()
        return yd.to_host(np.float32)[:n], cfg
    finally:
        w.free()
        xd.free()
        yd.free()


def zero_column(raw, n, k, col):
    """raw with weight column `col` exactly zero in every row: the element's
    4-bit code and its sub-block's 6-bit min set to 0 (so w = d*sc*0 - dmin*0)."""
    nb = k // 256
    r = raw.reshape(n, nb * 144).copy()
    b, e = divmod(col, 256)
    sb = e // 32
    p, i = divmod(e, 64)
    off = b * 144
    byte = off + 16 + 32 * p + (i % 32)
    r[:, byte] &= 0xF0 if i < 32 else 0x0F
    if sb < 4:                       # m = scales[sb + 4] & 63
        r[:, off + 4 + sb + 4] &= 0xC0
    else:                            # m = scales[sb + 4] >> 4 | (scales[sb] >> 6) << 4
        r[:, off + 4 + sb + 4] &= 0x0F
        r[:, off + 4 + sb] &= 0x3F
    out = r.reshape(-1)
    assert np.all(G.dequant_q4_k(out, (n, k))[:, col] == 0)
    return out


def oracle_check(y, raw, x, n, k, what):
    return assert_matvec_close(y, G.matmul_f64("Q4_K", x, raw, n, k), G.abs_matmul_f64("Q4_K", x, raw, n, k),
                               what=what)


# nb = 1 .. 128 blocks: one half up to 16 waves x 4 blocks, two halves up to
# 2 x 64; ragged last waves, odd block counts (uneven halves), short halves
@pytest.mark.parametrize("n,k", [(1, 256), (5, 512), (16, 1024), (17, 1280), (33, 3584), (40, 4096), (7, 9472),
                                 (100, 14336), (29, 18944), (64, 20224), (50, 20480), (31, 16640), (45, 32768)])
def test_mx_shapes_tiles_rows(frq, n, k):
    raw = synth.make_blocks("Q4_K", n, k, seed=n * 7 + k)
    x = synth.make_x(k, seed=k + 1)
    nb = k // 256
    for ks in (1, 2):
        if (ks == 1 and nb > 64) or (ks == 2 and nb < 2):
            continue
        ref = None
        for tiles, rows in ((1, 16), (1, 1), (1, 3), (2, 32), (2, 2), (2, 17), (2, 28), (1, 14)):
            try:
                y, cfg = run_mx(raw, x, n, k, rows=rows, tiles=tiles, ksplit=ks)
            except RuntimeError:
                assert tiles == 2 and -(-((nb + ks - 1) // ks) // 16) > 3      # two tiles need <= 3 blocks per wave
                continue
            assert cfg["kernel"] == _lib.GEMV_MX and cfg["rows"] == rows and cfg["cpl"] == tiles
            assert cfg["slices"] == ks and cfg["items"] == -(-n // rows) * ks
            if ref is None:
                oracle_check(y, raw, x, n, k, f"mx {n}x{k} ks={ks}")
                ref = y
            else:
                assert bits_equal(y, ref), (tiles, rows, ks)   # the row tiling never changes a row's sums


@pytest.mark.parametrize("q,n,k,mx", [("Q4_K", 3584, 18944, False), ("Q4_K", 18944, 3584, False),
                                      ("Q4_K", 4096, 4096, True), ("Q4_K", 1536, 8960, False),
                                      ("Q4_K", 2000, 2048, True), ("Q4_K", 8192, 11008, True),
                                      ("Q4_K", 14336, 4096, False)])
def test_default_path_kernel_choice_full_size(frq, q, n, k, mx):
    """frq_dev_gemv takes the matrix-core kernel where it measured 5 % or more
    faster (whole rows, one round of <= 256 workgroups), the element-wise
    kernel elsewhere; the tuned entry's AUTO mode reports the same choice and
    gives the same bits; both meet the oracle."""
    raw = synth.make_blocks(q, n, k, seed=n ^ k)
    x = synth.make_x(k, seed=k + 7)
    w = device.DeviceBuffer.from_host(raw)
    xd = device.DeviceBuffer.from_host(x)
    yd = device.DeviceBuffer(4 * n)
    try:
        device.gemv(q, w, xd, yd, n, k)
        device.synchronize()
        y = yd.to_host(np.float32)
        oracle_check(y, raw, x, n, k, f"default {q} {n}x{k}")
        cfg = device.gemv_tuned(q, w, xd, yd, n, k)
        device.synchronize()
        if mx:
            assert cfg["kernel"] == _lib.GEMV_MX and cfg["slices"] == 1 and cfg["items"] <= 256, cfg
        else:
            assert cfg["kernel"] == _lib.GEMV_ROWS, cfg
        assert bits_equal(yd.to_host(np.float32), y)
    finally:
        w.free()
        xd.free()
        yd.free()


def _x_cases(k, rng):
    base = synth.make_x(k, seed=3)
    spread = (base * np.exp2(rng.integers(-40, 40, k))).astype(np.float32)   # 80 binades in every sub-block
    outlier = base.copy()
    outlier[rng.integers(0, k, 3)] = 3.0e4                                 # lone large entries
    signs = np.where(rng.random(k) < 0.5, -1.0, 1.0).astype(np.float32)
    return {
        "spread": spread,
        "outlier": outlier,
        "tiny": (base * np.float32(1e-30)).astype(np.float32),
        "subnormal": (base * np.float32(1e-40)).astype(np.float32),
        "huge": (base * np.float32(1e30)).astype(np.float32),
        "zeros": np.zeros(k, np.float32),
        "sparse": np.where(rng.random(k) < 0.05, base, 0.0).astype(np.float32),
        "pow2": (signs * np.exp2(rng.integers(-8, 8, k))).astype(np.float32),
    }


@pytest.mark.parametrize("ks", [1, 2])
def test_mx_x_ranges(frq, ks):
    n, k = 48, 4096
    raw = synth.make_blocks("Q4_K", n, k, seed=11)
    rng = np.random.default_rng(5)
    for name, x in _x_cases(k, rng).items():
        y, _ = run_mx(raw, x, n, k, ksplit=ks)
        if name == "zeros":
            assert np.array_equal(y, np.zeros(n, np.float32))
            continue
        if name == "subnormal":
            # products and sums of ~1e-40 sit in the fp32 subnormal range for
            # every kernel; the check is that the scale round-trips (no zeroing)
            y64 = G.matmul_f64("Q4_K", x, raw, n, k)
            assert np.all(np.isfinite(y)) and np.max(np.abs(y - y64)) <= 1e-3 * np.max(np.abs(y64))
            continue
        oracle_check(y, raw, x, n, k, f"x {name} ks={ks}")


@pytest.mark.parametrize("n,k,ks", [(64, 4096, 1), (64, 4096, 2), (3584, 18944, 0)])
def test_mx_outlier_on_zero_weight_column(frq, n, k, ks):
    """An exactly-zero weight column (q = 0 and the sub-block's min 0) under
    x outliers of 2^20, 2^24 and 2^28, the rest N(0, 1): the outlier sets
    its sub-block's scale but multiplies nothing, so every other element of
    the sub-block must keep its own fp32 precision."""
    raw = zero_column(synth.make_blocks("Q4_K", n, k, seed=61), n, k, 0)
    for big in (2.0**20, 2.0**24, 2.0**28):
        x = synth.make_x(k, seed=62)
        x[0] = big
        y, cfg = run_mx(raw, x, n, k, ksplit=ks)
        nw, cw = oracle_check(y, raw, x, n, k, f"zero column, x[0] = {big:g}, {cfg}")
        assert nw <= 1e-6 and cw <= 1e-6, (big, nw, cw)


def test_mx_outliers_on_zero_columns_every_sub_block(frq):
    """Zero columns at every sub-block position of a block (lo / hi nibble
    planes, both loads), each with its own large outlier; and the same x
    against the unmodified weights."""
    n, k = 96, 2048
    raw = synth.make_blocks("Q4_K", n, k, seed=63)
    cols = [256 * b + 32 * s + (7 * s + b) % 32 for b in range(k // 256) for s in range(8)]
    rz = raw
    for c in cols:
        rz = zero_column(rz, n, k, c)
    x = synth.make_x(k, seed=64)
    x[cols] = np.float32(2.0**22) * np.where(np.arange(len(cols)) % 2, -1, 1)
    for r in (rz, raw):
        y, _ = run_mx(r, x, n, k)
        oracle_check(y, r, x, n, k, "zero columns under outliers")


@pytest.mark.parametrize("ks", [1, 2])
def test_mx_massive_activations(frq, ks):
    """A few channels at 1e3 .. 1e4 (the massive activations of LLM hidden
    states) among N(0, 1) channels, some of the others tiny."""
    n, k = 512, 4096
    raw = synth.make_blocks("Q4_K", n, k, seed=65)
    rng = np.random.default_rng(66)
    x = synth.make_x(k, seed=67)
    idx = rng.choice(k, 12, replace=False)
    x[idx] = (rng.uniform(1e3, 1e4, 12) * rng.choice([-1, 1], 12)).astype(np.float32)
    x[rng.choice(k, 40, replace=False)] *= np.float32(1e-6)
    y, _ = run_mx(raw, x, n, k, ksplit=ks)
    oracle_check(y, raw, x, n, k, f"massive activations ks={ks}")


@pytest.mark.parametrize("ks", [1, 2])
def test_mx_per_weight_blocks(frq, ks):
    """Sub-blocks whose x the 60-bit split cannot carry exactly (a range past
    2^36 on a zero column; |x| >= 2^30) go through the per-weight fp32 form
    block by block: the values meet the tolerance."""
    n, k = 40, 4096
    raw0 = synth.make_blocks("Q4_K", n, k, seed=68)
    raw = zero_column(raw0, n, k, 0)
    cases = []
    x = synth.make_x(k, seed=69)
    x[0], x[1] = 2.0**40, 3.0e-7                                   # 2^40 range in sub-block 0
    cases.append(("range 2^40 on a zero column", raw, x))
    x = synth.make_x(k, seed=70)
    x[300] = 3.0e9                                                 # max |x| >= 2^30
    cases.append(("|x| >= 2^30", raw0, x))
    x = synth.make_x(k, seed=71)
    x[::97] *= np.float32(2.0**60)                                 # many blocks, huge magnitudes
    cases.append(("2^60 scattered", raw0, x))
    for name, r, xx in cases:
        y, _ = run_mx(r, xx, n, k, ksplit=ks)
        oracle_check(y, r, xx, n, k, f"{name} ks={ks}")


@pytest.mark.parametrize("ks", [1, 2])
def test_mx_nonfinite_x(frq, ks):
    """Outside the contract (finite inputs), but defined: a block holding an
    inf or NaN is computed per weight, as the reference computes it: rows
    whose weight on that column is nonzero come out inf / NaN, others stay
    finite only if the reference's per-weight form keeps them so."""
    n, k = 20, 1024
    raw = synth.make_blocks("Q4_K", n, k, seed=2)
    for bad in (np.inf, -np.inf, np.nan):
        x = synth.make_x(k, seed=4)
        x[300] = bad
        y, _ = run_mx(raw, x, n, k, ksplit=ks)
        w = G.dequant_q4_k(raw, (n, k))
        with np.errstate(invalid="ignore"):
            ref = w.astype(np.float64) @ x.astype(np.float64)
        assert np.array_equal(np.isfinite(y), np.isfinite(ref)), bad
        assert not np.any(np.isfinite(y)), bad       # synthetic weights are nonzero on column 300


def test_mx_repeat_and_graph_replay(frq):
    n, k = 3584, 18944
    raw = synth.make_blocks("Q4_K", n, k, seed=21)
    x = synth.make_x(k, seed=22)
    w = device.DeviceBuffer.from_host(raw)
    xd = device.DeviceBuffer.from_host(x)
    yd = device.DeviceBuffer(4 * n)
    s = device.Stream()
    try:
        device.gemv_tuned("Q4_K", w, xd, yd, n, k, **_MX, stream=s)
        s.synchronize()
        ref = yd.to_host(np.float32)
        for _ in range(10):
            device.gemv_tuned("Q4_K", w, xd, yd, n, k, **_MX, stream=s)
        s.synchronize()
        assert bits_equal(yd.to_host(np.float32), ref)
        with device.Graph.capture(s) as cap:
            device.gemv_tuned("Q4_K", w, xd, yd, n, k, **_MX, stream=s)
        try:
            for _ in range(3):
                _lib.check(_lib.lib().frq_memcpy_h2d(yd.ptr, np.full(n, np.nan, np.float32).ctypes.data, 4 * n))
                cap.launch(s)
                s.synchronize()
                assert bits_equal(yd.to_host(np.float32), ref)
        finally:
            cap.destroy()
    finally:
        w.free()
        xd.free()
        yd.free()
        s.destroy()


def test_mx_batched_rows(frq):
    """frq_dev_gemv with batch 3 (Q4_K): every row meets the oracle."""
    n, k, b = 2048, 4096, 3
    raw = synth.make_blocks("Q4_K", n, k, seed=31)
    xs = synth.make_x(k, seed=32, batch=b)
    w = device.DeviceBuffer.from_host(raw)
    xd = device.DeviceBuffer.from_host(xs)
    yd = device.DeviceBuffer(4 * n * b)
    try:
        device.gemv("Q4_K", w, xd, yd, n, k, batch=b)
        device.synchronize()
        ys = yd.to_host(np.float32).reshape(b, n)
        for i in range(b):
            oracle_check(ys[i], raw, xs[i], n, k, f"batch row {i}")
    finally:
        w.free()
        xd.free()
        yd.free()


def test_mx_k_split_halves_any_order(frq):
    """K-split rows: repeated launches (the halves race to the slot in
    whatever order the hardware runs them) give identical bits, and the
    per-row slots are left at zero (the next launch of another shape on the
    same stream is still right)."""
    s = device.Stream()
    try:
        shapes = [(3584, 18944, 81), (4096, 4096, 82), (700, 16384, 83)]
        bufs = []
        for n, k, seed in shapes:
            raw = synth.make_blocks("Q4_K", n, k, seed=seed)
            x = synth.make_x(k, seed=seed + 1)
            bufs.append((n, k, raw, x, device.DeviceBuffer.from_host(raw), device.DeviceBuffer.from_host(x),
                         device.DeviceBuffer(4 * n)))
        ref = []
        for n, k, raw, x, w, xd, yd in bufs:
            cfg = device.gemv_tuned("Q4_K", w, xd, yd, n, k, **_MX, slices=2, stream=s)
            assert cfg["slices"] == 2
            s.synchronize()
            y = yd.to_host(np.float32)
            oracle_check(y, raw, x, n, k, f"k-split {n}x{k}")
            ref.append(y)
        for _ in range(30):
            for n, k, raw, x, w, xd, yd in bufs:
                device.gemv_tuned("Q4_K", w, xd, yd, n, k, **_MX, slices=2, stream=s)
        s.synchronize()
        for (n, k, *_, yd), r in zip(bufs, ref):
            assert bits_equal(yd.to_host(np.float32), r)
        for *_, w, xd, yd in bufs:
            w.free()
            xd.free()
            yd.free()
    finally:
        s.destroy()


def test_mx_rejects(frq):
    raw = synth.make_blocks("Q4_K", 4, 256 * 129, seed=1)
    w = device.DeviceBuffer.from_host(raw)
    xd = device.DeviceBuffer(4 * 256 * 129)
    yd = device.DeviceBuffer(64)
    q5 = device.DeviceBuffer.from_host(synth.make_blocks("Q5_K", 4, 512, seed=1))
    q6 = device.DeviceBuffer.from_host(synth.make_blocks("Q6_K", 4, 512, seed=1))
    try:
        with pytest.raises(RuntimeError):                      # 129 blocks: beyond 2 halves x 16 waves x 4 blocks
            device.gemv_tuned("Q4_K", w, xd, yd, 4, 256 * 129, **_MX)
        with pytest.raises(RuntimeError):                      # 65 blocks in one workgroup
            device.gemv_tuned("Q4_K", w, xd, yd, 4, 256 * 65, **_MX, slices=1, w_bytes=4 * 65 * 144)
        with pytest.raises(RuntimeError):                      # rows per workgroup above 16 per tile
            device.gemv_tuned("Q4_K", w, xd, yd, 4, 256, **_MX, rows=17, cpl=1, w_bytes=4 * 144)
        with pytest.raises(RuntimeError):                      # three tiles
            device.gemv_tuned("Q4_K", w, xd, yd, 4, 256, **_MX, cpl=3, w_bytes=4 * 144)
        with pytest.raises(RuntimeError):                      # Q4_K only
            device.gemv_tuned("Q5_K", q5, xd, yd, 4, 512, **_MX)
        with pytest.raises(RuntimeError):
            device.gemv_tuned("Q6_K", q6, xd, yd, 4, 512, **_MX)
        # the default path still serves k beyond the matrix-core limits
        device.gemv("Q4_K", w, xd, yd, 4, 256 * 129)
        device.synchronize()
    finally:
        for b in (w, xd, yd, q5, q6):
            b.free()


@pytest.mark.parametrize("ks", [1, 2])
def test_mx_outliers_on_cancelling_weights(frq, ks):
    """An outlier x of 2^24 (and -2^20) on ordinary weight columns, where
    some rows have d*sc*q close to dmin*m: each sub-block is combined from
    exact integer sums in fp64 and rounded once, so the error stays within
    2^-24 of the sub-block's own sum_j w_j x_j and the componentwise bound
    (1e-5 of sum_j |w_j x_j|) holds for every row."""
    n, k = 512, 4096 * ks
    raw = synth.make_blocks("Q4_K", n, k, seed=300 + ks)
    x = synth.make_x(k, seed=301)
    x[5] = 2.0**24
    x[1000] = -(2.0**20)
    x[777] = 3.0e4
    y, _ = run_mx(raw, x, n, k, ksplit=ks)
    oracle_check(y, raw, x, n, k, f"cancelling weights ks={ks}")
