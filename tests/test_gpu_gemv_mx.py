"""The matrix-core Q4_K / Q6_K GEMVs (int8 MFMA; frq_gemv_mx.hip) against the oracle.

Contract: the matvec tolerance (1e-5 normwise and componentwise
against the fp64 oracle); bits independent of the rows-per-workgroup choice
and of launch order (fixed per-row summation order); the default device path
takes the Q4_K kernel for n > 1280 and k <= 20480 (the Q6_K kernel, k <=
16384, only through the tuned entry: slower than the Q6_K ring). x is split
into four 8-bit digits per 32-element sub-block relative to the sub-block's
max |x|, so the cases below include x spread over many binades inside a
sub-block, tiny and huge x, zeros, and a lone outlier. Q6_K blocks are 210 B:
odd block counts and a 2-byte weight offset exercise the unaligned loads.
"""

from __future__ import annotations

import numpy as np
import pytest

from conftest import assert_matvec_close, bits_equal
from flatrun_amd import _lib, device, synth
from oracle import gguf_np as G

pytestmark = pytest.mark.gpu


def run_mx(raw, x, n, k, rows=0, q="Q4_K", w_offset=0):
    """One forced matrix-core launch; the weights sit w_offset bytes into their buffer."""
    w = device.DeviceBuffer.from_host(np.concatenate([np.zeros(w_offset, np.uint8), raw]))
    xd = device.DeviceBuffer.from_host(x)
    yd = device.DeviceBuffer(max(4, 4 * n))
    try:
        _lib.check(_lib.lib().frq_memcpy_h2d(yd.ptr, np.full(n, np.nan, np.float32).ctypes.data, 4 * n))
        cfg = device.gemv_tuned(q, w.ptr + w_offset, xd, yd, n, k, kernel=_lib.GEMV_MX, rows=rows,
                                w_bytes=raw.nbytes)
        device.synchronize()
        return yd.to_host(np.float32)[:n], cfg
    finally:
        w.free()
        xd.free()
        yd.free()


def oracle_check(y, raw, x, n, k, what, q="Q4_K"):
    assert_matvec_close(y, G.matmul_f64(q, x, raw, n, k), G.abs_matmul_f64(q, x, raw, n, k), what=what)


# Q4_K: nb = 1 .. 80 blocks (1 .. 5 per wave); Q6_K: nb = 1 .. 64 (1 .. 4 per
# wave), odd counts putting every other block at 2 mod 4; ragged last waves
@pytest.mark.parametrize("q,n,k", [("Q4_K", 1, 256), ("Q4_K", 5, 512), ("Q4_K", 16, 1024), ("Q4_K", 17, 1280),
                                   ("Q4_K", 33, 3584), ("Q4_K", 40, 4096), ("Q4_K", 7, 9472), ("Q4_K", 100, 14336),
                                   ("Q4_K", 29, 18944), ("Q4_K", 64, 20224), ("Q4_K", 50, 20480),
                                   ("Q6_K", 1, 256), ("Q6_K", 9, 768), ("Q6_K", 16, 1280), ("Q6_K", 33, 3584),
                                   ("Q6_K", 21, 4352), ("Q6_K", 40, 9472), ("Q6_K", 70, 14336), ("Q6_K", 19, 16384)])
def test_mx_shapes_and_rows(frq, q, n, k):
    raw = synth.make_blocks(q, n, k, seed=n * 7 + k)
    x = synth.make_x(k, seed=k + 1)
    ref = None
    for rows in (16, 1, 3, 8, 14):
        y, cfg = run_mx(raw, x, n, k, rows, q=q)
        assert cfg["kernel"] == _lib.GEMV_MX and cfg["rows"] == rows
        assert cfg["items"] == -(-n // rows)
        if ref is None:
            oracle_check(y, raw, x, n, k, f"mx {q} {n}x{k}", q=q)
            ref = y
        else:
            assert bits_equal(y, ref), rows      # the row tiling never changes a row's sums


def test_mx_q6_k_unaligned_weights(frq):
    """Q6_K weights 2 bytes into their buffer (every block at 2 mod 4 or 0 mod 4
    in turn, no 16-byte alignment anywhere): same bits as the aligned copy."""
    q, n, k = "Q6_K", 37, 3328
    raw = synth.make_blocks(q, n, k, seed=8)
    x = synth.make_x(k, seed=9)
    y0, _ = run_mx(raw, x, n, k, q=q)
    y2, _ = run_mx(raw, x, n, k, q=q, w_offset=2)
    oracle_check(y0, raw, x, n, k, "Q6_K aligned", q=q)
    assert bits_equal(y0, y2)


@pytest.mark.parametrize("q,n,k", [("Q4_K", 3584, 18944), ("Q4_K", 18944, 3584), ("Q4_K", 4096, 4096),
                                   ("Q4_K", 1536, 8960), ("Q4_K", 2000, 2048)])
def test_mx_default_path_full_size(frq, q, n, k):
    """frq_dev_gemv takes the matrix-core kernel for these shapes; the tuned
    entry's AUTO mode reports it and gives the same bits."""
    raw = synth.make_blocks(q, n, k, seed=n ^ k)
    x = synth.make_x(k, seed=k + 7)
    w = device.DeviceBuffer.from_host(raw)
    xd = device.DeviceBuffer.from_host(x)
    yd = device.DeviceBuffer(4 * n)
    try:
        device.gemv(q, w, xd, yd, n, k)
        device.synchronize()
        y = yd.to_host(np.float32)
        oracle_check(y, raw, x, n, k, f"default {q} {n}x{k}", q=q)
        cfg = device.gemv_tuned(q, w, xd, yd, n, k)
        device.synchronize()
        assert cfg["kernel"] == _lib.GEMV_MX and 6 <= cfg["rows"] <= 16
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


@pytest.mark.parametrize("q", ["Q4_K", "Q6_K"])
def test_mx_x_ranges(frq, q):
    n, k = 48, 4096
    raw = synth.make_blocks(q, n, k, seed=11)
    rng = np.random.default_rng(5)
    for name, x in _x_cases(k, rng).items():
        y, _ = run_mx(raw, x, n, k, q=q)
        if name == "zeros":
            assert np.array_equal(y, np.zeros(n, np.float32))
            continue
        if name == "subnormal":
            # products and sums of ~1e-40 sit in the fp32 subnormal range for
            # every kernel; the check is that the scale round-trips (no zeroing)
            y64 = G.matmul_f64(q, x, raw, n, k)
            assert np.all(np.isfinite(y)) and np.max(np.abs(y - y64)) <= 1e-3 * np.max(np.abs(y64))
            continue
        oracle_check(y, raw, x, n, k, f"{q} x {name}", q=q)


@pytest.mark.parametrize("q", ["Q4_K", "Q6_K"])
def test_mx_nonfinite_x_gives_nonfinite_y(frq, q):
    """Outside the contract (finite inputs); documented behaviour: every row
    whose dot product meets an inf or NaN comes out inf or NaN."""
    n, k = 20, 1024
    raw = synth.make_blocks(q, n, k, seed=2)
    for bad in (np.inf, -np.inf, np.nan):
        x = synth.make_x(k, seed=4)
        x[300] = bad
        y, _ = run_mx(raw, x, n, k, q=q)
        assert not np.any(np.isfinite(y)), bad


@pytest.mark.parametrize("n,k", [(4096, 14336), (3584, 3584)])
def test_mx_q6_k_full_size_forced(frq, n, k):
    """The Q6_K matrix-core kernel at the Llama down / Qwen q shapes, forced."""
    raw = synth.make_blocks("Q6_K", n, k, seed=n + k)
    x = synth.make_x(k, seed=k + 5)
    y, cfg = run_mx(raw, x, n, k, q="Q6_K")
    assert cfg["kernel"] == _lib.GEMV_MX
    oracle_check(y, raw, x, n, k, f"Q6_K {n}x{k}", q="Q6_K")


def test_mx_repeat_and_graph_replay(frq):
    n, k = 3584, 18944
    raw = synth.make_blocks("Q4_K", n, k, seed=21)
    x = synth.make_x(k, seed=22)
    w = device.DeviceBuffer.from_host(raw)
    xd = device.DeviceBuffer.from_host(x)
    yd = device.DeviceBuffer(4 * n)
    s = device.Stream()
    try:
        device.gemv_tuned("Q4_K", w, xd, yd, n, k, kernel=_lib.GEMV_MX, stream=s)
        s.synchronize()
        ref = yd.to_host(np.float32)
        for _ in range(10):
            device.gemv_tuned("Q4_K", w, xd, yd, n, k, kernel=_lib.GEMV_MX, stream=s)
        s.synchronize()
        assert bits_equal(yd.to_host(np.float32), ref)
        with device.Graph.capture(s) as cap:
            device.gemv("Q4_K", w, xd, yd, n, k, stream=s)
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
    """frq_dev_gemv with batch 3 runs the kernel once per x row."""
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
            y1, _ = run_mx(raw, xs[i], n, k)
            assert bits_equal(ys[i], y1)
    finally:
        w.free()
        xd.free()
        yd.free()


def test_mx_rejects(frq):
    raw = synth.make_blocks("Q4_K", 4, 256 * 81, seed=1)
    w = device.DeviceBuffer.from_host(raw)
    xd = device.DeviceBuffer(4 * 256 * 81)
    yd = device.DeviceBuffer(64)
    q5 = device.DeviceBuffer.from_host(synth.make_blocks("Q5_K", 4, 512, seed=1))
    q6 = device.DeviceBuffer.from_host(synth.make_blocks("Q6_K", 4, 256 * 65, seed=1))
    try:
        with pytest.raises(RuntimeError):                      # 81 blocks: beyond 16 waves x 5 blocks
            device.gemv_tuned("Q4_K", w, xd, yd, 4, 256 * 81, kernel=_lib.GEMV_MX)
        with pytest.raises(RuntimeError):                      # Q6_K: 65 blocks, beyond 16 waves x 4 blocks
            device.gemv_tuned("Q6_K", q6, xd, yd, 4, 256 * 65, kernel=_lib.GEMV_MX)
        with pytest.raises(RuntimeError):                      # rows per workgroup above 16
            device.gemv_tuned("Q4_K", w, xd, yd, 4, 256, kernel=_lib.GEMV_MX, rows=17, w_bytes=4 * 144)
        with pytest.raises(RuntimeError):                      # Q4_K and Q6_K only
            device.gemv_tuned("Q5_K", q5, xd, yd, 4, 512, kernel=_lib.GEMV_MX)
        # the default path still serves k beyond the matrix-core limits
        device.gemv("Q4_K", w, xd, yd, 4, 256 * 81)
        device.gemv("Q6_K", q6, xd, yd, 4, 256 * 65)
        device.synchronize()
    finally:
        for b in (w, xd, yd, q5, q6):
            b.free()
