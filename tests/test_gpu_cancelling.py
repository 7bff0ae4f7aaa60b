"""Every GPU matvec path on exactly-cancelling weights with outlier x.

Columns whose weights are exactly zero while their block scales are not
(tests/cancelling.py: Q4_K / Q5_K with d * sc = dmin * m and code 1, Q6_K
code 32, Q8_0 code 0) meet x outliers of 2^24, -2^20 and 2^28. A matvec that
forms a sub-block as s * sum(q x) - t * sum(x) (or subtracts 32 sum(x) or
128 sum(x)) cancels two terms of size |t x_j| there and misses the bound by
orders of magnitude (the CPU test beside this one shows it on an fp32
emulation); the contract -- 1e-5 of sum_j |w_ij x_j| per row, and of max |y|
-- must hold on every kernel: the defaults per format and shape, each
explicit launch geometry of the element-wise and split-K kernels, both
matrix-core GEMV layouts, the batched GEMM, the small-M matvec, the grouped
launch and the no-allocation entry point.
"""

from __future__ import annotations

import numpy as np
import pytest

from cancelling import cancel_columns, outlier_x
from conftest import assert_matvec_close
from flatrun_amd import _lib, device, synth
from oracle import gguf_np as G

pytestmark = pytest.mark.gpu


def _cols(q, k):
    be = synth.BLOCK[q][1]
    cols = [5, min(k - 1, be + 37), k - 3]
    if k >= 4 * be:
        cols.append(2 * be + be // 2 + 1)
    return sorted(set(cols))


def _input(q, n, k, seed):
    cols = _cols(q, k)
    raw = cancel_columns(q, synth.make_blocks(q, n, k, seed=seed), n, k, cols)
    return raw, cols


def _check(q, raw, x, n, k, y, what):
    y64 = G.matmul_f64(q, x, raw, n, k)
    a64 = G.abs_matmul_f64(q, x, raw, n, k)
    if np.ndim(x) == 1:
        assert_matvec_close(y, y64, a64, what=what)
    else:
        for r in range(x.shape[0]):
            assert_matvec_close(y[r], y64[r], a64[r], what=f"{what} row {r}")


def _run(q, raw, x, n, k, kernel=None, **geom):
    w = device.DeviceBuffer.from_host(raw)
    xd = device.DeviceBuffer.from_host(x)
    batch = 1 if np.ndim(x) == 1 else x.shape[0]
    yd = device.DeviceBuffer(4 * n * batch)
    try:
        if kernel is None:
            device.gemv(q, w, xd, yd, n, k, batch=batch)
            cfg = None
        else:
            cfg = device.gemv_tuned(q, w, xd, yd, n, k, kernel=kernel, **geom)
        device.synchronize()
        y = yd.to_host(np.float32)
        return (y if batch == 1 else y.reshape(batch, n)), cfg
    finally:
        w.free()
        xd.free()
        yd.free()


DEFAULT_SHAPES = [
    ("Q4_K", 512, 4096), ("Q4_K", 1024, 4096), ("Q4_K", 2048, 4096), ("Q4_K", 1536, 8960),
    ("Q4_K", 3584, 18944), ("Q4_K", 64, 40960),
    ("Q5_K", 300, 4096), ("Q5_K", 64, 14336),
    ("Q6_K", 1024, 4096), ("Q6_K", 4096, 14336), ("Q6_K", 200, 3584),
    ("Q8_0", 4864, 896), ("Q8_0", 256, 4096), ("Q8_0", 70, 14336),
]


@pytest.mark.parametrize("q,n,k", DEFAULT_SHAPES)
def test_default_path(frq, q, n, k):
    raw, cols = _input(q, n, k, seed=n + k)
    x = outlier_x(k, cols, seed=k)
    y, _ = _run(q, raw, x, n, k)
    _check(q, raw, x, n, k, y, f"{q} {n}x{k} default")


@pytest.mark.parametrize("q,n,k", [("Q4_K", 96, 4096), ("Q4_K", 40, 18944), ("Q5_K", 70, 4096),
                                   ("Q6_K", 64, 4096), ("Q6_K", 33, 14336), ("Q8_0", 70, 4096),
                                   ("Q8_0", 48, 896)])
def test_every_geometry(frq, q, n, k):
    """Element-wise (register ring) and split-K kernels, each work
    unit size, rows per workgroup and ring depth the library accepts."""
    raw, cols = _input(q, n, k, seed=3 * n + k)
    x = outlier_x(k, cols, seed=k + 1)
    kernels = [_lib.GEMV_SPLITK, _lib.GEMV_ROWS]
    runs = 0
    for kernel in kernels:
        for cpl in (1, 2, 4, 8):
            for rows in (1, 4, 7, 16):
                for unroll in (2, 4):
                    try:
                        y, cfg = _run(q, raw, x, n, k, kernel=kernel, cpl=cpl, rows=rows, unroll=unroll)
                    except RuntimeError:
                        continue                       # geometry not valid for this format / k
                    _check(q, raw, x, n, k, y, f"{q} {n}x{k} {cfg}")
                    runs += 1
    assert runs >= 6


@pytest.mark.parametrize("n,k", [(2048, 4096), (1536, 8960), (3584, 18944), (18944, 3584)])
@pytest.mark.parametrize("depth", [1, 4])
def test_matrix_core_load_depths(frq, n, k, depth):
    raw, cols = _input("Q4_K", n, k, seed=n)
    x = outlier_x(k, cols, seed=n + 1)
    y, cfg = _run("Q4_K", raw, x, n, k, kernel=_lib.GEMV_MX, unroll=depth)
    _check("Q4_K", raw, x, n, k, y, f"Q4_K {n}x{k} {cfg}")


@pytest.mark.parametrize("q,n,k", [("Q4_K", 3584, 18944), ("Q4_K", 512, 4096), ("Q6_K", 1024, 4096),
                                   ("Q8_0", 4864, 896), ("Q5_K", 128, 4096)])
@pytest.mark.parametrize("seq", [2, 3, 4, 5, 33])
def test_batched(frq, q, n, k, seq):
    """The fp32 GEMM for two or more rows (per-row GEMVs for Q5_K, the
    small-M matvec for a few rows of Q4_K, Q6_K and Q8_0), outliers in every
    row, each row with another outlier set."""
    raw, cols = _input(q, n, k, seed=n + seq)
    xs = np.stack([outlier_x(k, cols, seed=100 + r, big=(2.0**(20 + r % 9), -(2.0**24), 3.0e4)) for r in range(seq)])
    y, _ = _run(q, raw, xs, n, k)
    _check(q, raw, xs, n, k, y, f"{q} {n}x{k} seq {seq}")


@pytest.mark.parametrize("batch", [1, 3])
def test_grouped(frq, batch):
    """q | k | v of a Llama layer (Q4_K, Q4_K, Q6_K) in one grouped call."""
    k = 4096
    spec = [("Q4_K", 4096), ("Q4_K", 1024), ("Q6_K", 1024)]
    cols = _cols("Q4_K", k)
    raws = [cancel_columns(q, synth.make_blocks(q, n, k, seed=60 + i), n, k, cols) for i, (q, n) in enumerate(spec)]
    x = np.stack([outlier_x(k, cols, seed=70 + b) for b in range(batch)])
    ws = [device.DeviceBuffer.from_host(r) for r in raws]
    xd = device.DeviceBuffer.from_host(x)
    tot = sum(n for _, n in spec)
    yd = device.DeviceBuffer(4 * batch * tot)
    try:
        parts, off = [], 0
        for (q, n), w, r in zip(spec, ws, raws):
            parts.append((q, w, n, yd.ptr + 4 * off, r.nbytes))
            off += n
        device.gemv_group(parts, xd, k, batch=batch, y_stride=tot)
        device.synchronize()
        y = yd.to_host(np.float32).reshape(batch, tot)
    finally:
        for b in ws + [xd, yd]:
            b.free()
    off = 0
    for (q, n), r in zip(spec, raws):
        _check(q, r, x, n, k, y[:, off:off + n], f"group {q} {n}")
        off += n


@pytest.mark.parametrize("q,n,k", [("Q4_K", 3584, 18944), ("Q4_K", 300, 33024), ("Q6_K", 1024, 4096)])
def test_noalloc(frq, q, n, k):
    raw, cols = _input(q, n, k, seed=n + 9)
    x = outlier_x(k, cols, seed=k + 9)
    w = device.DeviceBuffer.from_host(raw)
    xd = device.DeviceBuffer.from_host(x)
    yd = device.DeviceBuffer(4 * n)
    try:
        _lib.check(_lib.lib().frq_dev_gemv_noalloc(device.qtype_id(q), w.ptr, raw.nbytes, xd.ptr, yd.ptr, n, k, 1,
                                                   None))
        device.synchronize()
        y = yd.to_host(np.float32)
    finally:
        for b in (w, xd, yd):
            b.free()
    _check(q, raw, x, n, k, y, f"noalloc {q} {n}x{k}")
