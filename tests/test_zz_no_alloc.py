"""frq_dev_gemv_noalloc against frq_dev_gemv, through the C ABI.

The no-allocation entry point runs the same kernels as frq_dev_gemv with
its scratch in one fixed device array per GPU, so its results must equal
frq_dev_gemv's bit for bit. Each case makes two calls in a row, the second
on a smaller shape (the array keeps the first call's contents), covering
every scratch user of the default path: split-K rows (partials), the
batched GEMM (K-split partial planes and its per-row flags), and kernels
with no scratch. Shapes whose scratch would not fit are refused before any
launch.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

from conftest import bits_equal
from flatrun_amd import _lib, device, synth

pytestmark = pytest.mark.gpu


def _noalloc(q, w, x, y, n, k, batch=1, stream=None, w_bytes=None):
    wb = w.nbytes if w_bytes is None else w_bytes
    return _lib.lib().frq_dev_gemv_noalloc(device.qtype_id(q), w.ptr, wb, x.ptr, y.ptr, n, k, batch,
                                           0 if stream is None else stream.handle)


def _case(q, n, k, batch, seed, stream):
    raw = synth.make_blocks(q, n, k, seed=seed)
    xs = synth.make_x(k, seed=seed + 1, batch=batch)
    w = device.DeviceBuffer.from_host(raw)
    xd = device.DeviceBuffer.from_host(xs)
    y_ref = device.DeviceBuffer(4 * n * batch)
    y_na = device.DeviceBuffer(4 * n * batch)
    nan = np.full(n * batch, np.nan, np.float32)
    _lib.check(_lib.lib().frq_memcpy_h2d(y_na.ptr, nan.ctypes.data, nan.nbytes))
    try:
        device.gemv(q, w, xd, y_ref, n, k, batch=batch, stream=stream)
        _lib.check(_noalloc(q, w, xd, y_na, n, k, batch=batch, stream=stream))
        stream.synchronize()
        a, b = y_ref.to_host(np.float32), y_na.to_host(np.float32)
        assert np.all(np.isfinite(b)), (q, n, k)
        assert bits_equal(a, b), (q, n, k)
    finally:
        for buf in (w, xd, y_ref, y_na):
            buf.free()


@pytest.mark.parametrize("q,shapes", [
    ("Q4_K", [(3584, 18944, 1), (2048, 18944, 1)]),     # element-wise, no scratch
    ("Q4_K", [(8192, 4096, 1), (4096, 4096, 1)]),       # matrix cores, whole rows: no scratch
    ("Q4_K", [(4096, 14336, 1), (1536, 8960, 2)]),      # then a batched call (small-M matvec)
    ("Q4_K", [(512, 4096, 40), (128, 4096, 12)]),       # batched GEMM: K-split partials and row flags
    ("Q4_K", [(1024, 4096, 8), (300, 14336, 4)]),       # fp32 matrix-core small batches: no scratch
    ("Q4_K", [(300, 33024, 1), (100, 33024, 1)]),       # k > 32768: split-K partials
    ("Q6_K", [(1024, 4096, 1), (512, 4096, 1)]),        # no scratch
    ("Q8_0", [(4864, 896, 1), (1000, 896, 1)]),
    ("Q1_0", [(4096, 4096, 1), (2048, 4096, 2)]),       # Q1_0 on the matrix cores: no scratch
])
def test_noalloc_equals_dev_gemv_two_calls(frq, q, shapes):
    s = device.Stream()
    try:
        for i, (n, k, batch) in enumerate(shapes):
            _case(q, n, k, batch, seed=100 + 7 * i + n, stream=s)
    finally:
        s.destroy()


def test_noalloc_graph_replay(frq):
    """Captured in a graph (the callers it is for): replays equal eager bits."""
    n, k = 3584, 18944
    raw = synth.make_blocks("Q4_K", n, k, seed=5)
    x = synth.make_x(k, seed=6)
    w, xd, yd = device.DeviceBuffer.from_host(raw), device.DeviceBuffer.from_host(x), device.DeviceBuffer(4 * n)
    s = device.Stream()
    try:
        _lib.check(_noalloc("Q4_K", w, xd, yd, n, k, stream=s))
        s.synchronize()
        ref = yd.to_host(np.float32)
        with device.Graph.capture(s) as cap:
            _lib.check(_noalloc("Q4_K", w, xd, yd, n, k, stream=s))
        try:
            for _ in range(3):
                device.copy(yd, xd, 16, stream=s)
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


def test_noalloc_refuses_oversized_scratch(frq):
    """Split-K partials past 3 MiB (one row of x, and two rows that run one
    GEMV each): refused with FRQ_ERR_UNSUPPORTED, nothing launched (the
    output keeps its contents). The buffers are real, of full size. (The
    default path no longer splits matrix-core rows in halves, so no default
    shape needs the row-exchange slots.)"""
    cases = []
    # split-K: learn the slice count for k = 33024, then ask for enough rows
    probe_raw = synth.make_blocks("Q4_K", 4, 33024, seed=1)
    pw, px, py = (device.DeviceBuffer.from_host(probe_raw), device.DeviceBuffer.from_host(synth.make_x(33024, seed=2)),
                  device.DeviceBuffer(16))
    cfg = device.gemv_tuned("Q4_K", pw, px, py, 4, 33024, kernel=_lib.GEMV_SPLITK)
    device.synchronize()
    for b in (pw, px, py):
        b.free()
    slices = cfg["slices"]
    cases.append(("Q4_K", (3 << 20) // (4 * slices) + 64, 33024, 1))
    # two rows of a matrix the small-M kernel does not take (k > 24576) run
    # one GEMV per row: the same per-row scratch, refused the same way
    cases.append(("Q4_K", (3 << 20) // (4 * slices) + 64, 33024, 2))
    for q, n, k, batch in (c if len(c) == 4 else c + (1,) for c in cases):
        wbytes = synth.nbytes(q, n, k)
        w = device.DeviceBuffer(wbytes)
        xd = device.DeviceBuffer(4 * k * batch)
        yd = device.DeviceBuffer(4 * n * batch)
        try:
            mark = np.full(n * batch, 7.0, np.float32)
            _lib.check(_lib.lib().frq_memcpy_h2d(yd.ptr, mark.ctypes.data, mark.nbytes))
            rc = _noalloc(q, w, xd, yd, n, k, batch=batch)
            assert rc == _lib.ERR_UNSUPPORTED, rc
            assert "fixed scratch" in _lib.lib().frq_last_error().decode()
            device.synchronize()
            assert np.array_equal(yd.to_host(np.float32), mark)
        finally:
            w.free()
            xd.free()
            yd.free()


def test_noalloc_symbol_declared():
    """The entry point is exported and bound like the others."""
    fn = _lib.lib().frq_dev_gemv_noalloc
    assert fn.restype is ctypes.c_int and len(fn.argtypes) == 9
