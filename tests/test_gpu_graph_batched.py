"""Captured graphs of the batched and fp16 paths replay to the eager bits.

A HIP graph replays the kernels a capture recorded with the pointers and
scratch they were given then. The batched matvec (frq_gemm_f32.hip) writes
fp32 partial planes into stream scratch and adds them in a second kernel
when it splits K, the few-row route runs one small-M kernel launch per
two or three rows, and the fp16 dequant is a plain kernel; each
is captured once, replayed four times with y clobbered before and eager
launches of other shapes (which reuse the same scratch) between the
replays, and every replay must give the eager result bit for bit.
"""

from __future__ import annotations

import numpy as np
import pytest

from conftest import bits_equal
from flatrun_amd import _lib, device, synth

pytestmark = pytest.mark.gpu

# (format, n, k, rows of x): 32-, 64- and 128-row tiles, split and unsplit
# grids, and the small-M route for a few rows.
CASES = [
    ("Q4_K", 3584, 18944, 7), ("Q4_K", 3584, 18944, 2), ("Q4_K", 1536, 8960, 3), ("Q4_K", 3584, 18944, 5),
    ("Q6_K", 4096, 14336, 7), ("Q8_0", 4864, 896, 3),
    ("Q4_K", 14336, 4096, 200), ("Q6_K", 1024, 4096, 100), ("Q6_K", 4096, 14336, 40),
    ("Q8_0", 4864, 896, 33), ("Q8_0", 4096, 4096, 512),
]


def _nan_fill(buf, count):
    nan = np.full(count, np.nan, np.float32)
    _lib.check(_lib.lib().frq_memcpy_h2d(buf.ptr, nan.ctypes.data, nan.nbytes))


def test_batched_graph_replay(frq):
    s = device.Stream()
    bufs = []
    try:
        for i, (q, n, k, m) in enumerate(CASES):
            raw = synth.make_blocks(q, n, k, seed=90 + i)
            xs = synth.make_x(k, seed=95 + i, batch=m)
            bufs.append((q, n, k, m, raw.nbytes, device.DeviceBuffer.from_host(raw), device.DeviceBuffer.from_host(xs),
                         device.DeviceBuffer(4 * n * m)))

        def run(sel):
            for q, n, k, m, nb, w, xd, yd in sel:
                device.gemv(q, w, xd, yd, n, k, batch=m, stream=s, w_bytes=nb)

        run(bufs)
        s.synchronize()
        eager = [yd.to_host(np.float32) for *_, yd in bufs]
        with device.Graph.capture(s) as cap:
            run(bufs)
        try:
            for rep in range(4):
                for q, n, k, m, *_, yd in bufs:
                    _nan_fill(yd, n * m)
                cap.launch(s)
                s.synchronize()
                for (q, n, k, m, *_, yd), ref in zip(bufs, eager):
                    assert bits_equal(yd.to_host(np.float32), ref), (rep, q, n, k, m)
                run(bufs[rep::3])                           # eager launches on the same scratch
                s.synchronize()
        finally:
            cap.destroy()
    finally:
        for *_, w, xd, yd in bufs:
            w.free()
            xd.free()
            yd.free()
        s.destroy()


@pytest.mark.parametrize("q,n,k", [("Q4_K", 2048, 4096), ("Q6_K", 1024, 3584), ("Q8_0", 300, 896),
                                   ("Q5_K", 64, 4096), ("Q1_0", 128, 4096)])
def test_dequant_f16_graph_replay(frq, q, n, k):
    raw = synth.make_blocks(q, n, k, seed=n + 7)
    s = device.Stream()
    w = device.DeviceBuffer.from_host(raw)
    yd = device.DeviceBuffer(2 * n * k)
    try:
        device.dequant_f16(q, w, yd, n * k, stream=s, w_bytes=raw.nbytes)
        s.synchronize()
        ref = yd.to_host(np.uint16)
        with device.Graph.capture(s) as cap:
            device.dequant_f16(q, w, yd, n * k, stream=s, w_bytes=raw.nbytes)
        try:
            for rep in range(3):
                ones = np.full(n * k, 0x7E00, np.uint16)            # fp16 NaN
                _lib.check(_lib.lib().frq_memcpy_h2d(yd.ptr, ones.ctypes.data, ones.nbytes))
                cap.launch(s)
                s.synchronize()
                assert np.array_equal(yd.to_host(np.uint16), ref), rep
        finally:
            cap.destroy()
    finally:
        w.free()
        yd.free()
        s.destroy()
