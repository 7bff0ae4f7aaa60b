"""Grouped prefill GEMM (frq_dev_gemm_bf16_group): up to four matrices that
multiply the same bf16 x in one launch, against the oracle and against one
frq_dev_gemm_bf16 launch per matrix.

Contract (written here, checked below):
  * each matrix's block of the output is within MATVEC_RTOL (1e-5) of fp64
    X . bf16(W_i)^T, as for the single GEMM (check() of test_gpu_gemm);
  * where the group splits K as each matrix alone would, the outputs are
    those of the single launches bit for bit;
  * repeated launches and graph replays give the same bits.
"""

from __future__ import annotations

import numpy as np
import pytest

from conftest import bits_equal
from flatrun_amd import _C, _lib, device, synth
from test_gpu_gemm import check, make_case

pytestmark = pytest.mark.gpu


def run_group(parts, xb, m, k, y_stride=0):
    """parts: [(qtype, raw, n)]; returns the per-matrix outputs (m x n_i each),
    read from one concatenated buffer when y_stride is set."""
    s = device.Stream()
    bufs = [device.DeviceBuffer.from_host(raw) for _, raw, _ in parts]
    xd = device.DeviceBuffer.from_host(_C.to_bf16_bits(xb))
    ns = [n for _, _, n in parts]
    try:
        if y_stride:
            yd = device.DeviceBuffer(4 * m * y_stride)
            offs = np.concatenate([[0], np.cumsum(ns)[:-1]]).astype(int)
            specs = [(q, b, n, yd.ptr + 4 * int(o), raw.nbytes) for (q, raw, n), b, o in zip(parts, bufs, offs)]
            device.gemm_bf16_group(specs, xd, m, k, y_stride=y_stride, stream=s)
            s.synchronize()
            y = yd.to_host(np.float32, m * y_stride).reshape(m, y_stride)
            yd.free()
            return [y[:, o:o + n].copy() for o, n in zip(offs, ns)]
        yds = [device.DeviceBuffer(4 * max(m * n, 1)) for n in ns]
        specs = [(q, b, n, yb, raw.nbytes) for (q, raw, n), b, yb in zip(parts, bufs, yds)]
        device.gemm_bf16_group(specs, xd, m, k, stream=s)
        s.synchronize()
        out = [yb.to_host(np.float32, m * n).reshape(m, n) for yb, n in zip(yds, ns)]
        for yb in yds:
            yb.free()
        return out
    finally:
        for b in bufs:
            b.free()
        xd.free()
        s.destroy()


def single(q, raw, xb, n, k):
    return _C.matmul_bf16(q, xb, raw, n, k)


def test_group_llama_qkv(frq):
    """Llama-3-8B q|k|v at 256 tokens (Q4_K, Q4_K, Q6_K; 48 tiles, K split in
    4 for the group where k and v alone split in 8): each block against the
    oracle and, to the matvec tolerance, against its own launch."""
    m, k = 256, 4096
    parts = [("Q4_K", 4096, 31), ("Q4_K", 1024, 32), ("Q6_K", 1024, 33)]
    xb = make_case(m, 1, k, seed=30)[1]
    raws = [synth.make_blocks(q, n, k, seed=sd) for q, n, sd in parts]
    ys = run_group([(q, raw, n) for (q, n, _), raw in zip(parts, raws)], xb, m, k, y_stride=6144)
    for (q, n, _), raw, y in zip(parts, raws, ys):
        check(y, raw, xb, n, k, q=q)
        ref = single(q, raw, xb, n, k)
        assert np.max(np.abs(y - ref)) <= 1e-5 * max(1.0, np.max(np.abs(ref)))


def test_group_same_split_bit_identical(frq):
    """Two 8320-row matrices at 512 tokens: alone and together one K-split
    (130 and 260 tiles), so the group gives each launch's bits; mixed formats,
    dense outputs."""
    m, k = 512, 512
    xb = make_case(m, 1, k, seed=40)[1]
    parts = [("Q4_K", synth.make_blocks("Q4_K", 8320, k, seed=41), 8320),
             ("Q6_K", synth.make_blocks("Q6_K", 8320, k, seed=42), 8320)]
    ys = run_group(parts, xb, m, k)
    for (q, raw, n), y in zip(parts, ys):
        assert bits_equal(y, single(q, raw, xb, n, k)), q


@pytest.mark.parametrize("m", [1, 300])
def test_group_ragged_three_formats(frq, m):
    """Ragged rows and columns, Q4_K | Q8_0 | Q6_K, concatenated output."""
    k = 1024
    parts = [("Q4_K", 200), ("Q8_0", 37), ("Q6_K", 129)]
    xb = make_case(m, 1, k, seed=50 + m)[1]
    raws = [synth.make_blocks(q, n, k, seed=51 + i) for i, (q, n) in enumerate(parts)]
    ys = run_group([(q, raw, n) for (q, n), raw in zip(parts, raws)], xb, m, k, y_stride=400)
    for (q, n), raw, y in zip(parts, raws, ys):
        check(y, raw, xb, n, k, q=q)


def test_group_single_and_empty_segments(frq):
    """A group of one matrix with a dense output is frq_dev_gemm_bf16; a
    segment of zero rows is skipped."""
    m, k = 40, 512
    xb = make_case(m, 1, k, seed=60)[1]
    raw = synth.make_blocks("Q4_K", 300, k, seed=61)
    (y,) = run_group([("Q4_K", raw, 300)], xb, m, k)
    assert bits_equal(y, single("Q4_K", raw, xb, 300, k))
    ys = run_group([("Q4_K", raw, 300), ("Q6_K", np.zeros(0, np.uint8), 0)], xb, m, k)
    check(ys[0], raw, xb, 300, k)


def test_group_repeat_and_graph_replay(frq):
    """Same bits on repeated launches and on graph replays (the split partials
    live in the stream's scratch)."""
    m, k = 256, 4096
    xb = make_case(m, 1, k, seed=70)[1]
    raws = [synth.make_blocks("Q4_K", 4096, k, seed=71), synth.make_blocks("Q6_K", 1024, k, seed=72)]
    s = device.Stream()
    bufs = [device.DeviceBuffer.from_host(r) for r in raws]
    xd = device.DeviceBuffer.from_host(_C.to_bf16_bits(xb))
    yd = device.DeviceBuffer(4 * m * 5120)
    specs = [("Q4_K", bufs[0], 4096, yd.ptr, raws[0].nbytes), ("Q6_K", bufs[1], 1024, yd.ptr + 4 * 4096, raws[1].nbytes)]
    try:
        device.gemm_bf16_group(specs, xd, m, k, y_stride=5120, stream=s)
        s.synchronize()
        y0 = yd.to_host(np.float32, m * 5120)
        check(y0.reshape(m, 5120)[:, :4096], raws[0], xb, 4096, k)
        with device.Graph.capture(s) as cap:
            device.gemm_bf16_group(specs, xd, m, k, y_stride=5120, stream=s)
        for _ in range(3):
            _lib.check(_lib.lib().frq_memcpy_h2d(yd.ptr, np.full(m * 5120, np.nan, np.float32).ctypes.data, m * 5120 * 4))
            cap.launch(s)
            s.synchronize()
            assert bits_equal(yd.to_host(np.float32, m * 5120), y0)
        cap.destroy()
    finally:
        for b in bufs + [xd, yd]:
            b.free()
        s.destroy()


def test_facade_matmul_fused_bf16(frq):
    """NativeBackend.matmul_fused_bf16: the concatenation of the per-matrix
    prefill GEMMs, from raw bytes or resident weights, 2-D and 1-D x."""
    from flatrun_amd import NativeBackend

    nb = NativeBackend()
    m, k = 24, 512
    xb = make_case(m, 1, k, seed=80)[1]
    parts = [("Q4_K", synth.make_blocks("Q4_K", 96, k, seed=81), 96),
             ("Q6_K", synth.make_blocks("Q6_K", 40, k, seed=82), 40)]
    y = nb.matmul_fused_bf16(xb, parts, k)
    assert y.shape == (m, 136)
    check(y[:, :96], parts[0][1], xb, 96, k)
    check(y[:, 96:], parts[1][1], xb, 40, k, q="Q6_K")
    dev = [(q, nb.upload(raw), n) for q, raw, n in parts]
    assert bits_equal(nb.matmul_fused_bf16(xb, dev, k), y)
    assert bits_equal(nb.matmul_fused_bf16(xb[3], parts, k), y[3])


def test_group_k_zero_fills(frq):
    """k = 0: every output is 0, dense or strided."""
    m = 5
    s = device.Stream()
    yd = device.DeviceBuffer(4 * m * 12)
    try:
        _lib.check(_lib.lib().frq_memcpy_h2d(yd.ptr, np.full(m * 12, np.nan, np.float32).ctypes.data, m * 12 * 4))
        device.gemm_bf16_group([("Q4_K", 0, 4, yd.ptr, 0), ("Q6_K", 0, 8, yd.ptr + 16, 0)], 0, m, 0, y_stride=12,
                               stream=s)
        s.synchronize()
        assert np.array_equal(yd.to_host(np.float32, m * 12), np.zeros(m * 12, np.float32))
        _lib.check(_lib.lib().frq_memcpy_h2d(yd.ptr, np.full(m * 12, np.nan, np.float32).ctypes.data, m * 12 * 4))
        device.gemm_bf16_group([("Q4_K", 0, 12, yd.ptr, 0)], 0, m, 0, stream=s)
        s.synchronize()
        assert np.array_equal(yd.to_host(np.float32, m * 12), np.zeros(m * 12, np.float32))
    finally:
        yd.free()
        s.destroy()
