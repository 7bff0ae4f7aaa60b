"""Grouped GEMV (frq_dev_gemv_group / NativeBackend.matmul_fused) on the GPU.

Contract: laid out as the forwarder's np.concatenate of the projections
(model/qwen2.py:1510-1519, 1690-1702). Fused into one launch for Q4_K / Q6_K
matrices, whose outputs are bit for bit those of separate launches of the
element-wise kernels (frq_dev_gemv_tuned with FRQ_GEMV_ROWS: same per-row
arithmetic; two Q4_K matrices of one shape share one row ring per workgroup,
same bits); one frq_dev_gemv launch per matrix otherwise, with its bits.
Values are checked against the fp64 oracle as well (1e-5 normwise and
componentwise, fp32 accumulation).
"""

from __future__ import annotations

import numpy as np
import pytest

from conftest import assert_matvec_close, bits_equal
from flatrun_amd import DeviceWeight, NativeBackend, _lib, device, synth
from oracle import gguf_np as G

pytestmark = pytest.mark.gpu

LLAMA_QKV = [("Q4_K", 4096), ("Q4_K", 1024), ("Q6_K", 1024)]
LLAMA_GATE_UP = [("Q4_K", 14336), ("Q4_K", 14336)]


def run_group(parts_spec, k, seed=0, batch=1, concat=True):
    """parts_spec: [(qtype, n)]. Returns (grouped output, separate outputs, raws, x)."""
    raws = [synth.make_blocks(q, n, k, seed=seed + i) for i, (q, n) in enumerate(parts_spec)]
    x = synth.make_x(k, seed=seed + 50, batch=batch) if batch > 1 else synth.make_x(k, seed=seed + 50)
    ws = [device.DeviceBuffer.from_host(r) if r.size else None for r in raws]
    xd = device.DeviceBuffer.from_host(x)
    ns = [n for _, n in parts_spec]
    total = sum(ns)
    yd = device.DeviceBuffer(max(4, batch * total * 4))
    try:
        grp, off = [], 0
        for (q, n), w, r in zip(parts_spec, ws, raws):
            grp.append((q, w if w is not None else 0, n, yd.ptr + 4 * off, r.nbytes))
            off += n
        device.gemv_group(grp, xd, k, batch=batch, y_stride=total)
        device.synchronize()
        y = yd.to_host(np.float32)[: batch * total].reshape(batch, total)
        fusable = device.gemv_group_fusable([(q, w if w is not None else 0) for (q, _), w in zip(parts_spec, ws)], k)
        sep = []
        for (q, n), w, r in zip(parts_spec, ws, raws):
            ys = device.DeviceBuffer(max(4, batch * n * 4))
            if n and fusable and batch == 1:       # the element-wise kernels
                for b in range(batch):
                    device.gemv_tuned(q, w, xd.ptr + 4 * b * k, ys.ptr + 4 * b * n, n, k, kernel=_lib.GEMV_ROWS,
                                      w_bytes=r.nbytes)
            elif n:
                device.gemv(q, w, xd, ys, n, k, batch=batch, w_bytes=r.nbytes)
            device.synchronize()
            sep.append(ys.to_host(np.float32)[: batch * n].reshape(batch, n))
            ys.free()
    finally:
        for w in ws:
            if w is not None:
                w.free()
        xd.free()
        yd.free()
    return y, np.concatenate(sep, axis=1), raws, x, fusable


@pytest.mark.parametrize("spec", [LLAMA_QKV, LLAMA_GATE_UP], ids=["qkv", "gate_up"])
def test_llama_groups_fused_and_exact(frq, spec):
    k = 4096
    y, ysep, raws, x, fusable = run_group(spec, k, seed=7)
    assert fusable
    assert bits_equal(y, ysep)
    off = 0
    for (q, n), r in zip(spec, raws):
        assert_matvec_close(y[0, off:off + n], G.matmul_f64(q, x, r, n, k), G.abs_matmul_f64(q, x, r, n, k),
                            what=f"group {q} {n}x{k}")
        off += n


@pytest.mark.parametrize("spec,k", [
    ([("Q4_K", 5), ("Q4_K", 3)], 256),                      # R = 4, ragged last workgroup
    ([("Q6_K", 3), ("Q4_K", 2)], 512),                      # tiny segments, mixed
    ([("Q4_K", 37), ("Q6_K", 64), ("Q4_K", 9), ("Q6_K", 130)], 1024),   # four segments
    ([("Q4_K", 9000), ("Q6_K", 9000)], 512),                # total > 8192: R from the occupancy rule
    ([("Q6_K", 300), ("Q4_K", 0), ("Q6_K", 7)], 2048),      # empty middle segment
    ([("Q4_K", 700), ("Q4_K", 300)], 18944),                # 10-wave workgroups
    ([("Q4_K", 3000), ("Q6_K", 2000)], 3584),
    # two Q4_K matrices of one shape: one ring over the same rows of both
    ([("Q4_K", 5), ("Q4_K", 5)], 256),                      # 2 rows of each, ragged last workgroup
    ([("Q4_K", 1001), ("Q4_K", 1001)], 4096),
    ([("Q4_K", 777), ("Q4_K", 777)], 18944),                # 10-wave workgroups
    ([("Q4_K", 9000), ("Q4_K", 9000)], 512),                # 4 rows of each
    ([("Q4_K", 0), ("Q4_K", 300), ("Q4_K", 300)], 1024),    # an empty segment, then a pair
])
def test_group_shapes_bit_identical(frq, spec, k):
    y, ysep, *_, fusable = run_group(spec, k, seed=len(spec) + k)
    assert fusable
    assert bits_equal(y, ysep)


@pytest.mark.parametrize("spec,k", [
    ([("Q8_0", 96), ("Q4_K", 64)], 4096),                   # Q8_0 has no grouped body
    ([("Q5_K", 40), ("Q1_0", 33)], 1024),
    ([("Q4_K", 40), ("Q4_K", 33)], 34816),                  # 136 blocks x 8 lanes > 1024: split-K
    ([("Q6_K", 40)], 768),                                  # odd block count: no ring kernel
    ([("Q4_K", 5)], 256),                                   # one matrix: one frq_dev_gemv launch
    ([("Q4_K", 4096)], 4096),                               # one matrix on the matrix cores
    ([("Q6_K", 300)], 3584),
])
def test_group_fallback_bit_identical(frq, spec, k):
    y, ysep, *_, fusable = run_group(spec, k, seed=3)
    assert not fusable
    assert bits_equal(y, ysep)


def test_group_batched_concat(frq):
    """x of 3 rows: row b of every matrix lands at b * (sum n) + offset."""
    y, ysep, raws, xs, _ = run_group(LLAMA_QKV, 4096, seed=11, batch=3)
    assert y.shape == (3, 6144) and bits_equal(y, ysep)
    q, n = LLAMA_QKV[2]
    assert_matvec_close(y[2, 5120:], G.matmul_f64(q, xs[2], raws[2], n, 4096),
                        G.abs_matmul_f64(q, xs[2], raws[2], n, 4096), what="batched row 2, v")


def test_facade_matmul_fused(frq):
    """matmul_fused equals the concatenation of the per-matrix products: to
    the oracle's tolerance (the separate q product runs on the matrix cores),
    and bit for bit between host and resident weights."""
    nb = NativeBackend()
    k = 4096
    parts = [(q, synth.make_blocks(q, n, k, seed=20 + i), n) for i, (q, n) in enumerate(LLAMA_QKV)]
    meth = {"Q4_K": nb.matmul_q4k, "Q6_K": nb.matmul_q6k}
    for x in (synth.make_x(k, seed=1), synth.make_x(k, seed=2, batch=2)):
        want = np.concatenate([meth[q](x, r, n, k) for q, r, n in parts], axis=-1)
        got = nb.matmul_fused(x, parts, k)
        assert got.shape == want.shape
        xs = np.atleast_2d(x)
        off = 0
        for q, r, n in parts:
            for b in range(xs.shape[0]):
                assert_matvec_close(np.atleast_2d(got)[b, off:off + n], G.matmul_f64(q, xs[b], r, n, k),
                                    G.abs_matmul_f64(q, xs[b], r, n, k), what=f"fused {q} {n}")
            off += n
        dev = [(q, nb.upload(r), n) for q, r, n in parts]
        assert bits_equal(nb.matmul_fused(x, dev, k), got)
    with pytest.raises(ValueError):
        nb.matmul_fused(np.zeros(k + 1, np.float32), parts, k)
    with pytest.raises(ValueError):
        nb.matmul_fused(np.zeros(k, np.float32), parts * 2, k)


def test_facade_matmul_fused_small_weight_cache(frq):
    """A weight cache smaller than the group: looking up a later part must
    not free an earlier part of the same call before the launch. Parts that
    do not fit beside the held ones go up for the call alone; the result is
    the uncached one bit for bit, on repeated calls (hits and misses mixed)."""
    k = 4096
    parts = [(q, synth.make_blocks(q, n, k, seed=40 + i), n) for i, (q, n) in enumerate(LLAMA_QKV)]
    sizes = [r.nbytes for _, r, _ in parts]                  # 9.4 MB, 2.4 MB, 3.4 MB
    plain = NativeBackend(weight_cache=False)
    small = NativeBackend(weight_cache=sizes[0] + sizes[1] // 2)   # holds q, not q and k
    x = synth.make_x(k, seed=5)
    want = plain.matmul_fused(x, parts, k)
    for rep in range(3):
        got = small.matmul_fused(x, parts, k)
        assert bits_equal(got, want), rep
    st = small.cache_stats()
    assert st["bytes"] <= st["capacity"] and st["entries"] >= 1
    gu = [(q, synth.make_blocks(q, n, k, seed=60 + i), n) for i, (q, n) in enumerate(LLAMA_GATE_UP)]
    one = NativeBackend(weight_cache=gu[0][1].nbytes + 1024)  # gate and up (58.7 MB each) never fit together
    want = plain.matmul_fused(x, gu, k)
    for rep in range(2):
        assert bits_equal(one.matmul_fused(x, gu, k), want), rep


def test_group_graph_replay(frq):
    k = 4096
    spec = LLAMA_QKV
    raws = [synth.make_blocks(q, n, k, seed=30 + i) for i, (q, n) in enumerate(spec)]
    ws = [device.DeviceBuffer.from_host(r) for r in raws]
    xd = device.DeviceBuffer.from_host(synth.make_x(k, seed=31))
    total = sum(n for _, n in spec)
    yd = device.DeviceBuffer(total * 4)
    s = device.Stream()
    grp, off = [], 0
    for (q, n), w, r in zip(spec, ws, raws):
        grp.append((q, w, n, yd.ptr + 4 * off, r.nbytes))
        off += n
    try:
        device.gemv_group(grp, xd, k, stream=s)
        s.synchronize()
        eager = yd.to_host(np.float32)
        with device.Graph.capture(s) as cap:
            device.gemv_group(grp, xd, k, stream=s)
        for _ in range(3):
            _lib.check(_lib.lib().frq_memcpy_h2d(yd.ptr, np.full(total, np.nan, np.float32).ctypes.data, total * 4))
            cap.launch(s)
            s.synchronize()
            assert bits_equal(yd.to_host(np.float32), eager)
        cap.destroy()
    finally:
        for w in ws:
            w.free()
        xd.free()
        yd.free()
        s.destroy()


def test_group_errors(frq):
    lib = _lib.lib()
    w = device.DeviceBuffer(144 * 4)
    x = device.DeviceBuffer(256 * 4)
    y = device.DeviceBuffer(64)
    try:
        with pytest.raises(ValueError):
            device.gemv_group([], x, 256)
        with pytest.raises(ValueError):
            device.gemv_group([("Q4_K", w, 4, y)] * 5, x, 256)
        with pytest.raises(RuntimeError):                      # byte size does not match n x k
            device.gemv_group([("Q4_K", w, 3, y, 144 * 4)], x, 256)
        assert lib.frq_dev_gemv_group(0, None, None, None, None, None, 256, None, 1, 0, None) != 0
    finally:
        w.free()
        x.free()
        y.free()
