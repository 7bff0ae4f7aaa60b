"""dequant_handle on the GPU (flatrun_amd.loader; the reference's
src/flatrun/dequant/loader.py:51-88) against the oracle's decoders cast the
way the reference's _finish casts (gguf.py:61-73: fp32 array, astype):
bit for bit in float16 (the default), float32 and float64, for every
format, ragged sizes, and fp16 edge cases (overflow to inf, subnormals,
signed zeros, NaN scales). Also the device entry point frq_dev_dequant_f16
on a strided-free device buffer."""

from __future__ import annotations

import mmap
from types import SimpleNamespace as NS

import numpy as np
import pytest

from flatrun_amd import device, loader, synth
from oracle import gguf_np as G

pytestmark = pytest.mark.gpu


def handle(q, shape, raw):
    view = np.frombuffer(raw.tobytes(), dtype=np.uint8)      # read-only, like an mmap slice
    return NS(metadata=NS(quantization=q, shape=shape), as_numpy=lambda: view)


def same_bits(a, b):
    """Equal bit patterns, NaN positions equal (payloads may differ)."""
    a, b = np.asarray(a), np.asarray(b)
    if a.shape != b.shape or a.dtype != b.dtype:
        return False
    na, nb = np.isnan(a), np.isnan(b)
    if not np.array_equal(na, nb):
        return False
    u = {2: np.uint16, 4: np.uint32, 8: np.uint64}[a.dtype.itemsize]
    return np.array_equal(a[~na].view(u), b[~nb].view(u))


def expect(q, raw, shape, dtype):
    return G.DEQUANT[q](raw, shape, np.float32).astype(dtype)


SHAPES = [(64, 512), (7, 300), (1, 129), (3, 4096)]


@pytest.mark.parametrize("q", loader.GGUF_DECODERS)
@pytest.mark.parametrize("dtype", ["float16", "float32", "float64"])
def test_formats_and_dtypes(frq, q, dtype):
    be = synth.BLOCK[q][1]
    for i, shape in enumerate(SHAPES):
        size = int(np.prod(shape))
        nblk = -(-size // be)
        raw = synth.make_blocks(q, nblk, be, seed=10 * i + len(q))
        out = loader.dequant_handle(handle(q, shape, raw), dtype=dtype)
        assert out.shape == shape and out.dtype == np.dtype(dtype)
        assert same_bits(out, expect(q, raw, shape, dtype)), (q, shape, dtype)


def _set_f16(col2, v):
    col2[:] = np.frombuffer(np.float16(v).tobytes(), np.uint8)


@pytest.mark.parametrize("q", ["Q8_0", "Q4_K", "Q6_K", "Q5_1", "Q1_0"])
def test_fp16_edges(frq, q):
    """Scales that push values past fp16's range (inf), into its subnormal
    range, to signed zeros, and NaN scales."""
    bb, be = synth.BLOCK[q]
    nblk = 8
    raw = synth.make_blocks(q, nblk, be, seed=77).reshape(nblk, bb)
    d_off = {"Q8_0": 0, "Q4_K": 0, "Q6_K": 208, "Q5_1": 0, "Q1_0": 0}[q]
    for b, d in enumerate([60000.0, 2.0**-24, 2.0**-20, -0.0, 0.0, np.nan, -3.0e4, 1.5]):
        _set_f16(raw[b, d_off:d_off + 2], d)
        if q == "Q4_K":                           # dmin too
            _set_f16(raw[b, 2:4], d if b != 1 else 2.0**-14)
        if q == "Q5_1":                           # the added min too
            _set_f16(raw[b, 2:4], d)
    raw = raw.reshape(-1)
    shape = (nblk * be,)
    for dtype in ("float16", "float32"):
        out = loader.dequant_handle(handle(q, shape, raw), dtype=dtype)
        ref = expect(q, raw, shape, dtype)
        assert same_bits(out, ref), (q, dtype)
    o16 = loader.dequant_handle(handle(q, shape, raw))
    assert np.isinf(o16).any() or q == "Q1_0"   # the 60000 block overflows fp16 once scaled (not for +-d)
    sub = np.abs(o16[np.isfinite(o16)])
    assert ((sub > 0) & (sub < np.float16(2.0**-14))).any()     # fp16 subnormals kept


def test_device_entry_point(frq):
    q, n, k = "Q4_K", 96, 4096
    raw = synth.make_blocks(q, n, k, seed=5)
    w = device.DeviceBuffer.from_host(raw)
    y = device.DeviceBuffer(2 * n * k + 2)
    try:
        device.dequant_f16(q, w, y, n * k)
        device.synchronize()
        got = y.to_host(np.uint16)[: n * k].view(np.float16).reshape(n, k)
        assert same_bits(got, expect(q, raw, (n, k), np.float16))
        with pytest.raises(RuntimeError):                        # 2-byte alignment of y
            device.dequant_f16(q, w, y.ptr + 1, n * k)
    finally:
        w.free()
        y.free()


def test_mmap_handle_like_the_reference(frq, tmp_path):
    """A handle whose as_numpy() slices an mmap (a fresh bytes copy per call,
    as MmapTensorHandle.view does, core/tensor.py:240-247)."""
    q, shape = "Q6_K", (40, 3584)
    raw = synth.make_blocks(q, *shape, seed=9)
    p = tmp_path / "t.bin"
    p.write_bytes(b"\0" * 64 + raw.tobytes())
    with open(p, "rb") as f, mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ) as mm:
        h = NS(metadata=NS(quantization=q, shape=shape),
               as_numpy=lambda: np.ndarray(shape=(raw.size,), dtype=np.uint8, buffer=mm[64:64 + raw.size]))
        assert same_bits(loader.dequant_handle(h), expect(q, raw, shape, np.float16))
