"""Streamed layer weights (pinned host -> device ring, copy / compute streams)
give the same bits as the same GEMVs on resident weights."""

from __future__ import annotations

import numpy as np
import pytest

from conftest import bits_equal
from flatrun_amd import device, synth
from flatrun_amd.streaming import LayerStreamer

pytestmark = pytest.mark.gpu

TENSORS = [("a", "Q4_K", 64, 512), ("b", "Q6_K", 48, 768), ("c", "Q8_0", 40, 256)]


@pytest.mark.parametrize("depth", [1, 2, 3])
def test_streamed_equals_resident(frq, depth):
    n_layers, stride = 5, 256
    st = LayerStreamer(TENSORS, n_layers, depth=depth)
    blocks = [{name: synth.make_blocks(q, n, k, seed=100 * L + i) for i, (name, q, n, k) in enumerate(TENSORS)}
              for L in range(n_layers)]
    for L in range(n_layers):
        st.fill(L, blocks[L])
    x = device.DeviceBuffer.from_host(synth.make_x(768, seed=7))
    y = device.DeviceBuffer(n_layers * len(TENSORS) * stride)
    zeros = device.DeviceBuffer.from_host(np.zeros(y.nbytes, np.uint8))
    s = device.Stream()
    try:
        for rep in range(2):                       # the second pass reuses every slot again
            device.copy(y, zeros, y.nbytes, stream=s)    # clear
            st.step(x, y, s, y_stride=stride)
            s.synchronize()
            out = y.to_host(np.float32).reshape(n_layers, len(TENSORS), stride // 4)
            for L in range(n_layers):
                for t, (name, q, n, k) in enumerate(TENSORS):
                    w = device.DeviceBuffer.from_host(blocks[L][name])
                    yr = device.DeviceBuffer(4 * n)
                    device.gemv(q, w, x, yr, n, k, stream=s)
                    s.synchronize()
                    assert bits_equal(out[L, t, :n], yr.to_host(np.float32)), (rep, L, name)
    finally:
        st.close()


@pytest.mark.parametrize("nbytes", [0, 16, 48, 4096, 16 * 1000003, 38281216])
def test_read_xor_checksum(frq, nbytes):
    """The streaming read kernel (the read-only bandwidth reference) XORs every
    32-bit word once: the fold of its output words equals NumPy's XOR,
    including sizes that split unevenly over workgroups, and every word past
    the grid is overwritten with zero (the output starts as garbage)."""
    rng = np.random.default_rng(nbytes)
    host = rng.integers(0, 2**32, max(nbytes // 4, 4), dtype=np.uint32)
    src = device.DeviceBuffer.from_host(host)
    out = device.DeviceBuffer.from_host(rng.integers(0, 2**32, device.READ_XOR_WORDS, dtype=np.uint32))
    try:
        device.read_xor(src, nbytes, out)
        device.synchronize()
        words = out.to_host(np.uint32)
        assert int(np.bitwise_xor.reduce(words)) == int(np.bitwise_xor.reduce(host[:nbytes // 4]))
        grid = min(device.READ_XOR_WORDS, max(1, -(-nbytes // 4096)))
        assert not np.any(words[grid:])
    finally:
        src.free()
        out.free()
