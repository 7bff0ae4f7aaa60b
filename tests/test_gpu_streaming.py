"""Streamed layer weights (pinned host -> device ring, copy / compute streams)
give the same bits as the same GEMVs on resident weights."""

from __future__ import annotations

import numpy as np
import pytest

from conftest import assert_matvec_close, bits_equal
from flatrun_amd import device, synth
from flatrun_amd.streaming import LayerStreamer
from oracle import gguf_np as G

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


# one Llama-3-8B decoder layer, the Q4_K_M projection mix (139 MB of blocks)
LLAMA_LAYER = [("q", "Q4_K", 4096, 4096), ("k", "Q4_K", 1024, 4096), ("v", "Q6_K", 1024, 4096),
               ("o", "Q4_K", 4096, 4096), ("gate", "Q4_K", 14336, 4096), ("up", "Q4_K", 14336, 4096),
               ("down", "Q6_K", 4096, 14336)]


def test_streamed_llama3_8b_layers(frq):
    """The streamed decode sweep at its real shapes: depth + 2 = 5 Llama-3-8B
    layers (139 MB ring slots, each layer different bytes) through a ring of
    3 device slots, twice over. Every output equals, bit for bit, the same
    GEMV on a resident copy of that tensor (the default device path); layer
    0 is also checked against the fp64 oracle."""
    depth, n_layers = 3, 5
    st = LayerStreamer(LLAMA_LAYER, n_layers, depth=depth)
    assert st.layer_bytes >= 138_903_552
    kmax = max(k for *_, k in LLAMA_LAYER)
    stride = 4 * max(n for _, _, n, _ in LLAMA_LAYER)
    blocks = []
    for L in range(n_layers):
        b = {name: synth.make_blocks(q, n, k, seed=1000 * L + i) for i, (name, q, n, k) in enumerate(LLAMA_LAYER)}
        st.fill(L, b)
        blocks.append(b)
    x_host = synth.make_x(kmax, seed=77)
    x = device.DeviceBuffer.from_host(x_host)
    y = device.DeviceBuffer(n_layers * len(LLAMA_LAYER) * stride)
    s = device.Stream()
    try:
        outs = []
        for rep in range(2):
            st.step(x, y, s, y_stride=stride)
            s.synchronize()
            outs.append(y.to_host(np.float32).reshape(n_layers, len(LLAMA_LAYER), stride // 4))
        assert bits_equal(outs[0], outs[1])
        out = outs[0]
        for L in range(n_layers):
            for t, (name, q, n, k) in enumerate(LLAMA_LAYER):
                w = device.DeviceBuffer.from_host(blocks[L][name])
                yr = device.DeviceBuffer(4 * n)
                try:
                    device.gemv(q, w, x, yr, n, k, stream=s)
                    s.synchronize()
                    assert bits_equal(out[L, t, :n], yr.to_host(np.float32)), (L, name)
                finally:
                    w.free()
                    yr.free()
        for t, (name, q, n, k) in enumerate(LLAMA_LAYER):
            xk = x_host[:k]
            assert_matvec_close(out[0, t, :n], G.matmul_f64(q, xk, blocks[0][name], n, k),
                                G.abs_matmul_f64(q, xk, blocks[0][name], n, k), what=f"layer 0 {name}")
    finally:
        st.close()
        x.free()
        y.free()
        s.destroy()


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
