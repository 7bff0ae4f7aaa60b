"""GPU dequant kernels: bit-exact against the oracle (oracle/gguf_np.py).

Bit-exact means equal fp32 bit patterns (NaN compared as NaN for the non-
finite-scale case). Covers every format, ragged sizes, the reference KATs,
hand-built layout blocks, fp16 edge scales, the committed reference vectors
and the device-pointer entry point.
"""

from __future__ import annotations

import numpy as np
import pytest

from conftest import GOLDEN, bits_equal
from flatrun_amd import _C, _lib, synth
from oracle import gguf_np as G

pytestmark = pytest.mark.gpu

QS = ["Q8_0", "Q4_K", "Q5_K", "Q6_K", "Q1_0", "Q4_0", "Q5_0", "Q5_1"]


def gpu_dequant(q, raw, shape):
    return _C.dequant(q, raw, shape)


@pytest.mark.parametrize("q", QS)
@pytest.mark.parametrize("n,k,seed", [(1, 256, 0), (7, 512, 1), (64, 1024, 2), (300, 3584, 3)])
def test_dequant_random_blocks(frq, q, n, k, seed):
    raw = synth.make_blocks(q, n, k, seed=seed)
    assert bits_equal(gpu_dequant(q, raw, (n, k)), G.DEQUANT[q](raw, (n, k)))


@pytest.mark.parametrize("q", QS)
@pytest.mark.parametrize("nel", [1, 3, 31, 33, 129, 255, 257, 1000, 4097])
def test_dequant_ragged_sizes(frq, q, nel):
    bb, be = synth.BLOCK[q]
    nblk = -(-nel // be)
    raw = synth.make_blocks(q, 1, nblk * be, seed=nel)
    assert bits_equal(gpu_dequant(q, raw, (nel,)), G.DEQUANT[q](raw, (nel,)))


@pytest.mark.parametrize("q", QS)
def test_dequant_empty(frq, q):
    out = gpu_dequant(q, np.zeros(0, np.uint8), (0,))
    assert out.shape == (0,)


@pytest.mark.parametrize("q", QS)
def test_dequant_fp16_edge_scales(frq, q):
    """Subnormal, negative, max, zero and non-finite fp16 scales."""
    bb, be = synth.BLOCK[q]
    edge = np.array([0x0001, 0x03FF, 0x8200, 0x7BFF, 0xFBFF, 0x0000, 0x8000, 0x3C00, 0x7C00, 0xFE00],
                    dtype=np.uint16)
    raw = synth.make_blocks(q, 1, len(edge) * be, seed=5).reshape(-1, bb)
    offs = {"Q8_0": [0], "Q4_K": [0, 2], "Q5_K": [0, 2], "Q6_K": [208], "Q1_0": [0], "Q4_0": [0], "Q5_0": [0],
            "Q5_1": [0, 2]}[q]
    for i, h in enumerate(edge):
        for o in offs:
            raw[i, o], raw[i, o + 1] = h & 0xFF, h >> 8
    raw = raw.reshape(-1)
    got = gpu_dequant(q, raw, (len(edge) * be,))
    exp = G.DEQUANT[q](raw, (len(edge) * be,))
    fin = np.isfinite(exp)
    assert bits_equal(got[fin], exp[fin])
    assert np.array_equal(np.isnan(got), np.isnan(exp))
    assert np.array_equal(got[np.isinf(exp)], exp[np.isinf(exp)])


def test_reference_kats_on_gpu(frq):
    """The KATs of src/flatrun/tests/test_dequant.py on the HIP kernels."""
    from test_oracle_kats import (kat_q1_0_pattern, kat_q4_0_nibble_order, kat_q5_0_all_high_bits, kat_q5_1_offset,
                                  kat_q6_k_qh_pairs, kat_q8_0_simple, kat_q8_0_two_blocks)

    for q, make in (("Q8_0", kat_q8_0_simple), ("Q8_0", kat_q8_0_two_blocks), ("Q1_0", kat_q1_0_pattern),
                    ("Q4_0", kat_q4_0_nibble_order), ("Q5_0", kat_q5_0_all_high_bits), ("Q5_1", kat_q5_1_offset)):
        raw, shape, exp = make()
        assert np.array_equal(gpu_dequant(q, np.frombuffer(raw, np.uint8), shape), exp)
    raw, shape, _ = kat_q6_k_qh_pairs()
    out = gpu_dequant("Q6_K", np.frombuffer(raw, np.uint8), shape)
    assert int((out == -16.0).sum()) == 128 and int((out == -15.0).sum()) == 128 and out.sum() == -3968.0
    for q, nb in (("Q4_K", 144), ("Q5_K", 176), ("Q6_K", 210), ("Q1_0", 18)):
        nel = 128 if q == "Q1_0" else 256
        assert np.all(gpu_dequant(q, np.zeros(nb, np.uint8), (nel,)) == 0)
    raw = np.frombuffer((np.float16(0.5).tobytes() + bytes(16)) * 2, np.uint8)
    assert np.array_equal(gpu_dequant("Q1_0", raw, (130,))[128:], np.array([-0.5, -0.5], np.float32))


def test_hand_built_layout_blocks_on_gpu(frq):
    import test_oracle_pins as P

    for d, dm in ((1.0, 0.0), (0.0, 1.0), (0.5, 0.25)):
        raw, exp = P._q4k_order_block(d, dm)
        assert bits_equal(gpu_dequant("Q4_K", np.frombuffer(raw, np.uint8), (256,)), exp.astype(np.float32))


def test_reference_native_vectors_on_gpu(frq):
    z = np.load(GOLDEN / "ref_native_vectors.npz")
    for q in ("Q4_K", "Q6_K", "Q8_0"):
        t = q.lower()
        n, k = z[f"{t}_shape"]
        assert bits_equal(getattr(_C, f"dequant_{t}")(z[f"{t}_raw"], (n, k)), z[f"{t}_dequant"])


def test_q5_k_reference_vectors_on_gpu(frq):
    z = np.load(GOLDEN / "q5k_ref_vectors.npz")
    for name in ("random", "wide", "subnormal"):
        out = z[f"{name}_out"]
        assert bits_equal(gpu_dequant("Q5_K", z[f"{name}_raw"], (out.size,)), out)
    assert bits_equal(gpu_dequant("Q5_K", z["ragged_raw"], (700,)), z["ragged_out"])


@pytest.mark.parametrize("q", QS)
def test_device_entry_point(frq, q):
    from flatrun_amd import device

    n, k = 96, 2048 if q != "Q8_0" else 1024
    raw = synth.make_blocks(q, n, k, seed=21)
    w = device.DeviceBuffer.from_host(raw)
    y = device.DeviceBuffer(n * k * 4)
    device.dequant(q, w, y, n * k)
    device.synchronize()
    assert bits_equal(y.to_host(np.float32).reshape(n, k), G.DEQUANT[q](raw, (n, k)))
