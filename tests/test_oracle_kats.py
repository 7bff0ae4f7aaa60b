"""The reference's known-answer tests, run against the oracle.

Each test restates one KAT of src/flatrun/tests/test_dequant.py (line numbers
cited) on the NumPy oracle (oracle/gguf_np.py); where the C restatement
(oracle/native_ref.c) covers the format, it is checked too. The same KATs run
on the GPU kernels in tests/test_gpu_dequant.py.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import gguf_np as G
from oracle.loader import c_oracle

F32 = np.float32


def kat_q8_0_simple():
    raw = bytearray(np.float16(0.5).tobytes())
    qs = np.array([-2, 4, 0, 8, -3, 1, 2, 3, -1, -4, 5, 6, 7, -8, 9, 0] * 2, dtype=np.int8)
    raw += qs.tobytes()
    return bytes(raw), (32,), qs.astype(F32) * F32(0.5)


def kat_q8_0_two_blocks():
    raw = bytearray()
    for s in (0.25, 0.75):
        raw += np.float16(s).tobytes() + np.full(32, 4, dtype=np.int8).tobytes()
    return bytes(raw), (64,), np.concatenate([np.full(32, 1.0, F32), np.full(32, 3.0, F32)])


def kat_q1_0_pattern():
    raw = bytearray(np.float16(0.5).tobytes())
    for i in range(16):
        raw.append(0xAA if i % 2 == 0 else 0x01)
    exp = np.tile(np.array([-0.5, 0.5, -0.5, 0.5, -0.5, 0.5, -0.5, 0.5,
                            0.5, -0.5, -0.5, -0.5, -0.5, -0.5, -0.5, -0.5], F32), 8)
    return bytes(raw), (128,), exp


def kat_q6_k_qh_pairs():
    raw = (np.full(128, 0x10, np.uint8).tobytes() + np.full(64, 0x55, np.uint8).tobytes()
           + np.full(16, 1, np.int8).tobytes() + np.float16(1.0).tobytes())
    return raw, (256,), None


def kat_q4_0_nibble_order():
    raw = np.float16(0.5).tobytes() + np.full(16, 0xF7, np.uint8).tobytes()
    return raw, (32,), np.concatenate([np.full(16, -0.5, F32), np.full(16, 3.5, F32)])


def kat_q5_0_all_high_bits():
    raw = np.float16(0.25).tobytes() + np.uint32(0xFFFFFFFF).tobytes() + np.zeros(16, np.uint8).tobytes()
    return raw, (32,), np.zeros(32, F32)


def kat_q5_1_offset():
    raw = (np.float16(0.5).tobytes() + np.float16(1.0).tobytes() + np.uint32(0).tobytes()
           + np.full(16, 0x55, np.uint8).tobytes())
    return raw, (32,), np.full(32, 5 * 0.5 + 1.0, F32)


KATS = {
    "q4_0_nibble_order": ("Q4_0", kat_q4_0_nibble_order),   # test_dequant.py:60-72
    "q5_0_all_high_bits": ("Q5_0", kat_q5_0_all_high_bits),  # test_dequant.py:212-224
    "q5_1_offset": ("Q5_1", kat_q5_1_offset),                # test_dequant.py:227-238
    "q8_0_simple": ("Q8_0", kat_q8_0_simple),          # test_dequant.py:32-42
    "q8_0_two_blocks": ("Q8_0", kat_q8_0_two_blocks),  # test_dequant.py:45-57
    "q1_0_pattern": ("Q1_0", kat_q1_0_pattern),        # test_dequant.py:297-317 (and :274-294)
}


@pytest.mark.parametrize("name", sorted(KATS))
def test_reference_kat_exact(name):
    q, make = KATS[name]
    raw, shape, exp = make()
    out = G.DEQUANT[q](raw, shape)
    assert out.shape == shape
    assert np.array_equal(out, exp)       # the reference asserts rtol 1e-4/1e-5; exact holds


def test_q8_0_kat_c_restatement():
    raw, shape, exp = kat_q8_0_simple()
    out = c_oracle().dequant("Q8_0", np.frombuffer(raw, np.uint8), 32)
    assert np.array_equal(out, exp)


def test_q4_k_finite_block():
    """test_dequant.py:188-197."""
    raw = (np.float16(0.1).tobytes() + np.float16(0.01).tobytes()
           + np.zeros(12, np.uint8).tobytes() + np.zeros(128, np.uint8).tobytes())
    out = G.dequant_q4_k(raw, (256,))
    assert out.shape == (256,) and np.all(np.isfinite(out))


@pytest.mark.parametrize("q,nbytes", [("Q4_K", 144), ("Q5_K", 176), ("Q6_K", 210), ("Q1_0", 18)])
def test_zero_blocks(q, nbytes):
    """test_dequant.py:240-271 (Q4_K/Q5_K/Q6_K zero blocks) and :320-326 (Q1_0 d=0)."""
    nel = 128 if q == "Q1_0" else 256
    out = G.DEQUANT[q](bytes(nbytes), (nel,))
    assert np.all(out == 0.0)


def test_q1_0_ragged_tail():
    """test_dequant.py:329-341: 130 elements -> 2 blocks, tail bits 0 -> -d."""
    raw = (np.float16(0.5).tobytes() + bytes(16)) * 2
    out = G.dequant_q1_0(raw, (130,))
    assert out.shape == (130,)
    assert np.array_equal(out[128:], np.array([-0.5, -0.5], F32))


def test_q6_k_qh_pair_kat():
    """Orphaned KAT at test_dequant.py:342-372: ql=0x10, qh=0x55, scales=1, d=1
    -> 128 values of -16 and 128 of -15, sum -3968."""
    raw, shape, _ = kat_q6_k_qh_pairs()
    out = G.dequant_q6_k(raw, shape)
    assert int((out == -16.0).sum()) == 128
    assert int((out == -15.0).sum()) == 128
    assert float(out.sum()) == -3968.0
    cout = c_oracle().dequant("Q6_K", np.frombuffer(raw, np.uint8), 256)
    assert np.array_equal(out, cout)
