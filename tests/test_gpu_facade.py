"""The reference's native-backend test cases, run on flatrun_amd.NativeBackend.

Mirrors src/flatrun_native/tests/test_native_backend.py, test_q4_k_parity.py,
test_q6_k_parity.py and test_q8_0_parity.py case by case (shapes, seeds,
generator distributions, the reference's own tolerances), with two
differences: a missing library is an error (the reference prints "SKIP" and
returns), and the tolerance of each parity case is also checked at the
1e-5 contract. The generators reproduce the reference test distributions
(d in [0.01, 1], random 12 scale bytes < 64, Q6_K qh < 4), see
test_native_backend.py:31-63.
"""

from __future__ import annotations

import struct

import numpy as np
import pytest

from conftest import assert_rel_close_to, bits_equal
from flatrun_amd import _C, NativeBackend, is_available, is_neon, version
from oracle import gguf_np as G

pytestmark = pytest.mark.gpu


def ref_style_q4_k(seed: int, n_blocks: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    out = bytearray()
    for _ in range(n_blocks):
        out += struct.pack("<ee", float(rng.uniform(0.01, 1.0)), float(rng.uniform(0.0, 0.5)))
        out += bytes(rng.integers(0, 64, size=12, dtype=np.uint8))
        out += bytes(rng.integers(0, 16, size=128, dtype=np.uint8))
    return np.frombuffer(bytes(out), np.uint8)


def ref_style_q6_k(seed: int, n_blocks: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    out = bytearray()
    for _ in range(n_blocks):
        out += bytes(rng.integers(0, 16, size=128, dtype=np.uint8))
        out += bytes(rng.integers(0, 4, size=64, dtype=np.uint8))
        out += bytes(rng.integers(-127, 127, size=16, dtype=np.int8))
        out += struct.pack("<e", float(rng.uniform(0.01, 1.0)))
    return np.frombuffer(bytes(out), np.uint8)


def ref_style_q8_0(seed: int, n_blocks: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    out = bytearray()
    for _ in range(n_blocks):
        out += struct.pack("<e", float(rng.uniform(0.01, 1.0)))
        out += bytes(rng.integers(-127, 127, size=32, dtype=np.int8))
    return np.frombuffer(bytes(out), np.uint8)


def test_module_helpers(backend):
    assert is_available() is True
    assert is_neon() is False
    assert isinstance(version(), str) and version()
    assert backend.available and backend._neon is False


def test_dequant_q4_k_parity(backend):
    """test_q4_k_parity.py:70-95 (atol 1e-4 there; bit-exact here)."""
    raw = ref_style_q4_k(42, 16)
    exp = G.dequant_q4_k(raw, (16, 256))
    got = backend.dequant_q4k(raw, (16, 256))
    assert bits_equal(got, exp)


def test_matmul_q4_k_parity(backend):
    """test_q4_k_parity.py:98-127 (atol 1e-2 there)."""
    n, k = 32, 512
    raw = ref_style_q4_k(7, n * k // 256)
    x = np.random.default_rng(99).standard_normal(k).astype(np.float32)
    exp = G.dequant_q4_k(raw, (n, k)) @ x
    got = backend.matmul_q4k(x, raw, n, k)
    assert np.abs(exp - got).max() < 1e-2
    assert_rel_close_to(got, exp)


@pytest.mark.parametrize("q,make,k,atol", [
    ("Q4_K", ref_style_q4_k, 512, 1e-4), ("Q6_K", ref_style_q6_k, 512, 5e-2), ("Q8_0", ref_style_q8_0, 256, 5e-2)])
def test_1d_vs_2d_match(backend, q, make, k, atol):
    """test_native_backend.py:109-148."""
    n = 16
    be = 32 if q == "Q8_0" else 256
    raw = make(1, n * k // be)
    x = np.random.default_rng(2).standard_normal(k).astype(np.float32)
    m = {"Q4_K": backend.matmul_q4k, "Q6_K": backend.matmul_q6_k, "Q8_0": backend.matmul_q8_0}[q]
    out_1d, out_2d = m(x, raw, n, k), m(x.reshape(1, k), raw, n, k)
    np.testing.assert_allclose(out_1d, out_2d[0], atol=atol)
    assert bits_equal(out_1d, out_2d[0])


@pytest.mark.parametrize("q,make,k", [("Q4_K", ref_style_q4_k, 512), ("Q6_K", ref_style_q6_k, 512),
                                      ("Q8_0", ref_style_q8_0, 256)])
def test_batched_seq_3_shape(backend, q, make, k):
    """test_native_backend.py:151-190."""
    n, seq = 16, 3
    be = 32 if q == "Q8_0" else 256
    raw = make(1, n * k // be)
    x = np.random.default_rng(3).standard_normal((seq, k)).astype(np.float32)
    m = {"Q4_K": backend.matmul_q4k, "Q6_K": backend.matmul_q6_k, "Q8_0": backend.matmul_q8_0}[q]
    assert m(x, raw, n, k).shape == (seq, n)


def test_error_paths(backend):
    """test_native_backend.py:198-240."""
    raw = ref_style_q4_k(1, 32)
    with pytest.raises(ValueError):
        backend.matmul_q4k(np.zeros(513, np.float32), raw, 16, 512)
    with pytest.raises(ValueError):
        backend.matmul_q6_k(np.zeros((1, 1, 512), np.float32), ref_style_q6_k(1, 32), 16, 512)
    with pytest.raises(ValueError):
        backend.matmul_q8_0(np.float32(1.0), ref_style_q8_0(1, 128), 16, 256)
    # layout rejections surface as RuntimeError, the reference runtime's fallback trigger
    with pytest.raises(RuntimeError):
        backend.matmul_q4k(np.zeros((2, 512), np.float32), raw[:-1], 16, 512)


def test_single_vs_batched_entry(frq):
    """test_native_backend.py:248-267 (the reference compares ST vs MT)."""
    n, k = 64, 512
    raw = ref_style_q4_k(7, n * k // 256)
    x = np.random.default_rng(99).standard_normal(k).astype(np.float32)
    assert bits_equal(_C.matmul_q4_k(x.copy(), raw, n, k), _C.matmul_q4_k_batched(x.reshape(1, k), raw, n, k)[0])


@pytest.mark.parametrize("q,make,k", [("Q6_K", ref_style_q6_k, 512), ("Q8_0", ref_style_q8_0, 256)])
def test_batched_matches_python(frq, q, make, k):
    """test_native_backend.py:270-305 (atol 5e-2 there)."""
    n, seq = 16, 4
    be = 32 if q == "Q8_0" else 256
    raw = make(13, n * k // be)
    x = np.random.default_rng(31).standard_normal((seq, k)).astype(np.float32)
    exp = x @ G.DEQUANT[q](raw, (n, k)).T
    got = getattr(_C, f"matmul_{q.lower()}_batched")(x, raw, n, k)
    np.testing.assert_allclose(got, exp, atol=5e-2)
    assert_rel_close_to(got, exp)


def test_ref_style_vs_live_reference(frq, ref_C):
    """Same bytes through the reference's compiled native module."""
    n, k = 48, 1024
    raw = ref_style_q4_k(5, n * k // 256)
    x = np.random.default_rng(6).standard_normal(k).astype(np.float32)
    assert_rel_close_to(_C.matmul_q4_k(x, raw, n, k), ref_C.matmul_q4_k(x, raw, n, k))
    assert bits_equal(_C.dequant_q4_k(raw, (n, k)), ref_C.dequant_q4_k(raw, (n, k)))
