"""Host-side logic of the package that needs no GPU."""

from __future__ import annotations

import numpy as np

from flatrun_amd import _C


def bf16_round(a: np.ndarray) -> np.ndarray:
    u = np.ascontiguousarray(a, np.float32).view(np.uint32)
    r = (u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) & np.uint32(0xFFFF0000)
    return r.view(np.float32)


def test_bf16_rounding_helper():
    """The product's host-side float32 -> bf16 conversion rounds to nearest even."""
    v = np.array([1.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -2.5, 3.0e38, 1e-40, 0.0, -0.0], np.float32)
    bits = _C.to_bf16_bits(v)
    back = (bits.astype(np.uint32) << 16).view(np.float32)
    assert np.array_equal(back.view(np.uint32), bf16_round(v).view(np.uint32))
    assert back[1] == 1.0 and back[2] == 1.0 + 2 ** -6          # ties to even
    assert np.isnan((_C.to_bf16_bits(np.array([np.nan], np.float32)).astype(np.uint32) << 16).view(np.float32)[0])
