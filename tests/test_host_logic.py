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


def test_group_fusable_rule():
    """frq_gemv_group_fusable is pointer and shape logic only (no device): two
    to four Q4_K (16-byte aligned) / Q6_K (4-byte aligned, even block count)
    matrices with k <= 32768 fuse; a single matrix never does, since it runs
    frq_dev_gemv's own kernel."""
    from flatrun_amd import device

    a16, a4, a2 = 0x10000, 0x10004, 0x10002
    fus = device.gemv_group_fusable
    assert not fus([("Q4_K", a16)], 4096)
    assert not fus([("Q6_K", a16)], 4096)
    assert fus([("Q4_K", a16), ("Q4_K", a16)], 4096)
    assert fus([("Q4_K", a16), ("Q4_K", a16), ("Q6_K", a4)], 4096)
    assert fus([("Q4_K", a16)] * 4, 256)
    assert not fus([("Q4_K", a16), ("Q4_K", a4)], 4096)          # Q4_K base not 16-byte aligned
    assert not fus([("Q4_K", a16), ("Q6_K", a2)], 4096)          # Q6_K base not 4-byte aligned
    assert not fus([("Q4_K", a16), ("Q6_K", a4)], 768)           # odd Q6_K block count
    assert not fus([("Q4_K", a16), ("Q5_K", a16)], 4096)         # format without a group body
    assert fus([("Q4_K", a16), ("Q4_K", a16)], 32768)
    assert not fus([("Q4_K", a16), ("Q4_K", a16)], 32768 + 256)  # row longer than one workgroup
    assert not fus([("Q4_K", a16), ("Q4_K", a16)], 300)          # k not a whole number of blocks
