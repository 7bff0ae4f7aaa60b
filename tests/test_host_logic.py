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


def _reference_try_kernel(kernel, fallback):
    """The reference runtime's dispatch (runtime/backend.py:259-268): call the
    native kernel, recompute in NumPy on RuntimeError."""
    try:
        return kernel()
    except RuntimeError:
        return fallback()


def test_device_failures_are_not_swallowed_by_the_fallback():
    """Refused arguments (shape, size, alignment, type, no device) raise
    FrqError, a RuntimeError, so the reference falls back as it does for its
    own kernels; a HIP runtime failure raises FrqDeviceError, which the
    fallback does not catch."""
    import pytest

    from flatrun_amd import FrqDeviceError, FrqError, _lib

    for code in (_lib.ERR_INVALID, _lib.ERR_SHAPE, _lib.ERR_SIZE, _lib.ERR_UNSUPPORTED, _lib.ERR_NO_DEVICE,
                 _lib.ERR_ALIGN):
        e = _lib.error_for(code, "refused")
        assert isinstance(e, FrqError) and isinstance(e, RuntimeError) and e.code == code

        def refuse(e=e):
            raise e
        assert _reference_try_kernel(refuse, lambda: "numpy") == "numpy"
    e = _lib.error_for(_lib.ERR_HIP, "hipLaunchKernel: an illegal memory access was encountered")
    assert isinstance(e, FrqDeviceError) and not isinstance(e, RuntimeError) and e.code == _lib.ERR_HIP

    def fail():
        raise e
    with pytest.raises(FrqDeviceError, match="FRQ_ERR_HIP"):
        _reference_try_kernel(fail, lambda: "numpy")
    if _lib.load_error() is None:             # through check(), with the library's own last-error text
        with pytest.raises(FrqDeviceError):
            _lib.check(_lib.ERR_HIP)
        with pytest.raises(FrqError):
            _lib.check(_lib.ERR_SHAPE)
