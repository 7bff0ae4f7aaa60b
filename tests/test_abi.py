"""C-ABI and facade checks that need no GPU.

* libfrq_hip.so loads and exports every function include/frq.h declares.
* Validation runs before any device work and mirrors src/flatrun_native/_C.cpp:
  the same rules, the same RuntimeError type (FrqError subclasses it), and --
  where the reference module is built in oracle/_ref -- the same outcome.
* The facade mirrors src/flatrun_native/python/__init__.py: RuntimeError when
  unavailable, ValueError for a bad 1-D length or ndim, no CPU fallback.
"""

from __future__ import annotations

import ctypes
import re

import numpy as np
import pytest

from conftest import ROOT
from flatrun_amd import _C, _lib, synth

HEADER = ROOT / "include" / "frq.h"


def declared_functions() -> list[str]:
    text = HEADER.read_text()
    return sorted(set(re.findall(r"\b(frq_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _lib.lib()
    names = declared_functions()
    assert len(names) >= 40
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    assert set(names) == set(_lib.SIGNATURES), "ctypes signature table out of sync with include/frq.h"


def test_info_entry_points():
    lib = _lib.lib()
    assert lib.frq_is_neon() == 0
    assert lib.frq_version().decode().startswith("flatrun_amd")
    bb, be = ctypes.c_int64(), ctypes.c_int64()
    for q, (b, e) in _lib.BLOCKS.items():
        assert lib.frq_block_info(q, ctypes.byref(bb), ctypes.byref(be)) == _lib.OK
        assert (bb.value, be.value) == (b, e)
    assert lib.frq_block_info(3, ctypes.byref(bb), ctypes.byref(be)) == _lib.ERR_INVALID
    assert _lib.device_count() >= 0


# (function, args, error code) -- each mirrors a runtime_error branch of _C.cpp
_W16 = synth.make_blocks("Q4_K", 2, 512, seed=0)
_X = np.zeros(512, np.float32)
BAD_CALLS = [
    ("matmul_q4_k", (_X, _W16, 2, 500), _lib.ERR_SHAPE),                  # k % 256   (:105-109)
    ("matmul_q4_k", (_X[:300], _W16, 2, 512), _lib.ERR_SHAPE),            # x.size != k (:110-114)
    ("matmul_q4_k", (_X, _W16[:-1], 2, 512), _lib.ERR_SIZE),              # weight size (:116-120)
    ("matmul_q4_k_batched", (_X, _W16, 2, 512), _lib.ERR_SHAPE),          # x not 2-D (:166-170)
    ("matmul_q4_k_batched", (np.zeros((3, 256), np.float32), _W16, 2, 512), _lib.ERR_SHAPE),  # (:172-176)
    ("matmul_q8_0", (np.zeros(48, np.float32), np.zeros(34 * 3, np.uint8), 2, 48), _lib.ERR_SHAPE),   # k % 32
    ("matmul_q6_k", (_X, np.zeros(2 * 2 * 210 - 1, np.uint8), 2, 512), _lib.ERR_SIZE),
    ("dequant_q4_k", (_W16, (2, 500)), _lib.ERR_SHAPE),                   # (:54-58)
    ("dequant_q4_k", (_W16, (1, 512)), _lib.ERR_SIZE),                    # (:60-67)
    ("dequant_q6_k", (np.zeros(210, np.uint8), (1, 512)), _lib.ERR_SIZE),
    ("dequant_q8_0", (np.zeros(34, np.uint8), (1, 33)), _lib.ERR_SHAPE),
]


@pytest.mark.parametrize("fn,args,code", BAD_CALLS, ids=[f"{c[0]}-{i}" for i, c in enumerate(BAD_CALLS)])
def test_validation_mirrors_reference(fn, args, code, ref_C_optional):
    with pytest.raises(RuntimeError) as ei:
        getattr(_C, fn)(*args)
    assert isinstance(ei.value, _lib.FrqError) and ei.value.code == code
    if ref_C_optional is not None:                      # the reference rejects the same call
        with pytest.raises(RuntimeError):
            getattr(ref_C_optional, fn)(*args)


@pytest.fixture
def ref_C_optional():
    from oracle.loader import ref_C

    return ref_C()


def test_compute_without_device_reports_no_device():
    if _lib.device_count() > 0:
        pytest.skip("a device is present")
    with pytest.raises(_lib.FrqError) as ei:
        _C.matmul_q4_k(_X, _W16, 2, 512)
    assert ei.value.code == _lib.ERR_NO_DEVICE


def test_empty_shapes_need_no_device():
    out = _C.matmul_q4_k(np.zeros(0, np.float32), np.zeros(0, np.uint8), 0, 0) if _lib.device_count() == 0 else None
    if out is not None:
        assert out.shape == (0,)


# ---------------------------------------------------------------- facade

def test_facade_names_match_reference():
    import flatrun_amd as fa

    for name in ("NativeBackend", "Q4K_GEMM_BLOCK", "is_available", "is_neon", "version"):
        assert hasattr(fa, name)
    assert fa.Q4K_GEMM_BLOCK == 256
    assert fa.is_neon() is False
    assert isinstance(fa.is_available(), bool)
    assert isinstance(fa.version(), str) and fa.version()
    b = fa.NativeBackend()
    assert isinstance(b.available, bool) and b._neon is False
    for m in ("matmul_q4k", "matmul_q8_0", "matmul_q6_k", "matmul_q6k", "dequant_q4k"):
        assert callable(getattr(b, m))


def test_facade_unavailable_raises_runtime_error():
    import flatrun_amd as fa

    b = fa.NativeBackend()
    b.available = False                                 # as test_backend.py:305-323 forces it
    with pytest.raises(RuntimeError):
        b.matmul_q4k(_X, _W16, 2, 512)
    with pytest.raises(RuntimeError):
        b.dequant_q4k(_W16, (2, 512))


@pytest.mark.parametrize("method,x", [
    ("matmul_q4k", np.zeros(513, np.float32)),          # 1-D length != k
    ("matmul_q6_k", np.zeros((1, 1, 512), np.float32)),  # 3-D
    ("matmul_q8_0", np.float32(1.0)),                   # 0-D
])
def test_facade_value_errors(method, x):
    """python/__init__.py:147-153: ValueError before any kernel call."""
    import flatrun_amd as fa

    b = fa.NativeBackend()
    b.available = True                                  # force past the availability gate
    with pytest.raises(ValueError):
        getattr(b, method)(x, _W16, 2, 512)


def test_gemm_k_limit():
    """The prefill GEMM takes k up to 2^22 (its buffer offsets stay below
    2^31): one Q4_K block past it is refused as unsupported before any pointer
    or device is touched; at the limit the checks pass and the null buffers
    are what is refused."""
    lib = _lib.lib()
    n = 1
    for k, code in (((1 << 22) + 256, _lib.ERR_UNSUPPORTED), (1 << 22, _lib.ERR_INVALID)):
        w_bytes = n * (k // 256) * 144
        rc = lib.frq_dev_gemm_bf16(_lib.QTYPES["Q4_K"], None, w_bytes, None, None, 4, n, k, None)
        assert rc == code, (k, rc)


def test_gemm_group_validation():
    """frq_dev_gemm_bf16_group refuses bad groups before touching a device:
    a count outside 1..4, a weight size that does not match, a y_stride below
    a matrix's rows; an empty group (m = 0) is a no-op."""
    import ctypes

    lib = _lib.lib()
    q = (ctypes.c_int * 2)(_lib.QTYPES["Q4_K"], _lib.QTYPES["Q6_K"])
    w = (ctypes.c_void_p * 2)(None, None)
    n = (ctypes.c_int64 * 2)(256, 128)
    wb = (ctypes.c_size_t * 2)(256 * 2 * 144, 128 * 2 * 210)
    y = (ctypes.c_void_p * 2)(None, None)
    assert lib.frq_dev_gemm_bf16_group(0, q, w, wb, n, None, 4, 512, y, 0, None) == _lib.ERR_INVALID
    assert lib.frq_dev_gemm_bf16_group(5, q, w, wb, n, None, 4, 512, y, 0, None) == _lib.ERR_INVALID
    bad = (ctypes.c_size_t * 2)(256 * 2 * 144, 128 * 2 * 210 - 1)
    assert lib.frq_dev_gemm_bf16_group(2, q, w, bad, n, None, 4, 512, y, 0, None) == _lib.ERR_SIZE
    assert lib.frq_dev_gemm_bf16_group(2, q, w, wb, n, None, 4, 512, y, 200, None) == _lib.ERR_SHAPE
    assert lib.frq_dev_gemm_bf16_group(2, q, w, wb, n, None, 0, 512, y, 0, None) == _lib.OK
