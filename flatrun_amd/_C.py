"""Drop-in for the reference's pybind11 module ``flatrun_native._C``.

Same function names, argument order, argument conversion and return shapes as
``src/flatrun_native/_C.cpp:455-488``; each function calls the matching
``frq_*`` entry point of libfrq_hip.so (include/frq.h), which runs the HIP
kernels. Arguments are converted the way ``py::array_t<T, c_style |
forcecast>`` converts them (any ndim, cast to the element type, made
contiguous). Errors the reference raises as ``std::runtime_error`` arrive as
:class:`flatrun_amd._lib.FrqError`, a ``RuntimeError``. A HIP runtime failure
(a failed launch, allocation or copy) arrives as
:class:`flatrun_amd._lib.FrqDeviceError`, which is not a ``RuntimeError``, so
the reference runtime's NumPy fallback does not swallow it.

Additions beyond the reference module, for the formats it lacks:
``dequant_q5_k``, ``dequant_q1_0``, ``dequant_q4_0``, ``dequant_q5_0``,
``dequant_q5_1``, ``matmul_q5_k``, ``matmul_q1_0`` and
their ``_batched`` forms, ``dequant(qtype, weight, shape)`` with the NumPy
decoders' ragged-size rule, and ``matmul_q4_k_bf16`` (prefill GEMM on the
matrix cores, bf16 inputs; also ``matmul_q6_k_bf16``, ``matmul_q8_0_bf16``,
``matmul_bf16(qtype, ...)``).
"""

from __future__ import annotations

import operator

import numpy as np

from . import _lib
from ._lib import check, lib, ptr


def _size_t(v, what: str) -> int:
    v = operator.index(v)
    if v < 0:
        raise TypeError(f"{what} must be a non-negative integer, got {v}")
    return v


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32))


def _u8(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.uint8))


def _shape2(shape) -> tuple[int, int]:
    o, i = shape
    return int(o), int(i)


# ------------------------------------------------------------------ dequant

def dequant_q4_k(weight, shape):
    """dequant_q4_k(weight_uint8, (out, in)) -> float32 (out, in). _C.cpp:47-86."""
    w = _u8(weight)
    o, i = _shape2(shape)
    out = np.empty((max(o, 0), max(i, 0)), dtype=np.float32)
    check(lib().frq_dequant_q4_k(ptr(w), w.size, o, i, ptr(out)))
    return out


def dequant_q8_0(weight, shape):
    """dequant_q8_0(weight_uint8, (out, in)). _C.cpp:285-320."""
    w = _u8(weight)
    o, i = _shape2(shape)
    out = np.empty((max(o, 0), max(i, 0)), dtype=np.float32)
    check(lib().frq_dequant_q8_0(ptr(w), w.size, o, i, ptr(out)))
    return out


def dequant_q6_k(weight, shape):
    """dequant_q6_k(weight_uint8, (out, in)). _C.cpp:363-398."""
    w = _u8(weight)
    o, i = _shape2(shape)
    out = np.empty((max(o, 0), max(i, 0)), dtype=np.float32)
    check(lib().frq_dequant_q6_k(ptr(w), w.size, o, i, ptr(out)))
    return out


def dequant(qtype, weight, shape):
    """Any supported type, NumPy-decoder size rule (ceil-div blocks, tail
    trimmed; gguf.py:61-73). Returns float32 of ``shape``."""
    q = _lib.QTYPES[qtype.upper()] if isinstance(qtype, str) else int(qtype)
    w = _u8(weight)
    shape = tuple(int(s) for s in (shape if isinstance(shape, (tuple, list)) else (shape,)))
    n = int(np.prod(shape)) if shape else 1
    out = np.empty(n, dtype=np.float32)
    check(lib().frq_dequant(q, ptr(w), w.size, n, ptr(out)))
    return out.reshape(shape)


def dequant_q5_k(weight, shape):
    return dequant(_lib.Q5_K, weight, shape)


def dequant_q1_0(weight, shape):
    return dequant(_lib.Q1_0, weight, shape)


def dequant_q4_0(weight, shape):
    return dequant(_lib.Q4_0, weight, shape)


def dequant_q5_0(weight, shape):
    return dequant(_lib.Q5_0, weight, shape)


def dequant_q5_1(weight, shape):
    return dequant(_lib.Q5_1, weight, shape)


# ------------------------------------------------------------------ matmul

def _matmul_1d(entry, x, weight, n, k):
    xc, w = _f32(x), _u8(weight)
    n, k = _size_t(n, "n"), _size_t(k, "k")
    out = np.empty(n, dtype=np.float32)
    check(entry(ptr(xc), xc.size, ptr(w), w.size, n, k, ptr(out)))
    return out


def _matmul_2d(entry, x, weight, n, k):
    xc, w = _f32(x), _u8(weight)
    n, k = _size_t(n, "n"), _size_t(k, "k")
    seq = xc.shape[0] if xc.ndim == 2 else 0
    cols = xc.shape[1] if xc.ndim == 2 else 0
    out = np.empty((seq, n), dtype=np.float32)
    check(entry(ptr(xc), xc.ndim, seq, cols, ptr(w), w.size, n, k, ptr(out)))
    return out


def matmul_q4_k(x, weight, n, k):
    """out[n] = W . x; x has k elements. _C.cpp:99-132."""
    return _matmul_1d(lib().frq_matmul_q4_k, x, weight, n, k)


def matmul_q4_k_batched(x, weight, n, k):
    """out[seq, n] for x of shape (seq, k). _C.cpp:154-197."""
    return _matmul_2d(lib().frq_matmul_q4_k_batched, x, weight, n, k)


def matmul_q8_0(x, weight, n, k):
    """_C.cpp:326-357."""
    return _matmul_1d(lib().frq_matmul_q8_0, x, weight, n, k)


def matmul_q8_0_batched(x, weight, n, k):
    """_C.cpp:199-242."""
    return _matmul_2d(lib().frq_matmul_q8_0_batched, x, weight, n, k)


def matmul_q6_k(x, weight, n, k):
    """_C.cpp:404-435."""
    return _matmul_1d(lib().frq_matmul_q6_k, x, weight, n, k)


def matmul_q6_k_batched(x, weight, n, k):
    """_C.cpp:244-283."""
    return _matmul_2d(lib().frq_matmul_q6_k_batched, x, weight, n, k)


def _generic_1d(q: int, name: str):
    def f(x, weight, n, k):
        xc, w = _f32(x), _u8(weight)
        n, k = _size_t(n, "n"), _size_t(k, "k")
        if xc.size != k:
            raise _lib.FrqError(_lib.ERR_SHAPE, f"{name} matmul: x.size() != k")
        out = np.empty(n, dtype=np.float32)
        check(lib().frq_matmul(q, ptr(xc), 1, ptr(w), w.size, n, k, ptr(out)))
        return out
    f.__name__ = f"matmul_{name.lower()}"
    return f


def _generic_2d(q: int, name: str):
    def f(x, weight, n, k):
        xc, w = _f32(x), _u8(weight)
        n, k = _size_t(n, "n"), _size_t(k, "k")
        if xc.ndim != 2:
            raise _lib.FrqError(_lib.ERR_SHAPE, f"{name} matmul (batched): x must be 2-D (seq, k)")
        if xc.shape[1] != k:
            raise _lib.FrqError(_lib.ERR_SHAPE, f"{name} matmul (batched): x.shape[1] != k")
        out = np.empty((xc.shape[0], n), dtype=np.float32)
        check(lib().frq_matmul(q, ptr(xc), xc.shape[0], ptr(w), w.size, n, k, ptr(out)))
        return out
    f.__name__ = f"matmul_{name.lower()}_batched"
    return f


matmul_q5_k = _generic_1d(_lib.Q5_K, "Q5_K")
matmul_q5_k_batched = _generic_2d(_lib.Q5_K, "Q5_K")
matmul_q1_0 = _generic_1d(_lib.Q1_0, "Q1_0")
matmul_q1_0_batched = _generic_2d(_lib.Q1_0, "Q1_0")


# ------------------------------------------------------------------ prefill GEMM (matrix cores)

def to_bf16_bits(a) -> np.ndarray:
    """float32 -> bf16 bit patterns (uint16), round to nearest even; NaN stays
    NaN (quiet). Input preparation for the bf16 GEMM, not arithmetic on W."""
    f = np.ascontiguousarray(np.asarray(a, dtype=np.float32))
    u = f.view(np.uint32)
    r = ((u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)).astype(np.uint16)
    nan = np.isnan(f)
    if nan.any():
        r[nan] = ((u[nan] >> np.uint32(16)) | np.uint32(0x40)).astype(np.uint16)
    return r


def matmul_bf16(qtype, x, weight, n, k):
    """out[seq, n] = x[seq, k] . W^T on the matrix cores, x and W in bf16
    (x given as float32 is rounded to bf16 first; a uint16 array is taken as
    bf16 bits), fp32 accumulation; W is Q4_K, Q6_K or Q8_0. 1-D x gives
    out[n]. The fp32 per-token paths are matmul_<q>_batched (_C.cpp:154-283)."""
    xa = np.asarray(x)
    xb = np.ascontiguousarray(xa) if xa.dtype == np.uint16 else to_bf16_bits(xa)
    one_d = xb.ndim == 1
    x2 = xb.reshape(1, -1) if one_d else xb
    if x2.ndim != 2:
        raise _lib.FrqError(_lib.ERR_SHAPE, "gemm: x must be 1-D or 2-D")
    n, k = _size_t(n, "n"), _size_t(k, "k")
    if x2.shape[1] != k:
        raise _lib.FrqError(_lib.ERR_SHAPE, "gemm: x.shape[-1] != k")
    w = _u8(weight)
    q = _lib.QTYPES[qtype.upper()] if isinstance(qtype, str) else int(qtype)
    out = np.empty((x2.shape[0], n), dtype=np.float32)
    check(lib().frq_gemm_bf16(q, ptr(x2), ptr(w), w.size, x2.shape[0], n, k, ptr(out)))
    return out[0] if one_d else out


def matmul_q4_k_bf16(x, weight, n, k):
    return matmul_bf16(_lib.Q4_K, x, weight, n, k)


def matmul_q6_k_bf16(x, weight, n, k):
    return matmul_bf16(_lib.Q6_K, x, weight, n, k)


def matmul_q8_0_bf16(x, weight, n, k):
    return matmul_bf16(_lib.Q8_0, x, weight, n, k)


# ------------------------------------------------------------------ diagnostics

def is_neon() -> bool:
    """Always False (no NEON path). _C.cpp:441-447."""
    return bool(lib().frq_is_neon())


def version() -> str:
    """Build identifier. _C.cpp:449-451."""
    return _lib.version()
